"""Host checks of the TurboQuant page layout and of the host-side bin buffers.

* vramancer_amd/csrc/vrm_tq_layout.h, compiled here with g++: for 2, 3 and 4
  bits, slot_of places the 127 angles of the reference's level-major order
  (level l holds 64 >> l angles) on distinct (quarter, slot) pairs,
  bin_index_of inverts it, and the one unused slot (quarter 3, slot 31)
  reads as -1.  The 4-bit order is also checked against its plain statement:
  per quarter, level 4, then 3, 2, 1, 0, each level's angles in order.
* level_bins returns the compressor's own [N, 127] buffer for the per-level
  views compress returns, and a concatenated copy for any other list.
"""
import ctypes
import os
import subprocess

import pytest
import torch

from vramancer_amd.turboquant_cuda import _split_levels, level_bins

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
CSRC = os.path.join(ROOT, "vramancer_amd", "csrc")

SRC = r"""
#define __host__
#define __device__
#include "vrm_tq_layout.h"
using namespace vrm::tq;
extern "C" int layout_errors(int bits) {
  int bad = 0;
  int seen[4][32] = {};
  for (int l = 0; l < kLevels; ++l)
    for (int i = 0; i < (64 >> l); ++i) {
      int g = -1, s = -1;
      slot_of(l, i, bits, g, s);
      if (g < 0 || g > 3 || s < 0 || s > 31) { ++bad; continue; }
      if (seen[g][s]++) ++bad;
      if (bin_index_of(g, s, bits) != level_offset(l) + i) ++bad;
    }
  for (int g = 0; g < 4; ++g)
    for (int s = 0; s < 32; ++s)
      if (!seen[g][s] && (g != 3 || s != 31 || bin_index_of(g, s, bits) != -1)) ++bad;
  return bad;
}
extern "C" int four_bit_order_errors() {
  int bad = 0;
  for (int g = 0; g < 4; ++g) {
    int s = 0;
    for (int l = 4; l >= 0; --l)
      for (int a = 0; a < (1 << (4 - l)); ++a, ++s)
        if (bin_index_of(g, s, 4) != level_offset(l) + g * (1 << (4 - l)) + a) ++bad;
  }
  return bad;
}
"""


@pytest.fixture(scope="module")
def layout_lib(tmp_path_factory):
    d = tmp_path_factory.mktemp("tq_layout")
    src = d / "layout.cpp"
    src.write_text(SRC)
    so = d / "layout.so"
    subprocess.run(["g++", "-std=c++17", "-O1", "-shared", "-fPIC", f"-I{CSRC}", str(src), "-o", str(so)],
                   check=True)
    return ctypes.CDLL(str(so))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_slots_cover_every_angle_once(layout_lib, bits):
    assert layout_lib.layout_errors(bits) == 0


def test_four_bit_slots_in_level_order(layout_lib):
    assert layout_lib.four_bit_order_errors() == 0


def test_level_bins_reuses_the_compressor_buffer():
    angles = torch.randint(0, 8, (37, 127), dtype=torch.uint8)
    views = _split_levels(angles, 128, 7)
    got = level_bins(views, 127)
    assert got.data_ptr() == angles.data_ptr() and got.shape == (37, 127) and got.is_contiguous()
    assert torch.equal(got, angles)


def test_level_bins_copies_other_lists():
    angles = torch.randint(0, 8, (37, 127), dtype=torch.uint8)
    levels = [t.clone() for t in _split_levels(angles, 128, 7)]  # separate allocations
    got = level_bins(levels, 127)
    assert got.data_ptr() != angles.data_ptr() and torch.equal(got, angles)
    shuffled = _split_levels(angles, 128, 7)
    shuffled[0], shuffled[1] = shuffled[1], shuffled[0]  # right widths in the wrong order
    want = torch.cat(shuffled, -1)
    assert torch.equal(level_bins(shuffled, 127), want)
    wide = [t.to(torch.int64) for t in _split_levels(angles, 128, 7)]  # another dtype
    assert torch.equal(level_bins(wide, 127), angles)
