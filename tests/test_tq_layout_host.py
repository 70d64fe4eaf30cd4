"""Host checks of the TurboQuant page layout and of the host-side bin buffers.

* vramancer_amd/csrc/vrm_tq_layout.h, compiled here with g++: for padded
  dims 64 and 128 and 2, 3 and 4 bits, slot_of places the pd - 1 angles of
  the reference's level-major order (level l holds pd / 2 >> l angles) on
  distinct (quarter, slot) pairs, bin_index_of inverts it, and the one
  unused slot (quarter 3, last slot) reads as -1.  Independently of those
  two functions' formulas: each quarter's slots hold angles of the subtree
  over its own dims, the spare slots hold the top two levels, the grouped
  2/3-bit order puts each level-1 / level-3 angle's two children right after
  it, and the 4-bit order matches its plain statement (per quarter, the
  quarter's top level down to 0, each level's angles in order).
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
extern "C" int layout_errors(int pd, int bits) {
  int bad = 0;
  const int Q = quarter_slots(pd);
  int seen[4][32] = {};
  for (int l = 0; l < log2_pd(pd); ++l)
    for (int i = 0; i < ((pd / 2) >> l); ++i) {
      int g = -1, s = -1;
      slot_of(pd, l, i, bits, g, s);
      if (g < 0 || g > 3 || s < 0 || s >= Q) { ++bad; continue; }
      if (seen[g][s]++) ++bad;
      if (bin_index_of(pd, g, s, bits) != level_offset(pd, l) + i) ++bad;
    }
  for (int g = 0; g < 4; ++g)
    for (int s = 0; s < Q; ++s)
      if (!seen[g][s] && (g != 3 || s != Q - 1 || bin_index_of(pd, g, s, bits) != -1)) ++bad;
  return bad;
}
// Level-major bin -> (level, index within the level).
static void level_of(int pd, int bin, int& l, int& i) {
  l = 0;
  while (bin >= level_offset(pd, l + 1)) ++l;
  i = bin - level_offset(pd, l);
}
// bits <= 3: the slot after a level-1 or level-3 angle holds its first child
// (index 2 i of the level below), the next one its second; every level-0 and
// level-2 angle is such a child.
extern "C" int grouped_errors(int pd, int bits) {
  int bad = 0, children = 0;
  const int Q = quarter_slots(pd);
  for (int g = 0; g < 4; ++g)
    for (int s = 0; s < Q - 1; ++s) {
      int l, i;
      level_of(pd, bin_index_of(pd, g, s, bits), l, i);
      if (l != 1 && l != 3) continue;
      for (int c = 0; c < 2; ++c) {
        int lc, ic;
        level_of(pd, bin_index_of(pd, g, s + 1 + c, bits), lc, ic);
        if (lc != l - 1 || ic != 2 * i + c) ++bad;
        ++children;
      }
    }
  // level-0 and level-2 angles per record: pd / 2 and pd / 8
  return children == pd / 2 + pd / 8 ? bad : bad + 1000;
}
// The spare slot: root angle in quarter 0, the next level's two angles in
// quarters 1 and 2; every other slot of quarter g lies in the subtree over
// dims Q g .. Q g + Q - 1 (angle i of level l covers dims 2^(l+1) i ..).
extern "C" int subtree_errors(int pd, int bits) {
  int bad = 0;
  const int Q = quarter_slots(pd), top = log2_pd(pd) - 1;
  for (int g = 0; g < 4; ++g)
    for (int s = 0; s < Q; ++s) {
      const int b = bin_index_of(pd, g, s, bits);
      if (b < 0) continue;
      int l, i;
      level_of(pd, b, l, i);
      if (s == Q - 1) {
        if (g == 0 && (l != top || i != 0)) ++bad;
        if (g > 0 && (l != top - 1 || i != g - 1)) ++bad;
      } else if (((i << (l + 1)) / Q) != g) {
        ++bad;
      }
    }
  return bad;
}
extern "C" int four_bit_order_errors(int pd) {
  int bad = 0;
  const int lq = quarter_top(pd);
  for (int g = 0; g < 4; ++g) {
    int s = 0;
    for (int l = lq; l >= 0; --l)
      for (int a = 0; a < (1 << (lq - l)); ++a, ++s)
        if (bin_index_of(pd, g, s, 4) != level_offset(pd, l) + g * (1 << (lq - l)) + a) ++bad;
  }
  return bad;
}
extern "C" int sizes(int pd, int bits, int which) {
  switch (which) {
    case 0: return slice_bytes(pd, bits);
    case 1: return angle_bytes(pd, bits);
    default: return tuned_pd(pd, bits, pd / 2, 16);
  }
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


@pytest.mark.parametrize("pd", [64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_slots_cover_every_angle_once(layout_lib, pd, bits):
    assert layout_lib.layout_errors(pd, bits) == 0
    assert layout_lib.subtree_errors(pd, bits) == 0


@pytest.mark.parametrize("pd", [64, 128])
@pytest.mark.parametrize("bits", [2, 3])
def test_grouped_slots_put_children_after_their_node(layout_lib, pd, bits):
    assert layout_lib.grouped_errors(pd, bits) == 0


@pytest.mark.parametrize("pd", [64, 128])
def test_four_bit_slots_in_level_order(layout_lib, pd):
    assert layout_lib.four_bit_order_errors(pd) == 0


@pytest.mark.parametrize("pd", [64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_tuned_slice_sizes(layout_lib, pd, bits):
    # (pd - 1) angles + 1 padding slot per token, pd / 2 sign bits, 2 fp16
    assert layout_lib.sizes(pd, bits, 1) * 8 == pd * bits
    assert layout_lib.sizes(pd, bits, 0) == 16 * (pd * bits // 8 + pd // 16 + 4)
    assert layout_lib.sizes(pd, bits, 2) == pd


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
