"""Host checks of the numerics headers shared with the gfx950 kernels.

vramancer_amd/csrc/vrm_fdlibm_atan2f.h must reproduce the C library's float
atan2 (what PyTorch's CPU kernel calls on the reference's strided views) and
vramancer_amd/csrc/vrm_e4m3.h must reproduce torch's float8_e4m3fn cast.
Both headers are compiled here with g++ (no FP contraction, as on the GPU).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
CSRC = os.path.join(ROOT, "vramancer_amd", "csrc")

SRC = r"""
#include "vrm_fdlibm_atan2f.h"
#include "vrm_e4m3.h"
#include <math.h>
#include <stdint.h>
extern "C" long atan2_mismatches(long n, uint64_t seed, int mode) {
  uint64_t s = seed * 6364136223846793005ull + 1442695040888963407ull;
  auto next = [&]() { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; };
  long bad = 0;
  for (long i = 0; i < n; ++i) {
    float y, x;
    if (mode == 0) {  // random bit patterns
      y = vrm_fdlibm::bitsf((uint32_t)next()); x = vrm_fdlibm::bitsf((uint32_t)next());
    } else {          // moderate magnitudes with random signs and exponents in [-20, 20]
      uint32_t r = (uint32_t)next(), q = (uint32_t)next();
      y = ldexpf(1.0f + (r & 0xffffff) / 16777216.0f, (int)(r >> 26) % 21 - 10) * ((r >> 25) & 1 ? -1.f : 1.f);
      x = ldexpf(1.0f + (q & 0xffffff) / 16777216.0f, (int)(q >> 26) % 21 - 10) * ((q >> 25) & 1 ? -1.f : 1.f);
    }
    float a = vrm_fdlibm::atan2f(y, x), b = ::atan2f(y, x);
    if (vrm_fdlibm::fbits(a) != vrm_fdlibm::fbits(b) && !(isnan(a) && isnan(b))) ++bad;
  }
  return bad;
}
extern "C" float atan2_one(float y, float x) { return vrm_fdlibm::atan2f(y, x); }
extern "C" void e4m3_encode(const float* x, uint8_t* y, long n) { for (long i = 0; i < n; ++i) y[i] = vrm_e4m3::encode(x[i]); }
extern "C" void e4m3_decode(const uint8_t* x, float* y, long n) { for (long i = 0; i < n; ++i) y[i] = vrm_e4m3::decode(x[i]); }
"""


@pytest.fixture(scope="module")
def hostlib(tmp_path_factory):
    d = tmp_path_factory.mktemp("hostnum")
    src = d / "hostnum.cpp"
    src.write_text(SRC)
    so = d / "hostnum.so"
    subprocess.check_call(["g++", "-O2", "-ffp-contract=off", "-Wno-unknown-pragmas", "-shared", "-fPIC",
                           f"-I{CSRC}", str(src), "-o", str(so), "-lm"])
    lib = ctypes.CDLL(str(so))
    lib.atan2_mismatches.restype = ctypes.c_long
    lib.atan2_mismatches.argtypes = [ctypes.c_long, ctypes.c_uint64, ctypes.c_int]
    lib.atan2_one.restype = ctypes.c_float
    lib.atan2_one.argtypes = [ctypes.c_float, ctypes.c_float]
    return lib


@pytest.mark.parametrize("mode", [0, 1])
def test_fdlibm_atan2f_matches_libm(hostlib, mode):
    assert hostlib.atan2_mismatches(4_000_000, 12345 + mode, mode) == 0


def test_fdlibm_atan2f_matches_torch_strided_atan2(hostlib):
    # torch's CPU atan2 on the reference's strided pair views is the libm routine
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, 2, generator=g)
    t = torch.atan2(x[:, 1], x[:, 0])
    mine = torch.tensor([hostlib.atan2_one(float(b), float(a)) for a, b in x.tolist()])
    assert torch.equal(t, mine)


def test_fdlibm_atan2f_special_values(hostlib):
    sp = [0.0, -0.0, 1.0, -1.0, float("inf"), -float("inf"), 1e-40, -1e-40, 3.4e38, 1.17e-38]
    libm = ctypes.CDLL("libm.so.6")
    libm.atan2f.restype = ctypes.c_float
    libm.atan2f.argtypes = [ctypes.c_float, ctypes.c_float]
    for y in sp:
        for x in sp:
            a, b = hostlib.atan2_one(y, x), libm.atan2f(y, x)
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (y, x)


def test_e4m3_encode_matches_torch_cast(hostlib):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    # add every float in [0, 512) on a fine grid, both signs
    grid = np.arange(0, 512, 1 / 4096, dtype=np.float32)
    f = np.concatenate([bits.view(np.float32), grid, -grid])
    f = f[~np.isnan(f)]
    mine = np.empty(f.size, np.uint8)
    hostlib.e4m3_encode(f.ctypes.data_as(ctypes.c_void_p), mine.ctypes.data_as(ctypes.c_void_p),
                        ctypes.c_long(f.size))
    ref = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_e4m3_decode_all_codes(hostlib):
    codes = np.arange(256, dtype=np.uint8)
    out = np.empty(256, np.float32)
    hostlib.e4m3_decode(codes.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p),
                        ctypes.c_long(256))
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(out[~nan], ref[~nan]) and np.isnan(out[nan]).all()
