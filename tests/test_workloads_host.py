"""Host checks of the synthetic benchmark inputs (vramancer_amd/workloads.py).

* q4_quantize writes the reference's 4-bit layout (byte j of a row holds
  dims 2j in the low nibble and 2j + 1 in the high one; one float16 scale
  and zero per 32 dims), checked on a row whose codes are known, and its
  codes reconstruct every input within half a quantisation step.
* Algorithmic bytes of the Q4 workload count 64 B of codes and 16 B of
  scales and zeros per token, kv-head and K/V side.
* bench.py refuses more than one GPU with a message and exit status 2, and
  lists its workloads and modes in --help.
"""
import os
import subprocess
import sys

import torch

from oracle import paged_decode as PD
from vramancer_amd import workloads as W


def test_q4_layout_on_a_known_row():
    # group g holds the values g*32 .. g*32 + 31 mapped onto 0 .. 15 twice:
    # min 0, max 15 -> scale 1, zero 0, nibble = value
    x = torch.tensor([float(d % 16) for d in range(128)])[None]
    codes, sc, zp = W.q4_quantize(x)
    assert codes.shape == (1, 64) and sc.shape == (1, 4) and zp.shape == (1, 4)
    assert torch.equal(sc, torch.ones(1, 4, dtype=torch.float16)) and torch.equal(zp, torch.zeros(1, 4, dtype=torch.float16))
    for j in range(64):
        lo, hi = (2 * j) % 16, (2 * j + 1) % 16
        assert int(codes[0, j]) == lo | (hi << 4), j


def test_q4_reconstruction_within_half_a_step():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 8, 16, 128, generator=g) * 3
    codes, sc, zp = W.q4_quantize(x)
    # dequantised by the oracle's own routine (the reference's formula)
    vals = PD.dequant_q4_page(codes, sc, zp)
    step = sc.float().repeat_interleave(32, dim=-1)
    # the scale and zero are float16, so allow their rounding on top of half a step
    assert ((vals.float() - x).abs() <= 0.5 * step + 2e-3 * (x.abs() + 1)).all()


def test_q4_algorithmic_bytes():
    ab = W.algorithmic_bytes(W.CONFIGS["14b-q4"], [4096] * 64)
    tokens = 64 * 4096
    assert ab["kv"] == tokens * 8 * 2 * 64
    assert ab["scales"] == tokens * 8 * 2 * 4 * 2 * 2
    assert ab["total"] == ab["kv"] + ab["scales"] + ab["qo"] + ab["table"]


ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_bench_help_lists_workloads_and_modes():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 0
    for word in ("14b-q4", "14b-turbo3", "mixed-fp8", "--batcher", "--codecs", "--hf-cache"):
        assert word in r.stdout, word
