"""Builds libvrm_paged.so (the gfx950 kernels and their C ABI) in-tree.

Each ``csrc/*.hip`` file is compiled to an object with ``hipcc
--offload-arch=gfx950`` in parallel, then linked into
``vramancer_amd/libvrm_paged.so`` next to this file.  Packed FP32 VALU
instructions are disabled for every device compilation.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from typing import List, Optional

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")
LIB_NAME = "libvrm_paged.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("VRM_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in VGPRs: the decode rescales them with VALU ops
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE_DIR}",
]


# Flags of single sources, on top of COMMON_FLAGS.
FILE_FLAGS = {
    # Machine LICM hoists lane addresses and literal constants out of the
    # shared-items kernel's loop over work items, where they stay live across
    # the whole decode and push it into spills; without it the kernel fits
    # 168 VGPRs with no scratch, and the other stream kernels of the file run
    # as fast or faster (c5 -5 us, head_dim 64 -2 us, bf16 unchanged).
    "vrm_decode_mfma.hip": ["-mllvm", "-disable-machine-licm"],
}


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def sources() -> List[str]:
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def _filter_noise(text: str) -> str:
    # The host pass does not know the gfx950-only feature name; that warning is expected.
    keep = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
    return "\n".join(keep)


def build(verbose: bool = False, out: Optional[str] = None) -> str:
    """Compiles every HIP source and links the shared library; returns its path."""
    hipcc = hipcc_path()
    out = out or LIB_PATH
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="vrm_build_") as tmp:
        procs = []
        objs = []
        for src in srcs:
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            objs.append(obj)
            cmd = [hipcc, *COMMON_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        failed = []
        for src, p in procs:
            log, _ = p.communicate()
            log = _filter_noise(log)
            if p.returncode != 0:
                failed.append((src, log))
            elif verbose and log.strip():
                print(log, flush=True)
        if failed:
            msg = "\n".join(f"--- {s}\n{l}" for s, l in failed)
            raise RuntimeError(f"hipcc failed:\n{msg}")
        tmp_out = out + ".tmp"
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_out]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{_filter_noise(r.stdout)}")
        os.replace(tmp_out, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
