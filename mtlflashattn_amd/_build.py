"""Ahead-of-time build of the HIP kernel library (gfx950 code objects).

The reference JIT-compiles Metal source strings at first use
(metal_flash_attn/_kernel.py:792-925, `torch.mps.compile_shader`).  Here the
kernels are compiled once, in-tree, into `mtlflashattn_amd/_lib/libmtlfa_hip.so`
with hipcc; nothing is compiled at run time.

Usage: python -m mtlflashattn_amd._build
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
# (source, extra flags): the backward kernels keep their MFMA accumulators in
# ordinary VGPRs (their accumulators outnumber the AGPR share the compiler
# picks, which otherwise moves them between register files every block)
SRCS = [
    (os.path.join(PKG_DIR, "csrc", "mfa_fwd.hip"), []),
    (os.path.join(PKG_DIR, "csrc", "mfa_bwd.hip"), ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]),
]
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libmtlfa_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # keep the compiler from forming packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc_path() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("mtlflashattn_amd: hipcc not found (ROCm toolchain required to build)")


def build(verbose: bool = False) -> str:
    """Compile the kernel library; returns its path.  Always recompiles."""
    os.makedirs(LIB_DIR, exist_ok=True)
    hipcc = hipcc_path()
    objs, procs = [], []
    for src, extra in SRCS:  # the sources compile in parallel
        obj = os.path.join(LIB_DIR, os.path.basename(src) + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        objs.append(obj)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    for pr in procs:
        _, err = pr.communicate()
        if pr.returncode != 0:
            raise RuntimeError(f"mtlflashattn_amd: hipcc failed ({pr.returncode}):\n{err[-4000:]}")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    for obj in objs:
        os.remove(obj)
    if res.returncode != 0:
        raise RuntimeError(f"mtlflashattn_amd: link failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
