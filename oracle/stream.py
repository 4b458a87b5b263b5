"""ORACLE -- test infrastructure only, never product code.

ctypes wrapper of oracle/stream_ref.c, the float64 two-pass restatement of
the reference's scalar kernel math (metal_flash_attn/_kernel.py:32-87).
Builds the shared object with gcc on first use if it is missing.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import torch

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "_build", "liboracle_stream.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        lib.oracle_stream_fwd.restype = I
        lib.oracle_stream_fwd.argtypes = [P, P, P, P, I, I, I, I, I, I, I, ctypes.c_double, ctypes.c_double,
                                          I, I, P, P]
        _lib = lib
    return _lib


def stream_fwd(q, k, v, scale, causal, softcap=0.0, window_left=-1, window_right=-1, alibi=None,
               return_lse=False):
    """Heads-second q [B,Hq,Lq,D], k/v [B,Hkv,Lk,D] -> float64 [B,Hq,Lq,D].

    Inputs are read as fp32 (bf16/fp16 inputs convert exactly); `alibi` is the
    broadcast [B*Hq] slope vector or None.  return_lse=True: (out, float64
    [B,Hq,Lq] log of the softmax normaliser, -inf for rows with no key).
    """
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    qc = q.detach().cpu().float().contiguous()
    kc = k.detach().cpu().float().contiguous()
    vc = v.detach().cpu().float().contiguous()
    out = torch.empty(B, Hq, Lq, D, dtype=torch.float64)
    lse = torch.empty(B, Hq, Lq, dtype=torch.float64) if return_lse else None
    al = None
    if alibi is not None:
        al = alibi.detach().cpu().float().contiguous()
    rc = _load().oracle_stream_fwd(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), B, Hq, Hkv, Lq, Lk, D,
        1 if causal else 0, float(scale), float(softcap), int(window_left), int(window_right),
        al.data_ptr() if al is not None else None, lse.data_ptr() if lse is not None else None,
    )
    if rc != 0:
        raise ValueError(f"oracle_stream_fwd failed ({rc})")
    return (out, lse) if return_lse else out
