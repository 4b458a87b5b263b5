"""Shared helpers of the GPU parity tests (inputs, tolerances, native-code check)."""
from __future__ import annotations

import math

import torch

DEV = "cuda"

# Bars from the north star: fp32 max abs error <= 1e-5; fp16/bf16 max abs error
# <= 2e-3 * max|ref| with fp32 accumulation, judged on the kernel's fp32 output
# (out_dtype=torch.float32).  The output rounded to bf16 cannot meet 2e-3 by
# construction (rounding an exact result to bf16 alone costs up to 2^-9 of each
# element), so the bf16/fp16 *output* is held to 4e-3 * max|ref| and its error is
# reported beside the parity figure.
FP32_ATOL = 1e-5
REL_16 = 2e-3
REL_16_OUT = 4e-3


def make_qkv(B, Lq, Lk, Hq, Hkv, D, dtype, seed=0, scale_inputs=1.0):
    """The reference's recipe (tests/test_flash_attn_func.py:52-57): CPU generator,
    randn for q, then k, then v in [B,S,H,D], cast, move to the device."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, Lq, Hq, D, generator=g) * scale_inputs
    k = torch.randn(B, Lk, Hkv, D, generator=g) * scale_inputs
    v = torch.randn(B, Lk, Hkv, D, generator=g) * scale_inputs
    return q.to(DEV, dtype), k.to(DEV, dtype), v.to(DEV, dtype)


def make_varlen(seqlens_q, seqlens_k, Hq, Hkv, D, dtype, seed=0):
    """tests/test_flash_attn_varlen_func.py:12-19."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(sum(seqlens_q), Hq, D, generator=g).to(DEV, dtype)
    k = torch.randn(sum(seqlens_k), Hkv, D, generator=g).to(DEV, dtype)
    v = torch.randn(sum(seqlens_k), Hkv, D, generator=g).to(DEV, dtype)
    cu_q = torch.tensor([0] + list(seqlens_q), dtype=torch.int32).cumsum(0, dtype=torch.int32).to(DEV)
    cu_k = torch.tensor([0] + list(seqlens_k), dtype=torch.int32).cumsum(0, dtype=torch.int32).to(DEV)
    return q, k, v, cu_q, cu_k


def max_err(out, ref):
    return (out.detach().float().cpu() - ref.float()).abs().max().item()


def assert_parity(out, ref, dtype, what=""):
    """out: kernel result (fp32 output mode for 16-bit inputs); ref: oracle fp32."""
    err = max_err(out, ref)
    if dtype == torch.float32:
        assert err <= FP32_ATOL, f"{what}: fp32 max abs err {err:.3e} > {FP32_ATOL}"
    else:
        ref_max = ref.abs().max().item()
        assert err <= REL_16 * ref_max, f"{what}: max abs err {err:.3e} > {REL_16}*{ref_max:.3f}"
    return err


def assert_output(out, ref, dtype, what=""):
    """out: kernel result in the input dtype (the public API's return)."""
    err = max_err(out, ref)
    if dtype == torch.float32:
        assert err <= FP32_ATOL, f"{what}: fp32 max abs err {err:.3e}"
    else:
        ref_max = ref.abs().max().item()
        assert err <= REL_16_OUT * ref_max, f"{what}: {dtype} output max abs err {err:.3e} > {REL_16_OUT}*{ref_max:.3f}"
    return err


def native_library_mapped() -> bool:
    """True when libmtlfa_hip.so is mapped into this process."""
    with open("/proc/self/maps") as f:
        return any("libmtlfa_hip.so" in line for line in f)


def default_scale(D):
    return 1.0 / math.sqrt(D)
