"""Single-row grouped-query decode: the library computes the query heads of a
K/V head as rows of one workgroup (the K/V head is read once for all of them).
The result must be bit-identical to the same call with K/V repeated per query
head (where each head runs alone) -- rows of single-row sequences use per-row
rescales, so no row depends on the others in its wavefront -- and meet the
oracle bars.  Windows and ALiBi (position-dependent) keep the per-head path."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _kernel
from oracle import chunked
from gpu_util import DEV, REL_16, REL_16_OUT, default_scale, make_qkv, max_err

pytestmark = pytest.mark.gpu

def fp32_out(q, k, v, kw):
    """The same call with the kernel's fp32 output (the parity mode)."""
    scale = kw.get("softmax_scale", default_scale(q.shape[-1]))
    ws = kw.get("window_size", (-1, -1))
    return _kernel.forward_bshd(q, k, v, scale, kw.get("causal", False), kw.get("softcap", 0.0), ws[0], ws[1],
                                kw.get("alibi_slopes"), out_dtype=torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lk,split", [(1000, 0), (5000, None), (777, 256)])
@pytest.mark.parametrize("kw", [dict(), dict(causal=True), dict(softcap=5.0, softmax_scale=0.07)],
                         ids=["plain", "causal", "softcap"])
def test_packed_decode_equals_repeated_heads(dtype, lk, split, kw, monkeypatch):
    monkeypatch.setattr(_kernel, "_SPLIT_KEYS", split)
    for hq, hkv, d in ((8, 2, 128), (32, 8, 64), (12, 1, 96)):
        q, k, v = make_qkv(3, 1, lk, hq, hkv, d, dtype, seed=lk + hq)
        a, la = mfa.flash_attn_func_with_lse(q, k, v, **kw)
        r = hq // hkv
        b, lb = mfa.flash_attn_func_with_lse(q, k.repeat_interleave(r, 2), v.repeat_interleave(r, 2), **kw)
        assert torch.equal(a, b), f"hq={hq} hkv={hkv}"
        assert torch.equal(la, lb), f"lse hq={hq} hkv={hkv}"
        ref, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), return_lse=True,
                                               **{x: y for x, y in kw.items()})
        rmax = ref.abs().max().item()
        assert max_err(a, ref) <= REL_16_OUT * rmax
        e32 = max_err(fp32_out(q, k, v, kw), ref)
        assert e32 <= REL_16 * rmax, f"fp32 output hq={hq} hkv={hkv} d={d}: {e32 / rmax:.3e} x max|ref| > {REL_16:.1e}"
        assert (la.cpu() - ref_lse).abs().max().item() <= 4e-3


def test_windows_and_alibi_keep_per_head_rows():
    # position-dependent masks/biases: results still match the oracle
    q, k, v = make_qkv(2, 1, 900, 8, 2, 64, torch.bfloat16, seed=3)
    slopes = torch.linspace(0.1, 0.8, 8, device=DEV)
    for kw in (dict(window_size=(100, 0)), dict(alibi_slopes=slopes), dict(window_size=(50, 0), causal=True)):
        out = mfa.flash_attn_func(q, k, v, **kw)
        ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(),
                                      **{x: (y.cpu() if torch.is_tensor(y) else y) for x, y in kw.items()})
        assert max_err(out, ref) <= REL_16_OUT * ref.abs().max().item(), kw
        assert max_err(fp32_out(q, k, v, kw), ref) <= REL_16 * ref.abs().max().item(), kw


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("split", [0, None, 256])
def test_packed_varlen_decode(dtype, split, monkeypatch):
    # varlen decode (at most one query token per sequence; empty sequences too):
    # bit-identical to repeated K/V heads and to each sequence's dense call
    from gpu_util import make_varlen
    from test_gpu_lse_paged import paginate

    monkeypatch.setattr(_kernel, "_SPLIT_KEYS", split)
    lens_q, lens_k = [1, 1, 0, 1, 1], [700, 4100, 9, 1, 2600]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 2, 128, dtype, seed=20)
    args = (cu_q, cu_k, 1, max(lens_k))
    for kw in (dict(causal=True), dict(softcap=4.0)):
        out = mfa.flash_attn_varlen_func(q, k, v, *args, **kw)
        rep = mfa.flash_attn_varlen_func(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), *args, **kw)
        assert torch.equal(out, rep), kw
        pk, pv, table = paginate(k, v, lens_k, 512, seed=21)
        paged = mfa.flash_attn_varlen_func(q, pk, pv, *args, block_table=table, **kw)
        assert torch.equal(out, paged), kw
        sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
        sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
        for i in range(len(lens_q)):
            if lens_q[i] == 0:
                continue
            dense = mfa.flash_attn_func(q[None, sq[i]:sq[i + 1]], k[None, sk[i]:sk[i + 1]], v[None, sk[i]:sk[i + 1]],
                                        **kw)[0]
            assert torch.equal(out[sq[i]:sq[i + 1]], dense), (kw, i)
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), **kw)
        assert max_err(out, ref) <= REL_16_OUT * ref.abs().max().item()
        out32 = _kernel.forward_varlen(q, k, v, *args, default_scale(128), kw.get("causal", False),
                                       kw.get("softcap", 0.0), out_dtype=torch.float32)
        assert max_err(out32, ref) <= REL_16 * ref.abs().max().item(), kw
    # with an lse output the varlen call keeps per-head rows (same values)
    out2, lse = mfa.flash_attn_varlen_func_with_lse(q, k, v, *args, causal=True)
    assert torch.equal(out2, mfa.flash_attn_varlen_func(q, k, v, *args, causal=True))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 2)])
def test_single_rows_carry_two_term_probabilities(dtype, hq, hkv):
    # One query row over 8192 near-equal weights (small scale): O is an
    # average with a small max|O|, against which one bf16 rounding of every
    # weight alone is ~2^-9 of max|ref| -- the size of the 2e-3 bar itself.
    # Single rows run the exact-row kernel (weights as a sum of two 16-bit
    # terms, ~16 mantissa bits), so the fp32 output stays 10x inside the bar
    # (one-row-per-head calls and packed grouped-query rows alike; split-KV
    # chunks included).
    q, k, v = make_qkv(4, 1, 8192, hq, hkv, 128, dtype, seed=77)
    assert _kernel.launch_info(q, k, v).kernel_name.startswith(b"mfa_fwd16x")
    for kw in (dict(softmax_scale=0.02), dict(softmax_scale=0.02, causal=True), dict(softcap=2.0)):
        ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), **kw)
        rmax = ref.abs().max().item()
        e32 = max_err(fp32_out(q, k, v, kw), ref)
        assert e32 <= 2e-4 * rmax, f"{kw}: fp32 output {e32 / rmax:.3e} x max|ref|"
        assert max_err(mfa.flash_attn_func(q, k, v, **kw), ref) <= REL_16_OUT * rmax, kw
