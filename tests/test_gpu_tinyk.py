"""Cross-attention to a short key sequence (at most 32 keys, many query rows):
the library runs the tiny-key kernel (keys held in registers, query rows
streamed).  This is the reference's tiny-Lk case (README.md:141-145: bf16
D=128 Lq=26136 Lk=5; tests/test_v2_dtype_modes.py:147-171 keeps such shapes
off its register-resident tier).  Results must meet the oracle bars and equal
the 4-wavefront kernel's bit for bit (per row the same operations in the same
order), so grouped-query heads equal repeated K/V and each varlen sequence
equals its dense call, as elsewhere."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import DEV, assert_output, assert_parity, default_scale, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

DTYPES16 = [torch.bfloat16, torch.float16]
SHAPES = [  # B, Lq, Lk, Hq, Hkv, D
    (1, 2000, 5, 4, 4, 128),
    (2, 700, 1, 4, 2, 64),
    (1, 1500, 17, 3, 1, 64),
    (2, 513, 32, 4, 4, 128),
    (1, 300, 16, 2, 2, 32),
    (1, 640, 9, 2, 2, 96),
    (1, 777, 12, 2, 1, 72),
]
FEATURES = [
    dict(),
    dict(causal=True),
    dict(softcap=4.0, softmax_scale=0.3),
    dict(alibi=True),
    dict(window_size=(3, 2)),
    dict(causal=True, softcap=20.0, alibi=True),
]


@pytest.fixture
def hint(monkeypatch):
    def set_(h):
        monkeypatch.setattr(_kernel, "_TILE_HINT", h)
    return set_


def _kw(feat, Hq):
    kw = dict(feat)
    if kw.pop("alibi", False):
        kw["alibi_slopes"] = torch.linspace(0.05, 0.9, Hq, device=DEV)
    return kw


def _oracle(q, k, v, kw, **extra):
    return chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(),
                                   **{x: (y.cpu() if torch.is_tensor(y) else y) for x, y in kw.items()}, **extra)


def _fp32_out(q, k, v, kw):
    ws = kw.get("window_size", (-1, -1))
    return _kernel.forward_bshd(q, k, v, kw.get("softmax_scale", default_scale(q.shape[-1])), kw.get("causal", False),
                                kw.get("softcap", 0.0), ws[0], ws[1], kw.get("alibi_slopes"), out_dtype=torch.float32)


def test_library_choice():
    q, k, v = make_qkv(1, 2000, 5, 4, 4, 128, torch.bfloat16, seed=1)
    assert _kernel.launch_info(q, k, v).kernel_name.startswith(b"mfa_fwd16tk<bf16,d128")
    q, k, v = make_qkv(1, 2000, 33, 4, 4, 128, torch.bfloat16, seed=1)  # a second key block: not tiny
    assert not _kernel.launch_info(q, k, v).kernel_name.startswith(b"mfa_fwd16tk")
    q, k, v = make_qkv(1, 64, 5, 4, 4, 128, torch.bfloat16, seed=1)  # few query rows
    assert not _kernel.launch_info(q, k, v).kernel_name.startswith(b"mfa_fwd16tk")


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
def test_oracle_and_four_wave_kernel(dtype, shape, feat, hint):
    B, Lq, Lk, Hq, Hkv, D = shape
    q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, dtype, seed=Lq + Lk + D)
    kw = _kw(feat, Hq)
    out, lse = mfa.flash_attn_func_with_lse(q, k, v, **kw)
    out32 = _fp32_out(q, k, v, kw)
    ref, ref_lse = _oracle(q, k, v, kw, return_lse=True)
    assert_parity(out32, ref, dtype, f"tiny-key fp32 out {shape} {feat}")
    assert_output(out, ref, dtype, f"tiny-key {dtype} out {shape} {feat}")
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isneginf(lse.cpu()), torch.isneginf(ref_lse))
    if fin.any():
        assert (lse.cpu()[fin] - ref_lse[fin]).abs().max().item() <= 4e-3
    # the 4-wavefront kernel gives the same bits
    hint(_hip.MFA_TILE_256)
    out_4w, lse_4w = mfa.flash_attn_func_with_lse(q, k, v, **kw)
    assert torch.equal(out, out_4w), f"{shape} {feat}"
    assert torch.equal(lse, lse_4w), f"{shape} {feat}"
    assert torch.equal(out32, _fp32_out(q, k, v, kw)), f"{shape} {feat}"


@pytest.mark.parametrize("dtype", DTYPES16)
def test_gqa_equals_repeated_heads(dtype):
    q, k, v = make_qkv(2, 1000, 7, 8, 2, 128, dtype, seed=5)
    a = mfa.flash_attn_func(q, k, v, causal=True)
    b = mfa.flash_attn_func(q, k.repeat_interleave(4, 2), v.repeat_interleave(4, 2), causal=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES16)
def test_varlen_sequences_equal_dense_calls(dtype):
    lens_q, lens_k = [300, 0, 513, 1000], [5, 7, 32, 1]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 4, 2, 64, dtype, seed=6)
    for kw in (dict(), dict(causal=True), dict(softcap=3.0)):
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), **kw)
        sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
        sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
        for i in range(len(lens_q)):
            if lens_q[i] == 0:
                continue
            dense = mfa.flash_attn_func(q[None, sq[i]:sq[i + 1]], k[None, sk[i]:sk[i + 1]], v[None, sk[i]:sk[i + 1]],
                                        **kw)[0]
            assert torch.equal(out[sq[i]:sq[i + 1]], dense), (kw, i)
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), **kw)
        assert_output(out, ref, dtype, f"varlen {kw}")


def test_reference_trace_shape():
    # the reference's trace example (README.md:141-145), 16 heads, rows checked
    # against the oracle on a subset
    q, k, v = make_qkv(1, 26136, 5, 16, 16, 128, torch.bfloat16, seed=10)
    out32 = _fp32_out(q, k, v, {})
    rows = torch.arange(0, 26136, 97)
    ref = chunked.flash_attn_func(q[:, rows].cpu(), k.cpu(), v.cpu())
    assert_parity(out32[:, rows], ref, torch.bfloat16, "trace shape")


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("Lk,D", [(5, 128), (32, 64), (1, 96)])
def test_packed_grouped_query_decode_with_few_keys(dtype, Lk, D, hint):
    # one query row per sequence with 128 query heads per K/V head: packed
    # into 128 rows per K/V head, enough rows for the tiny-key kernel's
    # threshold, but packed decode rows always run the exact-row kernel
    # (two-term probabilities), as any single-row call does
    B, Hq, Hkv = 3, 128, 1
    q, k, v = make_qkv(B, 1, Lk, Hq, Hkv, D, dtype, seed=40 + Lk)
    assert _kernel.launch_info(q, k, v).kernel_name.startswith(b"mfa_fwd16x")
    for kw in (dict(), dict(causal=True), dict(softcap=6.0, softmax_scale=0.2)):
        out = mfa.flash_attn_func(q, k, v, **kw)
        out32 = _fp32_out(q, k, v, kw)
        ref = _oracle(q, k, v, kw)
        assert_parity(out32, ref, dtype, f"packed decode, few keys, fp32 out Lk={Lk} D={D} {kw}")
        assert_output(out, ref, dtype, f"packed decode, few keys Lk={Lk} D={D} {kw}")
        # K/V repeated per query head: no packing, each head alone
        rep = mfa.flash_attn_func(q, k.repeat_interleave(Hq, 2), v.repeat_interleave(Hq, 2), **kw)
        assert torch.equal(out, rep), kw
        # a tile hint does not move exact rows off their kernel
        hint(_hip.MFA_TILE_256)
        assert torch.equal(out, mfa.flash_attn_func(q, k, v, **kw)), kw
        hint(_hip.MFA_TILE_AUTO)
    # varlen decode (one token per sequence) packs the same way
    lens_k = [Lk, max(1, Lk - 2), Lk]
    qv, kv_, vv, cu_q, cu_k = make_varlen([1, 1, 1], lens_k, Hq, Hkv, D, dtype, seed=50 + Lk)
    outv = mfa.flash_attn_varlen_func(qv, kv_, vv, cu_q, cu_k, 1, max(lens_k))
    refv = chunked.flash_attn_varlen_func(qv.cpu(), kv_.cpu(), vv.cpu(), cu_q.cpu(), cu_k.cpu())
    assert_output(outv, refv, dtype, f"packed varlen decode, few keys Lk={Lk} D={D}")
    sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
    for i in range(3):
        dense = mfa.flash_attn_func(qv[None, i:i + 1], kv_[None, sk[i]:sk[i + 1]], vv[None, sk[i]:sk[i + 1]])[0]
        assert torch.equal(outv[i:i + 1], dense), i


@pytest.mark.parametrize("dtype", DTYPES16)
def test_single_row_sequences_among_many_rows(dtype):
    # a varlen batch on the tiny-key kernel that also holds single-row
    # sequences: those run the exact-row kernel's launch, so every sequence
    # equals its dense call bit for bit
    lens_q, lens_k = [300, 1, 513, 1, 0], [5, 9, 32, 30, 4]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 4, 2, 64, dtype, seed=60)
    for kw in (dict(), dict(causal=True), dict(softcap=3.0)):
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), **kw)
        sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
        sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
        for i in range(len(lens_q)):
            if lens_q[i] == 0:
                continue
            dense = mfa.flash_attn_func(q[None, sq[i]:sq[i + 1]], k[None, sk[i]:sk[i + 1]], v[None, sk[i]:sk[i + 1]],
                                        **kw)[0]
            assert torch.equal(out[sq[i]:sq[i + 1]], dense), (kw, i)
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), **kw)
        assert_output(out, ref, dtype, f"mixed varlen {kw}")
