"""GPU parity of the split-KV forward (mfa_fwd_splitkv: key chunks computed in
parallel, merged by log-sum-exp weighting) against the oracle.  Small chunk
sizes are forced so that short test shapes run through many chunks, including
empty ones (causal, window, varlen tails) and chunks whose every row is masked.

Bar: the bf16/fp16 bars of the single-pass kernels (fp32 output <=
2e-3*max|ref|, 16-bit output <= 4e-3*max|ref|), for the split result and for
the single-pass result on the same inputs alike, on every shape: single query
rows over thousands of keys (O averages many keys, so max|ref| is small) run
the exact-row kernel, whose probabilities carry two 16-bit terms.  The
bit-exact properties hold
within split-KV too: GQA equals repeated K/V, each varlen sequence equals its
dense B=1 call, and a single chunk reproduces the single-pass result."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import REL_16, REL_16_OUT, default_scale, make_qkv, make_varlen, max_err

pytestmark = pytest.mark.gpu

DTYPES16 = [torch.bfloat16, torch.float16]

@pytest.fixture
def chunk(request, monkeypatch):
    monkeypatch.setattr(_kernel, "_SPLIT_KEYS", request.param)
    return request.param


def run_both(q, k, v, **kw):
    out = mfa.flash_attn_func(q, k, v, **kw)
    scale = kw.get("softmax_scale")
    scale = scale if scale is not None else default_scale(q.shape[-1])
    ws = kw.get("window_size", (-1, -1))
    out32 = _kernel.forward_bshd(q, k, v, scale, kw.get("causal", False), kw.get("softcap", 0.0), ws[0], ws[1],
                                 kw.get("alibi_slopes"), out_dtype=torch.float32)
    return out, out32


def check(q, k, v, what="", **kw):
    out, out32 = run_both(q, k, v, **kw)
    assert out.shape == q.shape and out.dtype == q.dtype
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), softmax_scale=kw.get("softmax_scale"),
                                  causal=kw.get("causal", False), window_size=kw.get("window_size", (-1, -1)),
                                  softcap=kw.get("softcap", 0.0),
                                  alibi_slopes=kw["alibi_slopes"].cpu() if kw.get("alibi_slopes") is not None
                                  else None)
    saved = _kernel._SPLIT_KEYS
    _kernel._SPLIT_KEYS = 0
    try:
        single, single32 = run_both(q, k, v, **kw)
    finally:
        _kernel._SPLIT_KEYS = saved
    ref_max = ref.abs().max().item()
    for got, base, bar, kind in ((out32, single32, REL_16 * ref_max, "fp32 out"),
                                 (out, single, REL_16_OUT * ref_max, f"{q.dtype} out")):
        err, err_single = max_err(got, ref), max_err(base, ref)
        assert err <= bar and err_single <= bar, \
            (f"{what} ({kind}): split err {err / ref_max:.3e}, single-pass err {err_single / ref_max:.3e} "
             f"x max|ref|, bar {bar / ref_max:.3e}")
    return out


@pytest.mark.parametrize("chunk", [64, 192, 1024, 2048], indirect=True)
@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("lq,lk", [(1, 1000), (5, 777), (130, 300), (1, 5), (16, 2100), (300, 64)])
def test_shapes(chunk, dtype, lq, lk):
    q, k, v = make_qkv(2, lq, lk, 4, 4, 64, dtype, seed=lq + lk)
    check(q, k, v, f"split {chunk} Lq={lq} Lk={lk}")
    check(q, k, v, f"split {chunk} Lq={lq} Lk={lk} causal", causal=True)


@pytest.mark.parametrize("chunk", [64, 128], indirect=True)
@pytest.mark.parametrize("d", [40, 96, 128])
def test_head_dims(chunk, d):
    q, k, v = make_qkv(1, 3, 700, 4, 2, d, torch.bfloat16, seed=d)
    check(q, k, v, f"D={d}")


@pytest.mark.parametrize("chunk", [64], indirect=True)
@pytest.mark.parametrize("dtype", DTYPES16)
def test_features(chunk, dtype):
    q, k, v = make_qkv(1, 9, 900, 4, 4, 64, dtype, seed=11)
    slopes = torch.tensor([0.5, 0.25, 0.125, 0.0625], device="cuda")
    check(q, k, v, "window", window_size=(200, 0), causal=True)
    check(q, k, v, "window both sides", window_size=(100, 50))
    check(q, k, v, "softcap+alibi", softcap=5.0, alibi_slopes=slopes)
    check(q, k, v, "negative scale", softmax_scale=-0.1)
    # rows that see no key at all (causal, Lq > Lk) stay exactly zero
    q2, k2, v2 = make_qkv(1, 40, 20, 2, 2, 64, dtype, seed=12)
    out = check(q2, k2, v2, "causal Lq > Lk", causal=True)
    assert torch.count_nonzero(out[:, :20]) == 0


@pytest.mark.parametrize("chunk", [64], indirect=True)
def test_gqa_bit_exact_vs_repeated_kv(chunk):
    q, k, v = make_qkv(2, 7, 500, 8, 2, 64, torch.bfloat16, seed=3)
    a = mfa.flash_attn_func(q, k, v, causal=True)
    b = mfa.flash_attn_func(q, k.repeat_interleave(4, dim=2), v.repeat_interleave(4, dim=2), causal=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("chunk", [64, 256], indirect=True)
@pytest.mark.parametrize("dtype", DTYPES16)
def test_varlen(chunk, dtype):
    lens_q, lens_k = [1, 4, 0, 3, 2], [700, 33, 9, 0, 1300]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 2, 64, dtype, seed=5)
    def run():
        o = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), causal=True)
        o32 = _kernel.forward_varlen(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), default_scale(64), True,
                                     out_dtype=torch.float32)
        return o, o32

    out, out32 = run()
    _kernel._SPLIT_KEYS = 0
    single, single32 = run()
    _kernel._SPLIT_KEYS = chunk
    ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True)
    ref_max = ref.abs().max().item()
    for got, base, bar in ((out32, single32, REL_16 * ref_max), (out, single, REL_16_OUT * ref_max)):
        err, err_single = max_err(got, ref), max_err(base, ref)
        assert err <= bar and err_single <= bar, \
            f"varlen split err {err / ref_max:.3e}, single {err_single / ref_max:.3e} x max|ref|"
    # each sequence equals its dense B=1 call bit for bit (same chunks)
    sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
    sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
    for i in range(len(lens_q)):
        if lens_q[i] == 0:
            continue
        dense = mfa.flash_attn_func(q[None, sq[i]:sq[i + 1]], k[None, sk[i]:sk[i + 1]], v[None, sk[i]:sk[i + 1]],
                                    causal=True)[0]
        assert torch.equal(out[sq[i]:sq[i + 1]], dense), f"sequence {i}"


@pytest.mark.parametrize("dtype", DTYPES16)
def test_one_chunk_equals_single_pass(dtype, monkeypatch):
    q, k, v = make_qkv(2, 6, 300, 4, 4, 64, dtype, seed=8)
    monkeypatch.setattr(_kernel, "_SPLIT_KEYS", 0)
    single = mfa.flash_attn_func(q, k, v, causal=True)
    monkeypatch.setattr(_kernel, "_SPLIT_KEYS", 320)  # one chunk covers every key
    assert torch.equal(mfa.flash_attn_func(q, k, v, causal=True), single)


@pytest.mark.parametrize("dtype", DTYPES16)
def test_library_choice_on_a_decode_shape(dtype):
    # the library splits decode-like calls (few query rows, long key range)
    q, k, v = make_qkv(1, 1, 4096, 8, 2, 128, dtype, seed=9)
    p = _hip.MfaFwdParams()
    p.seqlen_q, p.seqlen_k, p.dtype_in = 1, 4096, _hip.DTYPE_CODES[dtype]
    assert _hip.split_keys(p) == 2048
    check(q, k, v, "auto split decode")
    check(q, k, v, "auto split decode causal", causal=True)
