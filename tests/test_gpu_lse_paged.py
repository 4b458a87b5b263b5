"""GPU parity of the softmax_lse output and of paged K/V (block_table), two
features the reference raises NotImplementedError for
(metal_flash_attn/__init__.py:49-50, :130-131).

softmax_lse is checked against the oracle's log-sum-exp of the masked scores
(oracle/chunked.py, pinned against a float64 C statement and closed forms in
test_oracle_pinning.py).  Bars: fp32 inputs 1e-5 * max(1, max|lse|); bf16/fp16
inputs 4e-3 absolute -- the kernel sums probabilities after rounding them to
16 bits for the PV product (relative error <= 2^-8 of the row sum, i.e.
<= 3.9e-3 in lse).  Rows with no valid key must be exactly -inf.

Paged K/V must equal, bit for bit, the same call on the contiguous K/V the
pages hold (the kernels do the same arithmetic; only the addresses differ),
across page sizes (256, 512 and 768, which is not a power of two), every
kernel (256-row, ping-pong, fp32, split-KV) and sequences that end inside,
at and just past a page boundary; the oracle on the gathered K/V checks the
result itself.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import DEV, REL_16, assert_output, assert_parity, default_scale, make_qkv, make_varlen, max_err

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]
LSE_16 = 4e-3


@pytest.fixture
def knobs(monkeypatch):
    def set_(hint=0, split=None):
        monkeypatch.setattr(_kernel, "_TILE_HINT", hint)
        monkeypatch.setattr(_kernel, "_SPLIT_KEYS", split)
    return set_


def check_lse(got, ref, dtype, what=""):
    got = got.detach().cpu()
    assert got.shape == ref.shape and got.dtype == torch.float32, what
    assert torch.equal(torch.isneginf(got), torch.isneginf(ref)), f"{what}: -inf rows differ"
    fin = torch.isfinite(ref)
    assert torch.isfinite(got[fin]).all(), what
    if not fin.any():
        return 0.0
    err = (got[fin].double() - ref[fin].double()).abs().max().item()
    bar = 1e-5 * max(1.0, ref[fin].abs().max().item()) if dtype == torch.float32 else LSE_16
    assert err <= bar, f"{what}: lse max abs err {err:.3e} > {bar:.3e}"
    return err


FEATURES = [
    dict(),
    dict(causal=True),
    dict(causal=True, window_size=(64, 0)),
    dict(window_size=(50, 20)),
    dict(softcap=5.0, alibi=True),
    dict(softmax_scale=-0.1),
]


@pytest.mark.parametrize("hint", [0, 1, 2])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
def test_lse_dense(hint, dtype, feat, knobs):
    if hint == 2 and dtype == torch.float32:
        pytest.skip("ping-pong tiles are bf16/fp16 only")
    knobs(hint, 0)
    D = 64 if hint == 2 else 128
    q, k, v = make_qkv(2, 300, 333, 4, 2, D, dtype, seed=21)
    kw = dict(feat)
    if kw.pop("alibi", False):
        kw["alibi_slopes"] = torch.tensor([0.5, 0.25, 0.125, 0.0625], device=DEV)
    out, lse = mfa.flash_attn_func_with_lse(q, k, v, **kw)
    ref, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(),
                                           alibi_slopes=kw["alibi_slopes"].cpu() if "alibi_slopes" in kw else None,
                                           **{x: y for x, y in kw.items() if x != "alibi_slopes"}, return_lse=True)
    check_lse(lse, ref_lse, dtype, f"lse {feat}")
    assert_output(out, ref, dtype, f"out {feat}")
    # the lse call leaves O unchanged
    assert torch.equal(out, mfa.flash_attn_func(q, k, v, **kw))


@pytest.mark.parametrize("dtype", DTYPES)
def test_lse_of_rows_without_keys(dtype, knobs):
    knobs(0, 0)
    q, k, v = make_qkv(1, 40, 20, 2, 2, 64, dtype, seed=22)
    out, lse = mfa.flash_attn_func_with_lse(q, k, v, causal=True)
    assert torch.isneginf(lse[:, :, :20]).all() and torch.isfinite(lse[:, :, 20:]).all()
    assert torch.count_nonzero(out[:, :20]) == 0
    _, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), causal=True, return_lse=True)
    check_lse(lse, ref_lse, dtype)


@pytest.mark.parametrize("chunk", [64, 256, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lse_split_kv(chunk, dtype, knobs):
    knobs(0, chunk)
    for lq, lk, causal in ((1, 4100, False), (5, 777, True), (130, 300, False)):
        q, k, v = make_qkv(2, lq, lk, 4, 4, 64, dtype, seed=lq + lk)
        out, lse = mfa.flash_attn_func_with_lse(q, k, v, causal=causal)
        ref, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), causal=causal, return_lse=True)
        check_lse(lse, ref_lse, dtype, f"split {chunk} Lq={lq} Lk={lk}")
        # the merged O is the split path's O
        knobs(0, chunk)
        assert torch.equal(out, mfa.flash_attn_func(q, k, v, causal=causal))


@pytest.mark.parametrize("split", [0, 64])
@pytest.mark.parametrize("dtype", DTYPES)
def test_lse_varlen(split, dtype, knobs):
    if split and dtype == torch.float32:
        pytest.skip("split-KV is bf16/fp16 only")
    knobs(0, split)
    lens_q, lens_k = [1, 4, 0, 3, 20], [700, 33, 9, 0, 130]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 2, 64, dtype, seed=23)
    out, lse = mfa.flash_attn_varlen_func_with_lse(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), causal=True)
    ref, ref_lse = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True,
                                                  return_lse=True)
    assert lse.shape == (8, sum(lens_q))
    check_lse(lse, ref_lse, dtype, "varlen")
    assert_output(out, ref, dtype, "varlen out")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_merge_of_key_shards_on_the_kernel(dtype, knobs):
    # the context-parallel merge: attention over key shards, combined by lse
    knobs(0, 0)
    q, k, v = make_qkv(1, 200, 1000, 4, 4, 64, dtype, seed=24)
    parts = [_kernel.forward_bshd(q, k[:, a:b], v[:, a:b], default_scale(64), False, out_dtype=torch.float32,
                                  return_lse=True) for a, b in ((0, 300), (300, 301), (301, 1000))]
    out, lse = mfa.merge_attention_partials([o for o, _ in parts], [l for _, l in parts])
    ref, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), return_lse=True)
    assert_parity(out, ref, dtype, "merged shards")
    check_lse(lse, ref_lse, dtype, "merged lse")


# --------------------------------------------------------------------------- paged K/V


def paginate(k, v, lens_k, page, seed):
    """Packed k/v [T, H, D] -> (page pools with the sequences' pages in shuffled
    slots among garbage pages, int32 block table with -1 past each sequence)."""
    g = torch.Generator().manual_seed(seed)
    need = [-(-n // page) for n in lens_k]
    npages = sum(need) + 3
    slots = torch.randperm(npages, generator=g).tolist()
    H, D = k.shape[1], k.shape[2]
    pk = (torch.randn(npages, page, H, D, generator=g) * 7).to(k.device, k.dtype)  # garbage everywhere else
    pv = (torch.randn(npages, page, H, D, generator=g) * 7).to(k.device, k.dtype)
    table = torch.full((len(lens_k), max(need + [1]) + 1), -1, dtype=torch.int32)
    start, nxt = 0, 0
    for b, n in enumerate(lens_k):
        for i in range(need[b]):
            pid = slots[nxt]
            nxt += 1
            table[b, i] = pid
            rows = min(page, n - i * page)
            pk[pid, :rows] = k[start + i * page:start + i * page + rows]
            pv[pid, :rows] = v[start + i * page:start + i * page + rows]
        start += n
    return pk, pv, table.to(k.device)


PAGED_LENS = ([3, 1, 0, 17, 2, 40, 5], [255, 256, 9, 0, 257, 1300, 2])


@pytest.mark.parametrize("page", [256, 512, 768])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hint", [0, 1, 2])
def test_paged_equals_contiguous(page, dtype, hint, knobs):
    if hint == 2 and dtype == torch.float32:
        pytest.skip("ping-pong tiles are bf16/fp16 only")
    knobs(hint, 0)
    lens_q, lens_k = PAGED_LENS
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 2, 64, dtype, seed=page)
    pk, pv, table = paginate(k, v, lens_k, page, seed=page + 1)
    for kw in (dict(causal=True), dict(), dict(window_size=(100, 0), softcap=3.0)):
        args = (cu_q, cu_k, max(lens_q), max(lens_k))
        paged = mfa.flash_attn_varlen_func(q, pk, pv, *args, block_table=table, **kw)
        flat = mfa.flash_attn_varlen_func(q, k, v, *args, **kw)
        assert torch.equal(paged, flat), f"page {page} {kw}"
        ref = chunked.flash_attn_varlen_func(q.cpu(), chunked.gather_pages(pk, table, lens_k),
                                             chunked.gather_pages(pv, table, lens_k), cu_q.cpu(), cu_k.cpu(), **kw)
        assert_output(paged, ref, dtype, f"paged {page} {kw}")


@pytest.mark.parametrize("split", [None, 256, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_paged_split_kv(split, dtype, knobs):
    # decode-like: few query rows, long paged key ranges (auto split = 2048)
    knobs(0, split)
    lens_q, lens_k = [1, 4, 1, 2], [5000, 2049, 0, 777]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 1, 128, dtype, seed=31)
    pk, pv, table = paginate(k, v, lens_k, 512, seed=32)
    args = (cu_q, cu_k, max(lens_q), max(lens_k))
    out, lse = mfa.flash_attn_varlen_func_with_lse(q, pk, pv, *args, block_table=table, causal=True)
    flat, flat_lse = mfa.flash_attn_varlen_func_with_lse(q, k, v, *args, causal=True)
    assert torch.equal(out, flat) and torch.equal(lse, flat_lse)
    ref, ref_lse = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True,
                                                  return_lse=True)
    assert_output(out, ref, dtype, f"paged split {split}")
    check_lse(lse, ref_lse, dtype, f"paged split {split}")


def test_paged_dense_layout_through_the_launcher(knobs):
    # dense (non-varlen) paging: every sequence has seqlen_k keys
    knobs(0, 0)
    B, Lq, Lk, H, D = 3, 70, 600, 4, 64
    q, k, v = make_qkv(B, Lq, Lk, H, H, D, torch.bfloat16, seed=33)
    pk, pv, table = paginate(k.reshape(B * Lk, H, D), v.reshape(B * Lk, H, D), [Lk] * B, 256, seed=34)
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=DEV)
    _kernel._run(q, pk, pv, out, scale=default_scale(D), causal=True, softcap=0.0, window_left=-1,
                 window_right=-1, alibi=None, alibi_bstride=0, seqlen_k=Lk, block_table=table)
    assert torch.equal(out, mfa.flash_attn_func(q, k, v, causal=True))


def test_out_of_range_page_ids_read_as_zero(knobs):
    # The library guards its page-table reads: an id outside [0, num_pages)
    # reads zeros instead of memory (the Python API rejects such tables
    # before launch; this calls the C ABI directly).  Expected: attention
    # with those keys and values zero.
    knobs(0, 0)
    lens_q, lens_k = [4], [600]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 2, 2, 64, torch.bfloat16, seed=35)
    pk, pv, table = paginate(k, v, lens_k, 256, seed=36)
    bad = table.clone()
    bad[0, 1] = pk.shape[0]  # keys 256..511 -> an id one past the pool
    out = torch.empty_like(q)
    p = _hip.MfaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), pk.data_ptr(), pv.data_ptr(), out.data_ptr()
    p.q_seq_stride, p.q_head_stride = q.stride(0), q.stride(1)
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = pk.stride()[:3]
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = pv.stride()[:3]
    p.o_seq_stride, p.o_head_stride = out.stride(0), out.stride(1)
    p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim = 1, 2, 2, 4, 600, 64
    p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.scale, p.window_left, p.window_right = default_scale(64), -1, -1
    p.dtype_in = p.dtype_out = _hip.MFA_DTYPE_BF16
    p.block_table, p.block_table_batch_stride = bad.data_ptr(), bad.stride(0)
    p.page_block_size, p.num_pages = 256, pk.shape[0]
    _hip.fwd(p, torch.cuda.current_stream().cuda_stream)
    kz, vz = k.clone(), v.clone()
    kz[256:512] = 0
    vz[256:512] = 0
    assert torch.equal(out, mfa.flash_attn_varlen_func(q, kz, vz, cu_q, cu_k, 4, 600))
