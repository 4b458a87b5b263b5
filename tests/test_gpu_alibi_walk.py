"""ALiBi at head dims 96 and 128: the key blocks are walked from the last to
the first (the block nearest the diagonal holds the row maxima, so O is
rarely rescaled), and prefetches past the walk use an empty buffer
resource formed from a block inside the range.  Only the summation order
differs from a left-to-right walk, so every result must meet the oracle bars
(_kernel.py:1188-1207: scale -> softcap -> ALiBi -> masks), and the layout
invariants must hold bit for bit: paged equals contiguous K/V, each varlen
sequence equals its dense call, split-KV chunks (whose walks end at chunk
boundaries) merge to the single-pass result within the bars."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import DEV, assert_output, assert_parity, default_scale, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

DTYPES16 = [torch.bfloat16, torch.float16]
FEATURES = [
    dict(causal=True),
    dict(causal=True, window_size=(300, 0)),
    dict(causal=True, softcap=20.0),
    dict(window_size=(200, 100)),
    dict(),
]


@pytest.fixture
def knobs(monkeypatch):
    def set_(hint=0, split=None):
        monkeypatch.setattr(_kernel, "_TILE_HINT", hint)
        monkeypatch.setattr(_kernel, "_SPLIT_KEYS", split)
    return set_


def _slopes(H):
    return torch.tensor([2.0 ** (-8.0 * (i + 1) / H) for i in range(H)], device=DEV)


def _cpu(kw):
    return {x: (y.cpu() if torch.is_tensor(y) else y) for x, y in kw.items()}


def _fp32(q, k, v, kw):
    ws = kw.get("window_size", (-1, -1))
    return _kernel.forward_bshd(q, k, v, kw.get("softmax_scale", default_scale(q.shape[-1])), kw.get("causal", False),
                                kw.get("softcap", 0.0), ws[0], ws[1], kw.get("alibi_slopes"), out_dtype=torch.float32)


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("d", [96, 128])
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
def test_kernels_meet_the_oracle(dtype, d, feat, knobs):
    # Lq = Lk = 700: a partial last key block; 4 heads, the ALiBi slope set of
    # 4 heads; both kernels at D = 128 (the ping-pong tiles have no D = 96)
    q, k, v = make_qkv(1, 700, 700, 4, 4, d, dtype, seed=d + len(feat))
    kw = dict(feat, alibi_slopes=_slopes(4))
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), **_cpu(kw))
    hints = [_hip.MFA_TILE_256] + ([_hip.MFA_TILE_PINGPONG] if d == 128 else [])
    for hint in hints:
        knobs(hint, 0)
        assert_parity(_fp32(q, k, v, kw), ref, dtype, f"hint {hint} D={d} {feat} fp32 out")
        assert_output(mfa.flash_attn_func(q, k, v, **kw), ref, dtype, f"hint {hint} D={d} {feat}")


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("d", [96, 128])
@pytest.mark.parametrize("page", [256, 512])
def test_paged_equals_contiguous(dtype, d, page, knobs):
    from test_gpu_lse_paged import paginate
    knobs(0, 0)
    lens_q, lens_k = [3, 1, 0, 17, 40, 5], [255, 256, 9, 300, 1300, 2]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 8, 2, d, dtype, seed=page + d)
    pk, pv, table = paginate(k, v, lens_k, page, seed=page + d + 1)
    args = (cu_q, cu_k, max(lens_q), max(lens_k))
    for feat in (dict(causal=True), dict(causal=True, window_size=(200, 0), softcap=5.0), dict()):
        kw = dict(feat, alibi_slopes=_slopes(8))
        paged = mfa.flash_attn_varlen_func(q, pk, pv, *args, block_table=table, **kw)
        flat = mfa.flash_attn_varlen_func(q, k, v, *args, **kw)
        assert torch.equal(paged, flat), f"page {page} D={d} {feat}"
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), **_cpu(kw))
        assert_output(paged, ref, dtype, f"paged {page} D={d} {feat}")


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("d", [96, 128])
def test_varlen_sequences_equal_dense_calls(dtype, d, knobs):
    knobs(0, None)
    lens = [96, 257, 1, 700]
    q, k, v, cu_q, cu_k = make_varlen(lens, lens, 4, 2, d, dtype, seed=d)
    starts = [0] + torch.tensor(lens).cumsum(0).tolist()
    for feat in (dict(causal=True), dict(causal=True, window_size=(128, 0))):
        kw = dict(feat, alibi_slopes=_slopes(4))
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens), max(lens), **kw)
        for i in range(len(lens)):
            s, e = starts[i], starts[i + 1]
            dense = mfa.flash_attn_func(q[None, s:e], k[None, s:e], v[None, s:e], **kw)[0]
            assert torch.equal(out[s:e], dense), f"D={d} {feat} sequence {i}"


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("d", [96, 128])
@pytest.mark.parametrize("split", [64, 256])
def test_split_kv_chunks(dtype, d, split, knobs):
    # few query rows over long key ranges: the chunks' reversed walks end at
    # chunk boundaries (and at key 0 for the first chunk)
    q, k, v = make_qkv(2, 5, 1500, 4, 2, d, dtype, seed=split + d)
    for feat in (dict(causal=True), dict(causal=True, window_size=(700, 0), softcap=10.0), dict()):
        kw = dict(feat, alibi_slopes=_slopes(4))
        ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), **_cpu(kw))
        knobs(0, split)
        assert_parity(_fp32(q, k, v, kw), ref, dtype, f"split {split} D={d} {feat} fp32 out")
        assert_output(mfa.flash_attn_func(q, k, v, **kw), ref, dtype, f"split {split} D={d} {feat}")
