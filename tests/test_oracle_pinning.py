"""Pins the oracle (oracle/chunked.py, the reference's chunked-fp32 torch path
restated) before anything is checked against it.

The reference holds no golden vectors (its tests compare against a naive fp32
statement, tests/test_flash_attn_func.py:12-49).  The oracle is pinned here by
  * torch's scaled_dot_product_attention (a library routine) wherever the
    semantics coincide (no softcap/ALiBi/window; causal only with Lq == Lk;
    GQA through enable_gqa);
  * oracle/stream_ref.c, a float64 two-pass evaluation of the reference's
    scalar-kernel math (metal_flash_attn/_kernel.py:32-87) -- a different
    evaluation order in a different language;
  * closed forms that a plausible mistake breaks: a dropped or misplaced
    softcap, a flipped ALiBi sign or missing |.|, a wrong bottom-right offset
    (Lk - Lq), an off-by-one window bound, a top-left causal mask, a missing
    scale, a transposed operand.
All on CPU; sizes keep the whole file to a few seconds.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import chunked, stream

ATOL = 1e-5


def rnd(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def qkv(B, Hq, Hkv, Lq, Lk, D, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Lq, D, generator=g) * scale
    k = torch.randn(B, Hkv, Lk, D, generator=g) * scale
    v = torch.randn(B, Hkv, Lk, D, generator=g) * scale
    return q, k, v


def close(a, b, atol=ATOL):
    err = (a.double() - b.double()).abs().max().item() if a.numel() else 0.0
    assert err <= atol, f"max abs err {err:.3e} > {atol}"


# --------------------------------------------------------------------------- library cross-checks


@pytest.mark.parametrize("D", [16, 64, 128])
def test_plain_matches_sdpa(D):
    q, k, v = qkv(2, 3, 3, 70, 90, D, seed=1)
    ref = F.scaled_dot_product_attention(q, k, v)
    close(chunked.flash_torch(q, k, v, 1 / math.sqrt(D), False), ref)


def test_custom_scale_matches_sdpa():
    q, k, v = qkv(1, 2, 2, 64, 64, 32, seed=2)
    for s in (0.25, 1.0, 0.01):
        close(chunked.flash_torch(q, k, v, s, False), F.scaled_dot_product_attention(q, k, v, scale=s))


def test_causal_equal_lengths_matches_sdpa():
    q, k, v = qkv(1, 4, 4, 97, 97, 64, seed=3)
    close(chunked.flash_torch(q, k, v, 0.125, True), F.scaled_dot_product_attention(q, k, v, is_causal=True))


@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 1), (6, 3)])
def test_gqa_matches_sdpa_enable_gqa(hq, hkv):
    q, k, v = qkv(2, hq, hkv, 40, 56, 32, seed=4)
    ref = F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
    close(chunked.flash_torch(q, k, v, 1 / math.sqrt(32), False), ref)


def test_config1_matches_sdpa():
    # BASELINE config 1 inputs: [1,512,2,64] fp32 from seed 0, scale 1/8
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 512, 2, 64, generator=g) for _ in range(3))
    out = chunked.flash_attn_func(q, k, v, softmax_scale=0.125)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale=0.125)
    close(out, ref.transpose(1, 2))


# --------------------------------------------------------------------------- independent float64 restatement


CASES = [
    dict(causal=False),
    dict(causal=True),
    dict(causal=True, window_left=7),
    dict(causal=False, window_left=5, window_right=3),
    dict(causal=False, window_left=-1, window_right=2),
    dict(causal=False, softcap=2.5),
    dict(causal=True, softcap=30.0),
    dict(causal=False, alibi="head"),
    dict(causal=True, alibi="batch"),
    dict(causal=True, window_left=9, softcap=4.0, alibi="head"),
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
@pytest.mark.parametrize("shape", [(2, 4, 2, 33, 33, 16), (1, 2, 2, 20, 45, 8), (1, 4, 1, 45, 20, 24)],
                         ids=["square-gqa", "lq<lk", "lq>lk-mqa"])
def test_matches_float64_stream(case, shape):
    B, Hq, Hkv, Lq, Lk, D = shape
    q, k, v = qkv(B, Hq, Hkv, Lq, Lk, D, seed=5)
    kw = dict(case)
    al = kw.pop("alibi", None)
    alibi = None
    if al == "head":
        alibi = chunked.broadcast_alibi(torch.linspace(0.05, 0.6, Hq), B, Hq)
    elif al == "batch":
        alibi = chunked.broadcast_alibi(torch.rand(B, Hq, generator=torch.Generator().manual_seed(1)), B, Hq)
    a = chunked.flash_torch(q, k, v, 0.3, alibi=alibi, **kw)
    b = stream.stream_fwd(q, k, v, 0.3, alibi=alibi, **kw)
    close(a, b)


# --------------------------------------------------------------------------- closed forms


def test_single_key_returns_its_value():
    q, k, v = qkv(1, 2, 2, 9, 1, 16, seed=6)
    out = chunked.flash_torch(q, k, v, 0.7, False)
    close(out, v.expand(1, 2, 9, 16))


def test_constant_values_return_the_constant():
    q, k, _ = qkv(1, 2, 2, 30, 40, 16, seed=7)
    row = rnd(16, seed=8)
    v = row.expand(1, 2, 40, 16).contiguous()
    for kw in (dict(causal=False), dict(causal=True), dict(causal=False, window_left=3, window_right=0),
               dict(causal=False, softcap=1.0)):
        out = chunked.flash_torch(q, k, v, 0.5, **kw)
        close(out, row.expand_as(out))


def test_zero_query_is_mean_of_values():
    _, k, v = qkv(1, 2, 2, 24, 24, 16, seed=9)
    q = torch.zeros(1, 2, 24, 16)
    close(chunked.flash_torch(q, k, v, 0.9, False), v.mean(dim=2, keepdim=True).expand(1, 2, 24, 16))
    # causal, Lq == Lk: row i averages keys 0..i (prefix means)
    prefix = v.cumsum(dim=2) / torch.arange(1, 25).view(1, 1, 24, 1)
    close(chunked.flash_torch(q, k, v, 0.9, True), prefix)


def test_bottom_right_causal_with_lq_lt_lk():
    # Lq=5, Lk=12: center = i + 7, so row 0 averages keys 0..7 when q = 0
    _, k, v = qkv(1, 1, 1, 5, 12, 8, seed=10)
    q = torch.zeros(1, 1, 5, 8)
    out = chunked.flash_torch(q, k, v, 1.0, True)
    for i in range(5):
        close(out[0, 0, i], v[0, 0, : i + 8].mean(0))


def test_causal_lq_gt_lk_zero_rows():
    q, k, v = qkv(1, 2, 2, 12, 5, 8, seed=11)
    out = chunked.flash_torch(q, k, v, 0.4, True)
    assert torch.count_nonzero(out[:, :, :7]) == 0  # rows i < Lq-Lk see no key
    assert not torch.isnan(out).any()
    close(out[:, :, 7], v[:, :, 0])  # row Lq-Lk sees key 0 only


@pytest.mark.parametrize("Lq,Lk", [(10, 10), (6, 14), (14, 6)])
def test_window_zero_zero_picks_the_diagonal_key(Lq, Lk):
    q, k, v = qkv(1, 2, 2, Lq, Lk, 8, seed=12)
    out = chunked.flash_torch(q, k, v, 0.5, False, window_left=0, window_right=0)
    for i in range(Lq):
        c = i + Lk - Lq
        if 0 <= c < Lk:
            close(out[:, :, i], v[:, :, c])
        else:
            assert torch.count_nonzero(out[:, :, i]) == 0


def test_window_one_zero_averages_two_keys():
    _, k, v = qkv(1, 1, 1, 9, 9, 8, seed=13)
    q = torch.zeros(1, 1, 9, 8)
    out = chunked.flash_torch(q, k, v, 1.0, False, window_left=1, window_right=0)
    close(out[0, 0, 0], v[0, 0, 0])
    for i in range(1, 9):
        close(out[0, 0, i], (v[0, 0, i - 1] + v[0, 0, i]) / 2)


def test_window_minus_one_zero_is_causal_and_wide_window_is_full():
    q, k, v = qkv(1, 2, 2, 20, 31, 16, seed=14)
    assert torch.equal(chunked.flash_torch(q, k, v, 0.3, False, window_left=-1, window_right=0),
                       chunked.flash_torch(q, k, v, 0.3, True))
    assert torch.equal(chunked.flash_torch(q, k, v, 0.3, False, window_left=1000, window_right=1000),
                       chunked.flash_torch(q, k, v, 0.3, False))


@pytest.mark.parametrize("Lq,Lk", [(12, 12), (7, 15), (15, 7)])
def test_alibi_huge_slope_selects_the_center_key(Lq, Lk):
    q, k, v = qkv(1, 2, 2, Lq, Lk, 8, seed=15)
    alibi = torch.full((2,), 1e3)
    out = chunked.flash_torch(q, k, v, 0.1, False, alibi=alibi)
    for i in range(Lq):
        c = i + Lk - Lq
        if 0 <= c < Lk:
            close(out[:, :, i], v[:, :, c], atol=1e-4)


def test_alibi_three_key_closed_form():
    # q = 0: weights of query 1 are exp(-s*|1-j|) -> (e^-s v0 + v1 + e^-s v2) / (1 + 2 e^-s)
    _, k, v = qkv(1, 1, 1, 3, 3, 4, seed=16)
    q = torch.zeros(1, 1, 3, 4)
    s = 0.7
    out = chunked.flash_torch(q, k, v, 1.0, False, alibi=torch.tensor([s]))
    e = math.exp(-s)
    close(out[0, 0, 1], (e * v[0, 0, 0] + v[0, 0, 1] + e * v[0, 0, 2]) / (1 + 2 * e))
    # query 0: exp(-s*j)
    w = torch.tensor([1.0, e, e * e])
    close(out[0, 0, 0], (w[:, None] * v[0, 0]).sum(0) / w.sum())


def test_alibi_zero_slopes_is_plain():
    q, k, v = qkv(2, 2, 2, 16, 16, 8, seed=17)
    close(chunked.flash_torch(q, k, v, 0.4, True, alibi=torch.zeros(4)), chunked.flash_torch(q, k, v, 0.4, True))


def test_softcap_limits():
    q, k, v = qkv(1, 2, 2, 16, 24, 16, seed=18, scale=2.0)
    # a huge cap is the identity on scores
    close(chunked.flash_torch(q, k, v, 0.5, False, softcap=1e7), chunked.flash_torch(q, k, v, 0.5, False),
          atol=1e-5)
    # a tiny cap squashes every score into [-c, c]: uniform weights
    close(chunked.flash_torch(q, k, v, 0.5, False, softcap=1e-7), v.mean(dim=2, keepdim=True).expand(1, 2, 16, 16))


def test_softcap_two_key_closed_form():
    q, k, v = qkv(1, 1, 1, 1, 2, 8, seed=19, scale=3.0)
    c, scale = 2.0, 0.6
    a = scale * float(q[0, 0, 0] @ k[0, 0, 0])
    b = scale * float(q[0, 0, 0] @ k[0, 0, 1])
    wa, wb = math.exp(c * math.tanh(a / c)), math.exp(c * math.tanh(b / c))
    expect = (wa * v[0, 0, 0] + wb * v[0, 0, 1]) / (wa + wb)
    close(chunked.flash_torch(q, k, v, scale, False, softcap=c)[0, 0, 0], expect)


def test_softcap_applies_before_alibi():
    # q = 0 makes every raw score 0; softcap(0) = 0, so only ALiBi remains:
    # if the cap were applied after ALiBi the bias itself would be squashed.
    _, k, v = qkv(1, 1, 1, 3, 3, 4, seed=20)
    q = torch.zeros(1, 1, 3, 4)
    with_cap = chunked.flash_torch(q, k, v, 1.0, False, softcap=0.01, alibi=torch.tensor([2.0]))
    no_cap = chunked.flash_torch(q, k, v, 1.0, False, alibi=torch.tensor([2.0]))
    close(with_cap, no_cap)


def test_chunking_is_invisible():
    q, k, v = qkv(1, 2, 2, 100, 77, 16, seed=21)
    a = chunked.flash_torch(q, k, v, 0.3, True, softcap=5.0, alibi=torch.tensor([0.1, 0.2]), chunk=13)
    b = chunked.flash_torch(q, k, v, 0.3, True, softcap=5.0, alibi=torch.tensor([0.1, 0.2]))
    close(a, b, atol=1e-6)


def test_row_subset_equals_full_rows():
    q, k, v = qkv(1, 2, 2, 100, 60, 16, seed=22)
    full = chunked.flash_torch(q, k, v, 0.3, True, chunk=32)
    part = chunked.flash_torch(q, k, v, 0.3, True, chunk=32, rows={64})
    assert torch.equal(part[:, :, 64:96], full[:, :, 64:96])
    assert torch.isnan(part[:, :, :64]).all()


def test_empty_keys_give_zero_rows():
    q = rnd(1, 2, 5, 8, seed=23)
    k = torch.zeros(1, 2, 0, 8)
    out = chunked.flash_torch(q, k, k, 0.3, False)
    assert out.shape == (1, 2, 5, 8) and torch.count_nonzero(out) == 0


def test_varlen_rows_equal_dense_per_sequence():
    lens_q, lens_k = [5, 0, 9, 3], [7, 4, 9, 0]
    g = torch.Generator().manual_seed(24)
    q = torch.randn(sum(lens_q), 4, 8, generator=g)
    k = torch.randn(sum(lens_k), 2, 8, generator=g)
    v = torch.randn(sum(lens_k), 2, 8, generator=g)
    cu_q = [0] + list(torch.tensor(lens_q).cumsum(0).tolist())
    cu_k = [0] + list(torch.tensor(lens_k).cumsum(0).tolist())
    out = chunked.flash_attn_varlen_func(q, k, v, torch.tensor(cu_q), torch.tensor(cu_k), causal=True)
    for i in range(4):
        qs, ks, vs = q[cu_q[i]:cu_q[i + 1]], k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]]
        if qs.shape[0] == 0:
            continue
        dense = stream.stream_fwd(qs.permute(1, 0, 2)[None], ks.permute(1, 0, 2)[None], vs.permute(1, 0, 2)[None],
                                  1 / math.sqrt(8), True)[0].permute(1, 0, 2)
        close(out[cu_q[i]:cu_q[i + 1]], dense)


def test_alibi_broadcast_shapes():
    assert torch.equal(chunked.broadcast_alibi(torch.tensor([1.0, 2.0]), 3, 2), torch.tensor([1.0, 2.0] * 3))
    bh = torch.arange(6.0).reshape(3, 2)
    assert torch.equal(chunked.broadcast_alibi(bh, 3, 2), torch.arange(6.0))
    with pytest.raises(ValueError):
        chunked.broadcast_alibi(torch.ones(3), 3, 2)


# ---- uneven value head dim (the reference SDPA patch's exact path) ----------

@pytest.mark.parametrize("d,dv", [(64, 32), (64, 128), (32, 200)])
@pytest.mark.parametrize("causal", [False, True])
def test_uneven_v_matches_sdpa(d, dv, causal):
    g = torch.Generator().manual_seed(d + dv)
    q = torch.randn(2, 3, 40, d, generator=g)
    k = torch.randn(2, 3, 40, d, generator=g)
    v = torch.randn(2, 3, 40, dv, generator=g)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    out = chunked.uneven_v_attention(q, k, v, is_causal=causal)
    assert out.shape == (2, 3, 40, dv)
    assert (out - ref).abs().max() < 2e-6


def test_uneven_v_top_left_causal_cross_length_and_masks():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 2, 24, 16, generator=g)
    k = torch.randn(1, 2, 56, 16, generator=g)
    v = torch.randn(1, 2, 56, 48, generator=g)
    # top-left causal: query i sees keys 0..i (torch SDPA's convention)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert (chunked.uneven_v_attention(q, k, v, is_causal=True) - ref).abs().max() < 2e-6
    mask = torch.rand(24, 56, generator=g) > 0.3
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    assert (chunked.uneven_v_attention(q, k, v, attn_mask=mask) - ref).abs().max() < 2e-6
    add = torch.randn(24, 56, generator=g)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=add)
    assert (chunked.uneven_v_attention(q, k, v, attn_mask=add) - ref).abs().max() < 2e-6


def test_uneven_v_single_key_and_gqa():
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 4, 5, 16, generator=g)
    k = torch.randn(1, 2, 1, 16, generator=g)
    v = torch.randn(1, 2, 1, 40, generator=g)
    out = chunked.uneven_v_attention(q, k, v, enable_gqa=True)
    # one key: every query gets that key's value row (its kv head's)
    assert torch.allclose(out, v.repeat_interleave(2, dim=1).expand(1, 4, 5, 40), atol=0)
    with pytest.raises(ValueError):
        chunked.uneven_v_attention(q, k, v)  # Hq != Hkv without enable_gqa


# --------------------------------------------------------------------------- softmax_lse, merge, paging
# The reference computes the softmax normaliser but never returns it; the
# oracle's lse (torch.logsumexp of the masked scores) is pinned against the
# float64 C statement's m + log(l) and against closed forms.


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
@pytest.mark.parametrize("shape", [(2, 4, 2, 33, 33, 16), (1, 4, 1, 45, 20, 24)], ids=["square-gqa", "lq>lk-mqa"])
def test_lse_matches_float64_stream(case, shape):
    B, Hq, Hkv, Lq, Lk, D = shape
    q, k, v = qkv(B, Hq, Hkv, Lq, Lk, D, seed=15)
    kw = dict(case)
    al = kw.pop("alibi", None)
    alibi = None
    if al is not None:
        alibi = chunked.broadcast_alibi(torch.linspace(0.05, 0.6, Hq).repeat(B, 1), B, Hq)
    out, lse = chunked.flash_torch(q, k, v, 0.3, alibi=alibi, return_lse=True, **kw)
    ref_out, ref_lse = stream.stream_fwd(q, k, v, 0.3, alibi=alibi, return_lse=True, **kw)
    assert torch.equal(torch.isinf(lse), torch.isinf(ref_lse))
    fin = torch.isfinite(ref_lse)
    close(lse[fin], ref_lse[fin])
    close(out, ref_out)


def test_lse_zero_query_is_log_of_the_valid_key_count():
    # q = 0: every valid score is 0, so lse = ln(number of valid keys)
    _, k, v = qkv(1, 2, 2, 5, 9, 8, seed=16)
    q = torch.zeros(1, 2, 5, 8)
    _, lse = chunked.flash_torch(q, k, v, 0.5, True, return_lse=True)
    counts = torch.arange(5) + 1 + (9 - 5)  # bottom-right causal: keys 0..i+4
    close(lse, torch.log(counts.double()).expand(1, 2, 5))
    _, lse = chunked.flash_torch(q, k, v, 0.5, True, window_left=2, return_lse=True)
    close(lse, torch.full((1, 2, 5), math.log(3.0)))


def test_lse_single_key_is_its_transformed_score():
    q, k, v = qkv(1, 1, 1, 4, 1, 16, seed=17)
    _, lse = chunked.flash_torch(q, k, v, 0.7, False, softcap=3.0, return_lse=True)
    s = 3.0 * torch.tanh((q[0, 0] @ k[0, 0].T).squeeze(-1) * 0.7 / 3.0)
    close(lse[0, 0], s)


def test_lse_of_rows_without_keys_is_minus_inf():
    q, k, v = qkv(1, 2, 2, 7, 3, 8, seed=18)
    out, lse = chunked.flash_torch(q, k, v, 0.5, True, return_lse=True)
    assert torch.isneginf(lse[:, :, :4]).all() and torch.isfinite(lse[:, :, 4:]).all()
    assert (out[:, :, :4] == 0).all()
    _, vl = chunked.flash_attn_varlen_func(torch.randn(3, 2, 8), torch.randn(0, 2, 8), torch.randn(0, 2, 8),
                                           torch.tensor([0, 3]), torch.tensor([0, 0]), return_lse=True)
    assert torch.isneginf(vl).all()


@pytest.mark.parametrize("softcap", [0.0, 2.0])
def test_merge_of_key_shards_equals_full_attention(softcap):
    import mtlflashattn_amd as mfa

    q, k, v = qkv(2, 4, 2, 6, 40, 16, seed=19)
    full, full_lse = chunked.flash_torch(q, k, v, 0.4, False, softcap=softcap, return_lse=True)
    parts = [chunked.flash_torch(q, k[:, :, a:b], v[:, :, a:b], 0.4, False, softcap=softcap, return_lse=True)
             for a, b in ((0, 13), (13, 14), (14, 40), (40, 40))]  # the last shard is empty
    # flash_torch is heads-second; the merge takes the heads-third output layout
    out, lse = mfa.merge_attention_partials([o.transpose(1, 2) for o, _ in parts], [l for _, l in parts])
    close(out.transpose(1, 2), full)
    close(lse, full_lse)
    out, lse = mfa.merge_attention_partials([parts[3][0].transpose(1, 2)], [parts[3][1]])
    assert (out == 0).all() and torch.isneginf(lse).all()


def test_gather_pages_follows_the_block_table():
    pool = (100 * torch.arange(4)[:, None] + torch.arange(4)[None, :]).float()[:, :, None, None].expand(4, 4, 1, 2)
    table = torch.tensor([[2, 0], [-1, -1], [1, 3]], dtype=torch.int32)  # row 1 has no keys: never read
    got = chunked.gather_pages(pool, table, [5, 0, 8])
    want = torch.tensor([200, 201, 202, 203, 0, 100, 101, 102, 103, 300, 301, 302, 303]).float()
    assert torch.equal(got[:, 0, 0], want) and torch.equal(got[:, 0, 1], want)


# --------------------------------------------------------------------------- gradients (backward oracle)
# The reference has no backward; the oracle's gradients are torch autograd
# through the same restated forward, pinned here against finite differences
# (torch.autograd.gradcheck, float64) and closed forms.

GRAD_CASES = [
    dict(),
    dict(causal=True),
    dict(causal=True, window_size=(2, 0)),
    dict(window_size=(1, 2)),
    dict(softcap=1.5),
    dict(alibi=True, causal=True),
    dict(softcap=3.0, alibi=True, window_size=(3, 1)),
]


@pytest.mark.parametrize("case", GRAD_CASES, ids=[str(i) for i in range(len(GRAD_CASES))])
@pytest.mark.parametrize("shape", [(1, 5, 7, 2, 1, 8), (2, 6, 4, 2, 2, 8)], ids=["lq<lk-mqa", "lq>lk"])
def test_gradients_match_finite_differences(case, shape):
    B, Lq, Lk, Hq, Hkv, D = shape
    g = torch.Generator().manual_seed(20)
    q = torch.randn(B, Lq, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Lk, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Lk, Hkv, D, generator=g, dtype=torch.float64)
    kw = dict(case)
    alibi = chunked.broadcast_alibi(torch.tensor([0.3, 0.7]).repeat(B, 1), B, Hq) if kw.pop("alibi", False) else None
    ws = kw.pop("window_size", (-1, -1))

    def f(q, k, v):
        return chunked.flash_torch(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), 0.4,
                                   kw.get("causal", False), kw.get("softcap", 0.0), ws[0], ws[1], alibi,
                                   grad=True, dtype=torch.float64)

    assert torch.autograd.gradcheck(f, tuple(t.requires_grad_(True) for t in (q, k, v)))


def test_gradients_of_a_single_key_and_of_masked_rows():
    # one key: out = v for every row, so dv = sum of dout over rows, dq = dk = 0
    q, k, v = qkv(1, 2, 2, 6, 1, 8, seed=21)
    dout = rnd(1, 6, 2, 8, seed=22)
    dq, dk, dv = chunked.attention_grads(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), dout)
    close(dq, torch.zeros_like(dq))
    close(dk, torch.zeros_like(dk))
    close(dv, dout.sum(dim=1, keepdim=True))
    # causal Lq > Lk: the first Lq - Lk rows see no key and get no gradient
    q, k, v = qkv(1, 2, 2, 7, 3, 8, seed=23)
    dout = rnd(1, 7, 2, 8, seed=24)
    dq, _, _ = chunked.attention_grads(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), dout, causal=True)
    assert (dq[:, :4] == 0).all() and (dq[:, 4:] != 0).any()


def test_fp32_gradients_agree_with_float64():
    q, k, v = qkv(1, 4, 2, 33, 40, 16, seed=25)
    dout = rnd(1, 33, 4, 16, seed=26)
    args = (q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), dout)
    g32 = chunked.attention_grads(*args, causal=True, softcap=5.0)
    g64 = chunked.attention_grads(*args, causal=True, softcap=5.0, dtype=torch.float64)
    for a, b in zip(g32, g64):
        close(a, b, atol=2e-5)


def test_lse_gradient_matches_finite_differences_and_closed_form():
    g = torch.Generator().manual_seed(27)
    q = torch.randn(1, 5, 2, 8, generator=g, dtype=torch.float64)
    k = torch.randn(1, 7, 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(1, 7, 2, 8, generator=g, dtype=torch.float64)

    def lse_of(q, k):
        return chunked.flash_torch(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), 0.4, True, grad=True,
                                   dtype=torch.float64, return_lse=True)[1]

    assert torch.autograd.gradcheck(lse_of, (q.clone().requires_grad_(True), k.clone().requires_grad_(True)))
    # d lse_i / d q_i = scale * sum_j P_ij k_j (P the row's softmax): with dout = 0, dlse = 1
    dq, _, _ = chunked.attention_grads(q, k, v, torch.zeros_like(q), softmax_scale=0.4, causal=True,
                                       dlse=torch.ones(1, 2, 5, dtype=torch.float64), dtype=torch.float64)
    s = torch.einsum("bihd,bjhd->bhij", q, k) * 0.4
    mask = torch.arange(7)[None, :] > (torch.arange(5)[:, None] + 2)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1)
    want = 0.4 * torch.einsum("bhij,bjhd->bihd", p, k)
    close(dq, want, atol=1e-10)


def test_varlen_gradients_match_finite_differences_and_sdpa():
    """oracle.chunked.attention_grads_varlen: a gradcheck (float64) of the
    packed varlen forward over a ragged batch (an empty query sequence, an
    empty key sequence, Lq != Lk, grouped-query heads), and per sequence the
    gradients torch's own SDPA autograd gives (causal rows with Lq == Lk,
    where SDPA's top-left causal equals bottom-right)."""
    import torch.nn.functional as F

    g = torch.Generator().manual_seed(31)
    lens_q, lens_k = [3, 0, 5, 2], [4, 3, 5, 0]
    Hq, Hkv, D = 4, 2, 8
    q = torch.randn(sum(lens_q), Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(sum(lens_k), Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(sum(lens_k), Hkv, D, generator=g, dtype=torch.float64)
    cu_q = torch.tensor([0] + lens_q).cumsum(0)
    cu_k = torch.tensor([0] + lens_k).cumsum(0)
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)

    def _varlen_f64(q, k, v):
        outs = []
        for i in range(len(lens_q)):
            a, b, c, d = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
            if b == a:
                continue
            if d == c:
                outs.append(torch.zeros(b - a, Hq, D, dtype=torch.float64))
                continue
            o = chunked.flash_torch(q[None, a:b].transpose(1, 2), k[None, c:d].transpose(1, 2),
                                    v[None, c:d].transpose(1, 2), 0.3, True, grad=True, dtype=torch.float64)
            outs.append(o[0].transpose(0, 1))
        return torch.cat(outs, dim=0)

    assert torch.autograd.gradcheck(_varlen_f64, tuple(t.clone().requires_grad_(True) for t in (q, k, v)))
    dq, dk, dv = chunked.attention_grads_varlen(q, k, v, dout, cu_q, cu_k, softmax_scale=0.3, causal=True,
                                                dtype=torch.float64)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    (_varlen_f64(qa, ka, va) * dout).sum().backward()
    close(dq, qa.grad, atol=1e-12)
    close(dk, ka.grad, atol=1e-12)
    close(dv, va.grad, atol=1e-12)
    # the one sequence with Lq == Lk (5 x 5) against torch SDPA's autograd
    a, b, c, d = cu_q[2], cu_q[3], cu_k[2], cu_k[3]
    qs, ks, vs = (t[None, x:y].transpose(1, 2).clone().requires_grad_(True)
                  for t, x, y in ((q, a, b), (k, c, d), (v, c, d)))
    out = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True, scale=0.3, enable_gqa=True)
    (out * dout[None, a:b].transpose(1, 2)).sum().backward()
    close(dq[a:b], qs.grad[0].transpose(0, 1), atol=1e-10)
    close(dk[c:d], ks.grad[0].transpose(0, 1), atol=1e-10)
    close(dv[c:d], vs.grad[0].transpose(0, 1), atol=1e-10)
    # sequence 0 (Lq = 3 < Lk = 4): bottom-right causal as an explicit SDPA mask
    a, b, c, d = cu_q[0], cu_q[1], cu_k[0], cu_k[1]
    qs, ks, vs = (t[None, x:y].transpose(1, 2).clone().requires_grad_(True)
                  for t, x, y in ((q, a, b), (k, c, d), (v, c, d)))
    mask = torch.arange(d - c)[None, :] <= torch.arange(b - a)[:, None] + ((d - c) - (b - a))
    out = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, scale=0.3, enable_gqa=True)
    (out * dout[None, a:b].transpose(1, 2)).sum().backward()
    close(dq[a:b], qs.grad[0].transpose(0, 1), atol=1e-10)
    close(dk[c:d], ks.grad[0].transpose(0, 1), atol=1e-10)
    close(dv[c:d], vs.grad[0].transpose(0, 1), atol=1e-10)
    # sequences without queries or keys get no gradient on their rows
    assert (dk[cu_k[1]:cu_k[2]] == 0).all() and (dv[cu_k[1]:cu_k[2]] == 0).all()
    assert (dq[cu_q[3]:cu_q[4]] == 0).all()
