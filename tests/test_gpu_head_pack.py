"""Tiles that pack the query heads of one K/V head (grouped-query calls with
2, 4 or 8 query heads per K/V head on the ping-pong tiles, 2 or 4 on the
4-wavefront tiles): the heads share a tile and its K/V stream, each over 1/R
of the tile's rows at the same positions.
GQA head mapping (metal_flash_attn/_kernel.py:54, hkv = hq / (Hq/Hkv)) must
stay bit-exact: every row equals the same call with K/V repeated per query
head (where each head has tiles of its own), outputs and lse alike, and
meets the oracle's bars; varlen sequences equal their dense calls, single-row
sequences of a mixed batch included."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import DEV, assert_output, assert_parity, default_scale, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

TILES = [_hip.MFA_TILE_256, _hip.MFA_TILE_PINGPONG, _hip.MFA_TILE_PINGPONG256]


@pytest.fixture(params=TILES, ids=["4wave", "pingpong", "pingpong256"])
def pp(request, monkeypatch):
    monkeypatch.setattr(_kernel, "_TILE_HINT", request.param)
    return request.param


def _kw(feat, B, Hq):
    kw = dict(feat)
    al = kw.pop("alibi", None)
    if al == "head":
        kw["alibi_slopes"] = torch.linspace(0.05, 0.6, Hq, device=DEV)
    elif al == "batch":
        kw["alibi_slopes"] = torch.rand(B, Hq, generator=torch.Generator().manual_seed(Hq)).to(DEV) * 0.5
    return kw


FEATURES = [
    dict(),
    dict(causal=True),
    dict(causal=True, window_size=(300, 0)),
    dict(window_size=(200, 77)),
    dict(softcap=10.0, alibi="head"),
    dict(causal=True, alibi="batch"),
]


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(8, 4), (16, 4), (16, 2)])
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
def test_equals_repeated_kv_heads(pp, D, hq, hkv, feat):
    B, L = 2, 700
    q, k, v = make_qkv(B, L, L, hq, hkv, D, torch.bfloat16, seed=hq + D)
    kw = _kw(feat, B, hq)
    out, lse = mfa.flash_attn_func_with_lse(q, k, v, **kw)
    r = hq // hkv
    rep, lse_rep = mfa.flash_attn_func_with_lse(q, k.repeat_interleave(r, 2), v.repeat_interleave(r, 2), **kw)
    assert torch.equal(out, rep), feat
    assert torch.equal(lse, lse_rep), feat
    ref, ref_lse = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), return_lse=True,
                                           **{x: (y.cpu() if torch.is_tensor(y) else y) for x, y in kw.items()})
    assert_output(out, ref, torch.bfloat16, f"head-packed {feat}")
    ws = kw.get("window_size", (-1, -1))
    out32 = _kernel.forward_bshd(q, k, v, default_scale(D), kw.get("causal", False), kw.get("softcap", 0.0), ws[0],
                                 ws[1], kw.get("alibi_slopes"), out_dtype=torch.float32)
    assert_parity(out32, ref, torch.bfloat16, f"head-packed fp32 out {feat}")
    fin = torch.isfinite(ref_lse)
    assert (lse.cpu()[fin] - ref_lse[fin]).abs().max().item() <= 4e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_sequences_equal_dense_calls(pp, dtype):
    # config 4's geometry in small: Hq=32, Hkv=8, D=128, causal, plus a
    # single-row sequence (computed by the exact-row kernel's launch with the
    # unpacked heads) and an empty one
    lens = [300, 1, 517, 0, 64, 1000]
    q, k, v, cu_q, cu_k = make_varlen(lens, lens, 32, 8, 128, dtype, seed=31)
    out, lse = mfa.flash_attn_varlen_func_with_lse(q, k, v, cu_q, cu_k, max(lens), max(lens), causal=True)
    starts = [0] + torch.tensor(lens).cumsum(0).tolist()
    for i, n in enumerate(lens):
        if n == 0:
            continue
        s, e = starts[i], starts[i + 1]
        d, dl = mfa.flash_attn_func_with_lse(q[None, s:e], k[None, s:e], v[None, s:e], causal=True)
        assert torch.equal(out[s:e], d[0]), i
        assert torch.equal(lse[:, s:e], dl[0]), i
    ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True)
    assert_output(out, ref, dtype, "head-packed varlen")


def test_launch_geometry():
    # 16 query heads over 4 K/V heads at D=128 on ping-pong tiles: 4 heads x
    # 64 positions per 256-row tile
    q = torch.empty(1, 4096, 16, 128, dtype=torch.bfloat16)
    k = torch.empty(1, 4096, 4, 128, dtype=torch.bfloat16)
    _kernel._TILE_HINT = _hip.MFA_TILE_PINGPONG
    try:
        info = _kernel.launch_info(q, k, k)
    finally:
        _kernel._TILE_HINT = _hip.MFA_TILE_AUTO
    assert info.kernel_name.startswith(b"mfa_fwd16pp<bf16,d128")
    assert info.grid_x == 4 * 4096 // 64  # K/V heads x position tiles


def test_launch_geometry_four_wave():
    # the same call on 4-wavefront tiles: 4 heads x 32 positions per 128-row
    # tile at D=128, 4 heads x 64 positions per 256-row tile at D=64
    _kernel._TILE_HINT = _hip.MFA_TILE_256
    try:
        for D, pos in ((128, 32), (64, 64)):
            q = torch.empty(1, 4096, 16, D, dtype=torch.bfloat16)
            k = torch.empty(1, 4096, 4, D, dtype=torch.bfloat16)
            info = _kernel.launch_info(q, k, k)
            assert info.kernel_name.startswith(b"mfa_fwd16<bf16,d%d" % D), info.kernel_name
            assert info.grid_x == 4 * 4096 // pos, (D, info.grid_x)
    finally:
        _kernel._TILE_HINT = _hip.MFA_TILE_AUTO
