"""Head dim 128 calls that the automatic choice sends to the ping-pong tiles
because their key ranges are long: sliding windows of >= 1536 keys (512 on
packed grouped-query tiles) without a soft-cap / ALiBi transform, varlen calls whose longest sequence has >= 5
tiles (16 when causal) and dense rows of >= 2 tiles (8 when causal) -- of 256
rows, or of 256 / R positions when the tiles pack R = 2, 4 or 8 query heads
of one K/V head.  Each case checks the kernel the library picks
(launch_info / the plan's name) and the result against the oracle
(_kernel.py:1188-1207's mask order), in the fp32 parity
output and the 16-bit output; the 4-wavefront kernel on the same call meets
the same bars."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import DEV, assert_output, assert_parity, default_scale, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

DTYPES16 = [torch.bfloat16, torch.float16]


def _fp32_dense(q, k, v, causal, ws):
    return _kernel.forward_bshd(q, k, v, default_scale(q.shape[-1]), causal, 0.0, ws[0], ws[1], None,
                                out_dtype=torch.float32)


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("causal,ws,L,H,Hkv", [
    (False, (1024, 1023), 4096, 16, 16),  # 2048 keys wide, both sides
    (True, (2048, 0), 8192, 8, 8),        # causal sliding window
    (False, (2048, -1), 4096, 16, 16),    # left bound only
    (False, (768, 767), 4096, 16, 16),    # 1536 keys wide
    (False, (256, 256), 4096, 32, 8),     # packed grouped-query tiles: 513 keys wide
], ids=["both-sides", "causal", "left-only", "1536-wide", "packed-513-wide"])
def test_wide_windows_take_the_pingpong_tiles(dtype, causal, ws, L, H, Hkv, monkeypatch):
    q, k, v = make_qkv(1, L, L, H, Hkv, 128, dtype, seed=L + H + ws[0])
    info = _kernel.launch_info(q, k, v, causal=causal, window_left=ws[0], window_right=ws[1])
    assert info.kernel_name.startswith(b"mfa_fwd16pp<"), info.kernel_name
    kw = dict(causal=causal, window_size=ws)
    # the oracle on three 512-row chunks: the start (window not yet full),
    # the middle and the end
    starts = (0, L // 2, L - 512)
    sel = torch.cat([torch.arange(s0, s0 + 512) for s0 in starts])
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), chunk=512, rows=set(starts), **kw)[:, sel]
    assert_parity(_fp32_dense(q, k, v, causal, ws)[:, sel], ref, dtype, f"pp {ws} fp32 out")
    assert_output(mfa.flash_attn_func(q, k, v, **kw)[:, sel], ref, dtype, f"pp {ws}")
    monkeypatch.setattr(_kernel, "_TILE_HINT", _hip.MFA_TILE_256)  # the kernel these calls used before
    assert_output(mfa.flash_attn_func(q, k, v, **kw)[:, sel], ref, dtype, f"4-wave {ws}")


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("causal,B,L,H,Hkv", [(False, 32, 512, 8, 8), (True, 8, 2048, 4, 4), (False, 16, 512, 16, 4),
                                              (True, 8, 1536, 16, 4)],
                         ids=["2-tiles", "causal-8-tiles", "gqa4-512", "gqa4-causal-1536"])
def test_short_dense_rows_take_the_pingpong_tiles(dtype, causal, B, L, H, Hkv, monkeypatch):
    q, k, v = make_qkv(B, L, L, H, Hkv, 128, dtype, seed=B + L)
    info = _kernel.launch_info(q, k, v, causal=causal)
    assert info.kernel_name.startswith(b"mfa_fwd16pp<"), info.kernel_name
    sel = [0, B - 1]  # the oracle on the first and the last sequence
    ref = chunked.flash_attn_func(q[sel].cpu(), k[sel].cpu(), v[sel].cpu(), chunk=512, causal=causal)
    assert_parity(_fp32_dense(q, k, v, causal, (-1, -1))[sel], ref, dtype, "pp fp32 out")
    assert_output(mfa.flash_attn_func(q, k, v, causal=causal)[sel], ref, dtype, "pp")
    monkeypatch.setattr(_kernel, "_TILE_HINT", _hip.MFA_TILE_256)
    assert_output(mfa.flash_attn_func(q, k, v, causal=causal)[sel], ref, dtype, "4-wave")


@pytest.mark.parametrize("dtype", DTYPES16)
def test_long_varlen_non_causal_takes_the_pingpong_tiles(dtype, monkeypatch):
    lens = [3501, 2706, 3072, 400]  # longest: 14 tiles of 256 rows
    q, k, v, cu_q, cu_k = make_varlen(lens, lens, 8, 2, 128, dtype, seed=44)
    ran = []
    orig = _kernel._launch

    def spy(p, chunk, device):
        ran.append(_hip.launch_info(p).kernel_name)
        return orig(p, chunk, device)

    monkeypatch.setattr(_kernel, "_launch", spy)
    out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens), max(lens))
    assert ran and ran[-1].startswith(b"mfa_fwd16pp<"), ran
    ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu())
    assert_output(out, ref, dtype, "varlen non-causal (ping-pong)")
    out32 = _kernel.forward_varlen(q, k, v, cu_q, cu_k, max(lens), max(lens), default_scale(128), False,
                                   out_dtype=torch.float32)
    assert_parity(out32, ref, dtype, "varlen non-causal fp32 out")
    # causal: 4 query heads per K/V head pack into each ping-pong tile, so
    # the longest sequence has 55 tiles of 64 positions (>= 20): ping-pong
    ran.clear()
    outc = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens), max(lens), causal=True)
    assert ran and ran[-1].startswith(b"mfa_fwd16pp<"), ran
    refc = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True)
    assert_output(outc, refc, dtype, "varlen causal GQA (ping-pong)")
    # the same lengths with one query head per K/V head: 14 tiles of 256 rows
    # are below the causal threshold (16), so the 4-wavefront kernel
    qm, km, vm, _, _ = make_varlen(lens, lens, 4, 4, 128, dtype, seed=45)
    ran.clear()
    outm = mfa.flash_attn_varlen_func(qm, km, vm, cu_q, cu_k, max(lens), max(lens), causal=True)
    assert ran and ran[-1].startswith(b"mfa_fwd16<"), ran
    refm = chunked.flash_attn_varlen_func(qm.cpu(), km.cpu(), vm.cpu(), cu_q.cpu(), cu_k.cpu(), causal=True)
    assert_output(outm, refm, dtype, "varlen causal (4-wave)")
