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
from gpu_util import DEV, REL_16_OUT, make_qkv, max_err

pytestmark = pytest.mark.gpu


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
        assert max_err(a, ref) <= REL_16_OUT * ref.abs().max().item()
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
