"""Fixed-seed random sweep of the backward pass through autograd: shapes,
head dims, GQA ratios, dense and varlen (empty sequences, single keys),
causal, windows, soft-cap, ALiBi, small and negative scales, against the
oracle's autograd gradients (oracle.chunked.attention_grads[_varlen]).

Bar: the bf16/fp16 gradients of test_gpu_backward (2 * GRAD_REL of the
gradient's scale).  The scale is max|ref grad|, floored at 1e-3 of |dout| *
|v| (the size of a gradient that does not vanish): dQ and dK vanish exactly
when every row sees a single key (P = 1), and the kernel's dS = P * (dP -
Dsum) then holds the rounding of the 16-bit forward output that Dsum is
built from (measured up to 9.4e-6 against a natural scale of ~10)."""
from __future__ import annotations

import random

import pytest
import torch

import mtlflashattn_amd as mfa
from oracle import chunked
from gpu_util import DEV, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

GRAD_REL = {torch.bfloat16: 6e-3, torch.float16: 1.5e-3}
CASES = 80


def _draw(i):
    rng = random.Random(5000 + i)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    D = rng.choice([8, 16, 32, 40, 64, 64, 96, 128, 128])
    Hkv = rng.choice([1, 2, 4])
    Hq = Hkv * rng.choice([1, 1, 2, 4])
    kw = {}
    if rng.random() < 0.5:
        kw["causal"] = True
    if rng.random() < 0.2:
        kw["window_size"] = (rng.choice([0, 5, 64, 300]), rng.choice([-1, 0, 7, 100]))
    if rng.random() < 0.25:
        kw["softcap"] = rng.choice([3.0, 20.0])
    if rng.random() < 0.25:
        kw["alibi_slopes"] = [rng.uniform(0.0, 0.5) for _ in range(Hq)]
    if rng.random() < 0.1:
        kw["softmax_scale"] = rng.choice([0.05, 0.3, -0.1])
    if rng.random() < 0.3:
        nb = rng.randint(1, 3)
        shape = ("varlen", [rng.choice([0, 1, rng.randint(1, 40), rng.randint(1, 300)]) for _ in range(nb)],
                 [rng.choice([0, 1, rng.randint(1, 70), rng.randint(1, 400)]) for _ in range(nb)])
    else:
        shape = ("dense", rng.randint(1, 2), rng.choice([1, rng.randint(1, 64), rng.randint(1, 400)]),
                 rng.choice([1, rng.randint(1, 64), rng.randint(1, 500)]))
    return dtype, D, Hq, Hkv, kw, shape


@pytest.mark.parametrize("i", range(CASES))
def test_random_grads(i):
    dtype, D, Hq, Hkv, kw, shape = _draw(i)
    if "alibi_slopes" in kw:
        kw["alibi_slopes"] = torch.tensor(kw["alibi_slopes"], device=DEV)
    al = kw["alibi_slopes"].cpu() if "alibi_slopes" in kw else None
    if shape[0] == "varlen":
        _, lq, lk = shape
        q, k, v, cu_q, cu_k = make_varlen(lq, lk, Hq, Hkv, D, dtype, seed=i)
        fn = lambda q, k, v: mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lq + [1]), max(lk + [1]), **kw)  # noqa: E731
    else:
        _, B, Lq, Lk = shape
        q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, dtype, seed=i)
        fn = lambda q, k, v: mfa.flash_attn_func(q, k, v, **kw)  # noqa: E731
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(i)).to(DEV, dtype)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    fn(qq, kk, vv).backward(dout)
    args = (kw.get("softmax_scale"), kw.get("causal", False), kw.get("window_size", (-1, -1)), kw.get("softcap", 0.0), al)
    if shape[0] == "varlen":
        ref = chunked.attention_grads_varlen(q, k, v, dout, cu_q.cpu(), cu_k.cpu(), *args)
    else:
        ref = chunked.attention_grads(q, k, v, dout, *args)
    natural = dout.float().abs().max().item() * v.float().abs().max().item() if v.numel() and dout.numel() else 1.0
    for name, g, r in zip(("dq", "dk", "dv"), (qq.grad, kk.grad, vv.grad), ref):
        if r.numel() == 0:
            continue
        assert torch.isfinite(g).all(), f"case {i} {name}"
        scale = max(r.float().abs().max().item(), 1e-3 * natural)
        err = (g.detach().float().cpu() - r.float()).abs().max().item()
        assert err <= 2 * GRAD_REL[dtype] * scale, f"case {i} {name}: {err:.3e} > {2 * GRAD_REL[dtype]:.1e} * {scale:.3e} {dtype} D={D} {shape} {sorted(kw)}"
