"""fp32 inputs with a soft-cap / ALiBi transform, against exact float64 math.

The fp32 kernel evaluates the soft-cap with a tanh accurate to 2 ulp and
ALiBi as -slope * (|center - j| - dmin), dmin the row's smallest distance to a
valid key (a per-row constant: the softmax is unchanged, the lse adds
-slope * dmin back), so a row hundreds of keys from every key keeps its
scores near zero.  The reference's chunked fp32 path (_kernel.py:1188-1207)
subtracts slope * |center - j| itself: such rows then hold scores near -10^2,
where fp32 spacing is ~1e-5, and that path is up to ~2e-5 from the exact
result there.  The bars: the kernel within the fp32 bar (1e-5) of the float64
restatement (oracle/stream_ref.c), and within the bar plus the oracle's own
distance to float64 of the chunked oracle."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from oracle import chunked
from oracle.stream import stream_fwd
from gpu_util import DEV, make_qkv

pytestmark = pytest.mark.gpu

BAR = 1e-5
SHAPES = [(481, 52), (700, 700), (300, 1200), (1, 900)]  # Lq, Lk (bottom-right centers)
FEATURES = [
    dict(),
    dict(softcap=20.0),
    dict(causal=True),
    dict(window_size=(400, 100)),
    dict(causal=True, softcap=3.0),
]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
def test_fp32_alibi_against_float64(d, shape, feat):
    Lq, Lk = shape
    H, Hkv = 4, 2
    q, k, v = make_qkv(2, Lq, Lk, H, Hkv, d, torch.float32, seed=Lq + Lk + d)
    slopes = torch.tensor([[0.45, 0.3, 0.2, 0.05], [0.5, 0.25, 0.125, 0.0625]], device=DEV)  # [B, Hq]
    kw = dict(feat, alibi_slopes=slopes)
    out, lse = mfa.flash_attn_func_with_lse(q, k, v, **kw)
    ws = kw.get("window_size", (-1, -1))
    exact, exact_lse = stream_fwd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), d ** -0.5,
                                  kw.get("causal", False), kw.get("softcap", 0.0), ws[0], ws[1],
                                  alibi=slopes.reshape(-1), return_lse=True)
    exact = exact.transpose(1, 2)
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), **{x: (y.cpu() if torch.is_tensor(y) else y)
                                                                for x, y in kw.items()})
    e_exact = (out.cpu().double() - exact).abs().max().item()
    e_oracle = (out.cpu() - ref).abs().max().item()
    oracle_own = (ref.double() - exact).abs().max().item()
    assert e_exact <= BAR, f"{shape} {feat}: kernel vs float64 {e_exact:.3e}"
    assert e_oracle <= BAR + oracle_own, f"{shape} {feat}: kernel vs oracle {e_oracle:.3e} (oracle vs float64 {oracle_own:.3e})"
    fin = torch.isfinite(exact_lse)
    assert torch.equal(torch.isneginf(lse.cpu()), torch.isneginf(exact_lse))
    if fin.any():
        lerr = (lse.cpu().double() - exact_lse)[fin].abs().max().item()
        assert lerr <= BAR * max(1.0, exact_lse[fin].abs().max().item()), f"{shape} {feat}: lse {lerr:.3e}"
