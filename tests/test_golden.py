"""Committed fixtures (tests/golden/attn_cases.npz, written by
tests/golden/make_golden.py from the float64 C restatement) against the
oracle on CPU and against the HIP kernels on the GPU."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import chunked

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
META = json.load(open(os.path.join(HERE, "attn_cases.json")))
DATA = np.load(os.path.join(HERE, "attn_cases.npz"))  # allow_pickle=False by default


def case(c):
    n = c["name"]
    q, k, v = (torch.from_numpy(DATA[f"{n}.{x}"]) for x in "qkv")
    slopes = torch.from_numpy(DATA[f"{n}.slopes"]) if f"{n}.slopes" in DATA else None
    out = torch.from_numpy(DATA[f"{n}.out"])
    return q, k, v, slopes, out


def kwargs(c, slopes):
    return dict(softmax_scale=c["scale"], causal=c["causal"], window_size=(c.get("wl", -1), c.get("wr", -1)),
                softcap=c.get("softcap", 0.0), alibi_slopes=slopes)


@pytest.mark.parametrize("c", META, ids=[c["name"] for c in META])
def test_oracle_matches_fixture(c):
    q, k, v, slopes, out = case(c)
    got = chunked.flash_attn_func(q, k, v, **kwargs(c, slopes))
    assert (got.double() - out).abs().max().item() <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("c", META, ids=[c["name"] for c in META])
def test_hip_matches_fixture(c, dtype):
    import mtlflashattn_amd as mfa
    from mtlflashattn_amd import _kernel

    q, k, v, slopes, out = case(c)
    qd, kd, vd = (x.to("cuda", dtype) for x in (q, k, v))
    kw = kwargs(c, slopes.cuda() if slopes is not None else None)
    got = mfa.flash_attn_func(qd, kd, vd, **kw)
    assert got.dtype == dtype
    if dtype == torch.float32:
        assert (got.double().cpu() - out).abs().max().item() <= 1e-5
    else:
        got32 = _kernel.forward_bshd(qd, kd, vd, c["scale"], c["causal"], kw["softcap"], *kw["window_size"],
                                     kw["alibi_slopes"], out_dtype=torch.float32)
        assert (got32.double().cpu() - out).abs().max().item() <= 2e-3 * out.abs().max().item()
