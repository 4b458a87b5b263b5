"""Writes tests/golden/attn_cases.npz: small seeded attention cases and their
outputs from oracle/stream_ref.c (float64 two-pass restatement of the
reference's kernel math, metal_flash_attn/_kernel.py:32-87).

The reference repository holds no golden vectors (its tests compare against
a naive fp32 statement at run time), so these fixtures are regression anchors
produced by this build's pinned float64 oracle, not vectors taken from the
reference.  Inputs are bf16-representable so that 16-bit kernels see exactly
the same values.  Regenerate with: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import chunked, stream  # noqa: E402

CASES = [
    dict(name="plain", B=1, Hq=2, Hkv=2, Lq=33, Lk=33, D=16, scale=0.25, causal=False),
    dict(name="causal_cross_lq_lt_lk", B=1, Hq=2, Hkv=1, Lq=17, Lk=40, D=32, scale=0.2, causal=True),
    dict(name="causal_lq_gt_lk", B=2, Hq=2, Hkv=2, Lq=40, Lk=17, D=16, scale=0.3, causal=True),
    dict(name="window", B=1, Hq=4, Hkv=2, Lq=50, Lk=50, D=16, scale=0.25, causal=False, wl=6, wr=3),
    dict(name="softcap", B=1, Hq=2, Hkv=2, Lq=30, Lk=45, D=24, scale=0.5, causal=False, softcap=3.0),
    dict(name="alibi_batch", B=2, Hq=3, Hkv=3, Lq=25, Lk=25, D=8, scale=0.35, causal=True, alibi="batch"),
    dict(name="mix", B=1, Hq=4, Hkv=1, Lq=64, Lk=64, D=64, scale=0.125, causal=True, wl=20, softcap=5.0,
         alibi="head"),
]


def build_case(c, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(c["B"], c["Lq"], c["Hq"], c["D"], generator=g).bfloat16().float()
    k = torch.randn(c["B"], c["Lk"], c["Hkv"], c["D"], generator=g).bfloat16().float()
    v = torch.randn(c["B"], c["Lk"], c["Hkv"], c["D"], generator=g).bfloat16().float()
    slopes = None
    if c.get("alibi") == "head":
        slopes = torch.tensor([2 ** (-8 * (i + 1) / c["Hq"]) for i in range(c["Hq"])])
    elif c.get("alibi") == "batch":
        slopes = torch.rand(c["B"], c["Hq"], generator=g)
    return q, k, v, slopes


def main():
    arrays, meta = {}, []
    for i, c in enumerate(CASES):
        q, k, v, slopes = build_case(c, seed=100 + i)
        alibi = chunked.broadcast_alibi(slopes, c["B"], c["Hq"]) if slopes is not None else None
        out = stream.stream_fwd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), c["scale"], c["causal"],
                                c.get("softcap", 0.0), c.get("wl", -1), c.get("wr", -1), alibi).transpose(1, 2)
        n = c["name"]
        arrays[f"{n}.q"], arrays[f"{n}.k"], arrays[f"{n}.v"] = q.numpy(), k.numpy(), v.numpy()
        arrays[f"{n}.out"] = out.numpy()
        if slopes is not None:
            arrays[f"{n}.slopes"] = slopes.numpy()
        meta.append(c)
    np.savez_compressed(os.path.join(HERE, "attn_cases.npz"), **arrays)
    with open(os.path.join(HERE, "attn_cases.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(f"wrote {len(CASES)} cases")


if __name__ == "__main__":
    main()
