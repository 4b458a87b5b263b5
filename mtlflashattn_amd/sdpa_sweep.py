"""Re-measure the SDPA patch's speed gate on this machine.

    python -m mtlflashattn_amd.sdpa_sweep [--lens 128,256,...] [--dims 64,128]

Times stock F.scaled_dot_product_attention against the HIP forward on the same
[B, H, L, D] inputs (median of 9 calls between HIP events, after 3 warm-up
calls) for fp16, bf16 and fp32, causal and not, and prints stock_ms, hip_ms and
their ratio.  The smallest length from which the HIP path is at least as fast
in every row is the value for MTLFLASHATTN_SDPA_FAST_MIN_SEQ (the defaults in
sdpa.py come from this sweep on MI355X).  Needs a ROCm GPU.
"""
from __future__ import annotations

import argparse
import math

import torch
import torch.nn.functional as F

from ._kernel import flash_attn_forward


def _median_ms(fn, warmup=3, reps=9):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sorted(a.elapsed_time(b) for a, b in evs)[reps // 2]


def sweep(lens=(128, 256, 512, 1024, 2048, 4096, 8192), dims=(64, 128),
          dtypes=(torch.bfloat16, torch.float16, torch.float32)):
    """Yield (dtype, D, causal, L, B, H, stock_ms, hip_ms) rows."""
    for dt in dtypes:
        for D in dims:
            for causal in (False, True):
                for L in lens:
                    B, H = (8, 16) if L <= 1024 else (1, 16)
                    g = torch.Generator().manual_seed(0)
                    q, k, v = (torch.randn(B, H, L, D, generator=g).to("cuda", dt) for _ in range(3))
                    stock = _median_ms(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal))
                    hip = _median_ms(lambda: flash_attn_forward(q, k, v, scale=1 / math.sqrt(D), causal=causal))
                    yield dt, D, causal, L, B, H, stock, hip


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--lens", default="128,256,512,1024,2048,4096,8192")
    ap.add_argument("--dims", default="64,128")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("sdpa_sweep needs a ROCm GPU")
    print("dtype     D   causal L      B  H   stock_ms  hip_ms  stock/hip")
    for dt, D, causal, L, B, H, ts, th in sweep([int(x) for x in args.lens.split(",")],
                                                [int(x) for x in args.dims.split(",")]):
        print(f"{str(dt)[6:]:9s} {D:3d} {int(causal)}      {L:6d} {B:2d} {H:3d} {ts:8.3f} {th:8.3f} {ts / th:6.2f}",
              flush=True)


if __name__ == "__main__":
    main()
