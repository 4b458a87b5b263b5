#!/usr/bin/env python
"""Benchmark of the BASELINE metric: attention forward effective TFLOP/s and %
of MI355X dense bf16 MFMA peak, on one GPU.

Default workload = BASELINE config 2 (the headline shape): bf16, B=1,
Lq=Lk=8192, H=16, D=64, non-causal, default scale, q/k/v ~ N(0,1) from seed 1
(the reference test recipe, tests/test_flash_attn_func.py:52-57).  One step =
one `flash_attn_func` forward over inputs already resident in HBM.

Prints ONE JSON line (rank 0).  Besides the driver's fields it carries
  roofline     : the dominant kernel's algorithmic FLOPs / its average launch
                 time (HIP events over the K back-to-back timed launches, on
                 the launch stream), against the dense bf16 MFMA peak
                 (2.5 PFLOP/s);
  cpu_baseline : the reference's chunked-fp32 torch path (oracle/chunked.py)
                 timed on this host's cores on a bounded sample of the same
                 workload (a subset of heads).
Before the W warm-up steps the step also runs untimed for --clock-warmup
seconds (default 1.0, declared in the line as clock_warmup_s/_steps) so that
the K timed steps see the steady-state shader clock.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2|3|4|5|6|7|8|9|10|11]
(6-10: HBM-bound short-L, decode and tiny-key shapes, roofline in GB/s against
8 TB/s; 8 runs split-KV; 11: the fp32 path against the 157.3 TFLOP/s fp32
MFMA peak)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "attn fwd effective TFLOP/s + % MFMA peak, bf16 H=16 D=64/128 L=8k, 1 MI355X"
PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp32": 157.3}  # MI355X dense MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
COPY_BYTES = 256 * 2**20  # calibration copy: bytes read = bytes written


def measured_traffic(cfg: int):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of this config.

    profiles/*_cfg<N>.md record FETCH_SIZE and WRITE_SIZE per dispatch, each
    scaled by what the same counter reads for a plain 256 MiB device copy
    (bench.py --copy-calibration), as `traffic_bytes_per_launch: <int>`.
    Returns None when no summary exists.
    """
    import glob
    import re

    for path in sorted(glob.glob(os.path.join(REPO, "profiles", f"mfa_fwd*_cfg{cfg}.md"))):
        m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", open(path).read(), re.M)
        if m:
            return int(m.group(1))
    return None


def make_config(cfg: int):
    import torch

    dev = "cuda"
    if cfg == 2:
        g = torch.Generator().manual_seed(1)
        B, L, H, D = 1, 8192, 16, 64
        q, k, v = (torch.randn(B, L, H, D, generator=g) for _ in range(3))
        q, k, v = (t.to(dev, torch.bfloat16) for t in (q, k, v))
        kw = dict(causal=False)
        pairs = B * H * L * L
        return dict(q=q, k=k, v=v, kw=kw, dtype="bf16", D=D, formula=4 * B * H * L * L * D,
                    algo=4 * pairs * D, varlen=None,
                    workload="cfg2: bf16 B=1 Lq=Lk=8192 H=16 D=64 non-causal, seed 1")
    if cfg == 3:
        g = torch.Generator().manual_seed(2)
        B, L, H, D = 1, 8192, 16, 128
        q, k, v = (torch.randn(B, L, H, D, generator=g) for _ in range(3))
        q, k, v = (t.to(dev, torch.float16) for t in (q, k, v))
        pairs = B * H * L * (L + 1) // 2
        return dict(q=q, k=k, v=v, kw=dict(causal=True), dtype="fp16", D=D, formula=4 * B * H * L * L * D // 2,
                    algo=4 * pairs * D, varlen=None,
                    workload="cfg3: fp16 B=1 Lq=Lk=8192 H=16 D=128 causal, seed 2")
    if cfg == 4:
        g = torch.Generator().manual_seed(3)
        lens = torch.randint(256, 4097, (8,), generator=g)
        T = int(lens.sum())
        q = torch.randn(T, 32, 128, generator=g).to(dev, torch.bfloat16)
        k = torch.randn(T, 8, 128, generator=g).to(dev, torch.bfloat16)
        v = torch.randn(T, 8, 128, generator=g).to(dev, torch.bfloat16)
        cu = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)]).to(torch.int32).to(dev)
        Ls = [int(x) for x in lens]
        pairs = sum(32 * L * (L + 1) // 2 for L in Ls)
        formula = sum(4 * 32 * L * L * 128 // 2 for L in Ls)
        return dict(q=q, k=k, v=v, kw=dict(causal=True), dtype="bf16", D=128, formula=formula,
                    algo=4 * pairs * 128, varlen=(cu, max(Ls)),
                    workload=f"cfg4: bf16 varlen lens={Ls} Hq=32 Hkv=8 D=128 causal, seed 3")
    if cfg == 5:
        g = torch.Generator().manual_seed(4)
        B, L, H, D = 1, 32768, 16, 128
        q, k, v = (torch.randn(B, L, H, D, generator=g) * 0.5 for _ in range(3))
        q, k, v = (t.to(dev, torch.bfloat16) for t in (q, k, v))
        slopes = torch.tensor([2 ** (-8 * (i + 1) / 16) for i in range(H)], dtype=torch.float32, device=dev)
        # valid pairs per head: keys j in [i-2048, i]
        pairs = B * H * sum(min(i, 2048) + 1 for i in range(L))
        return dict(q=q, k=k, v=v, kw=dict(causal=True, window_size=(2048, 0), softcap=30.0, alibi_slopes=slopes),
                    dtype="bf16", D=D, formula=4 * B * H * L * L * D // 2, algo=4 * pairs * D, varlen=None,
                    workload="cfg5: bf16 B=1 L=32768 H=16 D=128 causal window=(2048,0) softcap=30 ALiBi, seed 4")
    if cfg in (6, 7, 8):
        # not BASELINE configs: the short-L, HBM-bound shapes the metric asks
        # HBM GB/s for (6: short sequences, 7: one query row per sequence,
        # 8: one long decode row per head, run split-KV)
        g = torch.Generator().manual_seed(cfg)
        B, H, D = (64, 16, 64) if cfg != 8 else (1, 16, 128)
        Lq, Lk = {6: (256, 256), 7: (1, 4096), 8: (1, 131072)}[cfg]
        q = torch.randn(B, Lq, H, D, generator=g).to(dev, torch.bfloat16)
        k = torch.randn(B, Lk, H, D, generator=g).to(dev, torch.bfloat16)
        v = torch.randn(B, Lk, H, D, generator=g).to(dev, torch.bfloat16)
        pairs = B * H * Lq * Lk
        return dict(q=q, k=k, v=v, kw=dict(causal=False), dtype="bf16", D=D, formula=4 * pairs * D,
                    algo=4 * pairs * D, varlen=None, hbm_bytes=2 * (2 * B * Lq * H * D + 2 * B * Lk * H * D),
                    workload=f"cfg{cfg} (HBM-bound, not a BASELINE config): bf16 B={B} Lq={Lq} Lk={Lk} "
                             f"H={H} D={D} non-causal, seed {cfg}")
    if cfg == 9:
        # not a BASELINE config: single-row grouped-query decode (query heads
        # of a K/V head computed together; HBM-bound, roofline in GB/s)
        g = torch.Generator().manual_seed(9)
        B, Lk, Hq, Hkv, D = 64, 4096, 32, 8, 128
        q = torch.randn(B, 1, Hq, D, generator=g).to(dev, torch.bfloat16)
        k = torch.randn(B, Lk, Hkv, D, generator=g).to(dev, torch.bfloat16)
        v = torch.randn(B, Lk, Hkv, D, generator=g).to(dev, torch.bfloat16)
        pairs = B * Hq * Lk
        return dict(q=q, k=k, v=v, kw=dict(causal=True), dtype="bf16", D=D, formula=4 * pairs * D,
                    algo=4 * pairs * D, varlen=None, hbm_bytes=2 * (2 * B * Hq * D + 2 * B * Lk * Hkv * D),
                    workload=f"cfg9 (HBM-bound, not a BASELINE config): bf16 B={B} Lq=1 Lk={Lk} Hq={Hq} Hkv={Hkv} "
                             f"D={D} causal (grouped-query decode), seed 9")
    if cfg == 10:
        # not a BASELINE config: tiny-key cross-attention (image conditioning),
        # the shape of the reference's trace example (README.md:141-145:
        # bf16 D=128 Lq=26136 Lk=5); Q and O dominate the bytes (HBM-bound)
        g = torch.Generator().manual_seed(10)
        B, Lq, Lk, H, D = 1, 26136, 5, 16, 128
        q = torch.randn(B, Lq, H, D, generator=g).to(dev, torch.bfloat16)
        k = torch.randn(B, Lk, H, D, generator=g).to(dev, torch.bfloat16)
        v = torch.randn(B, Lk, H, D, generator=g).to(dev, torch.bfloat16)
        pairs = B * H * Lq * Lk
        return dict(q=q, k=k, v=v, kw=dict(causal=False), dtype="bf16", D=D, formula=4 * pairs * D,
                    algo=4 * pairs * D, varlen=None, hbm_bytes=2 * (2 * B * Lq * H * D + 2 * B * Lk * H * D),
                    workload=f"cfg10 (HBM-bound, not a BASELINE config): bf16 B={B} Lq={Lq} Lk={Lk} H={H} D={D} "
                             f"non-causal (tiny-key cross-attention), seed 10")
    if cfg == 11:
        # not a BASELINE config: the fp32 path (BASELINE config 1's dtype and
        # head dim, at the headline sequence length; MFMA-bound on the fp32
        # matrix cores, peak 157.3 TFLOP/s)
        g = torch.Generator().manual_seed(11)
        B, L, H, D = 1, 8192, 16, 64
        q, k, v = (torch.randn(B, L, H, D, generator=g).to(dev) for _ in range(3))
        pairs = B * H * L * L
        return dict(q=q, k=k, v=v, kw=dict(causal=False), dtype="fp32", D=D, formula=4 * pairs * D,
                    algo=4 * pairs * D, varlen=None,
                    workload="cfg11 (fp32 path, not a BASELINE config): fp32 B=1 Lq=Lk=8192 H=16 D=64 non-causal, "
                             "seed 11")
    raise SystemExit(f"unknown config {cfg}")


def run_step(c):
    import mtlflashattn_amd as mfa

    if c["varlen"] is not None:
        cu, mx = c["varlen"]
        return mfa.flash_attn_varlen_func(c["q"], c["k"], c["v"], cu, cu, mx, mx, **c["kw"])
    return mfa.flash_attn_func(c["q"], c["k"], c["v"], **c["kw"])


def cpu_model() -> str:
    """The host CPU's model name (the `Model name` lscpu prints, from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(cfg: int, budget_s: float = 12.0):
    """Oracle (reference chunked-fp32 torch path) on host cores, bounded sample."""
    import torch

    from oracle import chunked

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = make_config(cfg)
    if c["varlen"] is not None:
        # one sequence of the batch (the shortest), all heads
        cu, _ = c["varlen"]
        cu = cu.cpu().tolist()
        i = min(range(len(cu) - 1), key=lambda j: cu[j + 1] - cu[j])
        q, k, v = (t[cu[i]:cu[i + 1]].cpu() for t in (c["q"], c["k"], c["v"]))
        L = cu[i + 1] - cu[i]
        fn = lambda: chunked.flash_attn_varlen_func(q, k, v, [0, L], [0, L], causal=True)  # noqa: E731
        flops = 4 * 32 * L * L * 128 // 2
        sample = f"sequence {i} (L={L}) of the varlen batch, all 32 heads"
    else:
        q, k, v = (t.cpu() for t in (c["q"], c["k"], c["v"]))
        H = q.shape[2]
        heads = 1
        kw = {kk: (vv.cpu() if hasattr(vv, "cpu") else vv) for kk, vv in c["kw"].items()}
        t0 = time.perf_counter()
        rows = None
        if cfg == 5:
            rows = {q.shape[1] - 2048}  # last 2048-row chunk, full key range computed by the oracle
        chunked.flash_attn_func(q[:, :, :1], k[:, :, :1], v[:, :, :1], alibi_slopes=None if "alibi_slopes" not in kw
                                else kw["alibi_slopes"][:1], rows=rows,
                                **{kk: vv for kk, vv in kw.items() if kk != "alibi_slopes"})
        one = time.perf_counter() - t0
        heads = max(1, min(H, int(budget_s / 3 / max(one, 1e-3))))
        qs, ks, vs = q[:, :, :heads], k[:, :, :heads], v[:, :, :heads]
        kws = {kk: vv for kk, vv in kw.items() if kk != "alibi_slopes"}
        al = kw["alibi_slopes"][:heads] if "alibi_slopes" in kw else None
        fn = lambda: chunked.flash_attn_func(qs, ks, vs, alibi_slopes=al, rows=rows, **kws)  # noqa: E731
        Lq, Lk = q.shape[1], k.shape[1]
        nrows = 2048 if rows else Lq
        flops = 4 * heads * nrows * Lk * c["D"] // (2 if (c["kw"].get("causal") and not rows) else 1)
        sample = f"{heads} of {H} heads" + (", last 2048 query rows" if rows else ", all rows") + \
            f" (full Lq x Lk grid computed, as the reference torch path does)"
    fn()  # warm-up
    # timed runs until the budget is spent (at least 3), median reported
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": round(flops / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "model": cpu_model(), "sample": sample, "seconds": round(med, 3), "runs": len(times),
            "cpu_seconds_total": round(sum(times), 2),
            "note": f"formula FLOPs of the sample (4*H*Lq*Lk*D, halved for causal) / median of {len(times)} runs "
                    f"(timed runs repeat until {budget_s:.0f} s of CPU work)"}


def make_backward_step(c):
    """A closure running the HIP backward (dq, dk, dv) of config c's forward:
    out / lse / dout prepared once, outside the timed region."""
    import math

    import torch

    from mtlflashattn_amd import _kernel

    kw = c["kw"]
    scale = 1.0 / math.sqrt(c["D"])
    wl, wr = kw.get("window_size", (-1, -1))
    cfgk = dict(scale=scale, causal=kw.get("causal", False), softcap=kw.get("softcap", 0.0), window_left=wl,
                window_right=wr)
    g = torch.Generator().manual_seed(99)
    if c["varlen"] is not None:
        cu, mx = c["varlen"]
        out, lse = _kernel.forward_varlen(c["q"], c["k"], c["v"], cu, cu, mx, mx, return_lse=True, **cfgk)
        dout = torch.randn(out.shape, generator=g).to(out.device, out.dtype)
        q, k, v, o, d = (t[None] for t in (c["q"], c["k"], c["v"], out, dout))
        extra = dict(cu_q=cu, cu_k=cu, seqlen_q=mx, seqlen_k=mx)
    else:
        out, lse = _kernel.forward_bshd(c["q"], c["k"], c["v"], alibi_slopes=kw.get("alibi_slopes"),
                                        return_lse=True, **cfgk)
        dout = torch.randn(out.shape, generator=g).to(out.device, out.dtype)
        q, k, v, o, d = c["q"], c["k"], c["v"], out, dout
        extra = {}
    alibi, bstride = _kernel._alibi_arg(kw.get("alibi_slopes"), q.shape[0], q.shape[2], q.device)
    return lambda: _kernel._run_bwd(q, k, v, o, d, lse, alibi=alibi, alibi_bstride=bstride, **cfgk, **extra)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5, 6, 7, 8, 9, 10, 11],
                    help="BASELINE config 2-5 (default 2, the headline); 6-9 are HBM-bound short-L / decode "
                         "shapes (roofline in GB/s; 8 runs split-KV, 9 is grouped-query decode)")
    ap.add_argument("--clock-warmup", type=float, default=1.0,
                    help="seconds of untimed back-to-back steps before the W warm-up steps, so the timed steps "
                         "run at the steady-state shader clock (reported as clock_warmup_s / _steps)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--backward", action="store_true",
                    help="time the HIP backward (dq, dk, dv) of the config instead of the forward (configs 2-5; "
                         "effective TFLOP/s = 10*D FLOPs per valid pair; no CPU baseline)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after timing, run one plain 256 MiB device copy (rocprofv3 PMC calibration of "
                         "FETCH_SIZE / WRITE_SIZE against known bytes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "bench.py measures one GPU only: this build's path is single-GPU "
                                   "(head/sequence sharding across GPUs is a design note, not built); "
                                   f"--gpus {args.gpus} is not supported"}))
        sys.exit(2)

    import torch

    from mtlflashattn_amd import _kernel

    c = make_config(args.config)
    step = (lambda: run_step(c))
    if args.backward:
        if args.config not in (2, 3, 4, 5):
            raise SystemExit("--backward takes configs 2-5")
        step = make_backward_step(c)
        c = dict(c, formula=c["formula"] * 5 // 2, algo=c["algo"] * 5 // 2)
        args.no_cpu_baseline = True
    # Clock warm-up, untimed and declared in the output line: the shader
    # clock ramps up over the first ~0.1-0.5 s of load, so a few warm-up
    # steps alone would leave the timed steps running during the ramp.  The
    # same step runs back to back until `--clock-warmup` seconds of wall
    # time have passed; then the W warm-up steps and the K timed steps follow
    # unchanged.
    clock_steps = 0
    t_cw = time.perf_counter()
    while time.perf_counter() - t_cw < args.clock_warmup:
        for _ in range(8):
            step()
        clock_steps += 8
        torch.cuda.synchronize()
    clock_s = time.perf_counter() - t_cw
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    # whole-job timing: K back-to-back steps
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / args.steps
    # Kernel time per launch: the same HIP event pair over the K back-to-back
    # steps, on the stream the kernels are launched on.  The host queues the
    # steps faster than the GPU runs them, so the GPU runs the kernels back to
    # back and this is their average duration (plus the dispatch gap between
    # consecutive kernels).  A forward step is one launch; split-KV (config 8)
    # adds the merge kernel and --backward runs three kernels, whose sum this
    # is.  (Events bracketing each call separately would add the event
    # records' own cost to every launch.)
    kernel_ms = ms_step

    value = c["formula"] / (ms_step / 1e3) / 1e12
    peak = PEAK_TFLOPS[c["dtype"]]
    achieved = c["algo"] / (kernel_ms / 1e3) / 1e12
    if args.backward:
        # (the eight-wavefront dK/dV kernel above head dim 64; GQA adds the partial-sum kernel)
        dkdv = "mfa_bwd_dkdv8" if c["D"] > 64 else "mfa_bwd_dkdv"
        grouped = c["q"].shape[-2] != c["k"].shape[-2]
        kname = f"mfa_bwd_dsum + {dkdv}" + (" + mfa_bwd_dkdv_sum" if grouped else "") + " + mfa_bwd_dq"
    elif c["varlen"] is not None:
        cu, mx = c["varlen"]
        info = _kernel.launch_info_varlen(c["q"], c["k"], cu.shape[0] - 1, mx, mx, causal=c["kw"].get("causal", False))
        kname = info.kernel_name.decode() + " (varlen)"
    else:
        info = _kernel.launch_info(c["q"], c["k"], c["v"], causal=c["kw"].get("causal", False),
                                   softcap=c["kw"].get("softcap", 0.0),
                                   alibi="alibi_slopes" in c["kw"],
                                   window_left=c["kw"].get("window_size", (-1, -1))[0],
                                   window_right=c["kw"].get("window_size", (-1, -1))[1])
        kname = info.kernel_name.decode()
        chunk = _kernel.split_chunk(c["q"], c["k"])
        if chunk:
            kname += f" split-KV {chunk} keys + mfa_combine"
    traffic = None if args.backward else measured_traffic(args.config)
    line = {
        "metric": METRIC if not args.backward else "attn bwd effective TFLOP/s (10*D FLOPs per valid pair)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_s": round(clock_s, 3),
        "clock_warmup_steps": clock_steps,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": c["dtype"],
        "data": "synthetic (seeded randn, reference recipe)",
        "config": {"workload": c["workload"], "pct_mfma_peak": round(100 * value / peak, 2),
                   "formula_flops": c["formula"], "algorithmic_flops": c["algo"]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": kname,
                     "kernel_ms": round(kernel_ms, 4),
                     "note": f"algorithmic FLOPs ({'10' if args.backward else '4'}*D per valid (query,key) pair) "
                             "/ mean launch time (HIP events over the K back-to-back timed launches)"},
    }
    if "hbm_bytes" in c:
        gbs = c["hbm_bytes"] / (kernel_ms / 1e3) / 1e9
        line["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": kname,
                            "kernel_ms": round(kernel_ms, 4), "algorithmic_bytes": c["hbm_bytes"],
                            "note": "algorithmic bytes (Q + K + V + O, each once) / mean launch time "
                                    "(HIP events over the K back-to-back timed launches)"}
    if args.copy_calibration:
        x = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.config)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
