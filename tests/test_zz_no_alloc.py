"""mfa_fwd_splitkv_static -- split-KV forward without a caller workspace (its
partials live in the library's static per-GPU scratch array) -- against
mfa_fwd_splitkv with a torch-allocated workspace, through the C ABI.

Both entry points run the same kernels with the same chunks, so their outputs
and log-sum-exps must be bit-identical; the oracle (the reference's
chunked-fp32 torch path) checks the numbers as well.  Two calls in a row, the
second on a smaller problem, show the shared scratch being reused; a call
whose workspace would exceed MFA_STATIC_SCRATCH_BYTES is rejected with a
message before any launch.
"""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from mtlflashattn_amd import _hip
from oracle import chunked
from gpu_util import REL_16, make_qkv

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 64 << 20  # MFA_STATIC_SCRATCH_BYTES in include/mfa.h


def params_bshd(q, k, v, o, causal=False, lse=None):
    """mfa_fwd_params for contiguous heads-third q/k/v/o (and a [B, Hq, Lq] lse)."""
    B, Lq, Hq, D = q.shape
    p = _hip.MfaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = q.stride()[:3]
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = k.stride()[:3]
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = v.stride()[:3]
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = o.stride()[:3]
    p.batch, p.heads_q, p.heads_kv = B, Hq, k.shape[2]
    p.seqlen_q, p.seqlen_k, p.head_dim = Lq, k.shape[1], D
    p.scale = 1.0 / math.sqrt(D)
    p.window_left = p.window_right = -1
    p.causal = int(causal)
    p.dtype_in = _hip.DTYPE_CODES[q.dtype]
    p.dtype_out = _hip.DTYPE_CODES[o.dtype]
    if lse is not None:
        p.softmax_lse = lse.data_ptr()
        p.lse_batch_stride, p.lse_head_stride = lse.stride(0), lse.stride(1)
    return p


def run_pair(B, Lq, Lk, Hq, Hkv, D, causal, seed):
    q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, torch.bfloat16, seed=seed)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for static in (True, False):
        o = torch.full((B, Lq, Hq, D), float("nan"), dtype=torch.float32, device="cuda")
        lse = torch.full((B, Hq, Lq), float("nan"), dtype=torch.float32, device="cuda")
        p = params_bshd(q, k, v, o, causal, lse)
        chunk = _hip.split_keys(p)
        assert chunk > 0, "the shape must take the split-KV path"
        nbytes = _hip.workspace_bytes(p, chunk)
        assert 0 < nbytes <= STATIC_SCRATCH_BYTES
        if static:
            _hip.fwd_splitkv_static(p, chunk, stream)
        else:
            ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
            _hip.fwd_splitkv(p, chunk, ws.data_ptr(), nbytes, stream)
        torch.cuda.synchronize()
        outs.append((o, lse, -(-Lk // chunk)))
    (o_s, lse_s, nch), (o_w, lse_w, _) = outs
    assert nch > 1
    assert torch.equal(o_s, o_w), "static-scratch output differs from the workspace entry point's"
    assert torch.equal(lse_s, lse_w), "static-scratch lse differs from the workspace entry point's"
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), causal=causal)
    err = (o_s.cpu() - ref).abs().max().item()
    assert err <= REL_16 * ref.abs().max().item(), f"err {err:.3e}"
    return nch, err


def test_static_scratch_matches_workspace_entry_point_twice():
    # first call: 5 chunks of 2048 keys, grouped-query heads, lse output
    n1, e1 = run_pair(B=2, Lq=4, Lk=9000, Hq=8, Hkv=2, D=128, causal=False, seed=31)
    # second call, smaller: 2 chunks, one query row (packed grouped-query decode
    # is off: Hq == Hkv), causal -- reuses the scratch the first call filled
    n2, e2 = run_pair(B=1, Lq=1, Lk=3000, Hq=4, Hkv=4, D=64, causal=True, seed=32)
    print(f"static scratch: {n1} chunks err {e1:.2e}; {n2} chunks err {e2:.2e}")


def test_static_scratch_rejects_an_oversized_call():
    # 64 x 64 units x 256 rows x 32 chunks of fp32 partials: far beyond the
    # scratch; rejected at planning time, so placeholder pointers never run
    p = _hip.MfaFwdParams()
    p.q = p.k = p.v = p.o = 256
    B, Lq, Lk, H, D = 64, 256, 65536, 64, 128
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = Lq * H * D, H * D, D
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = Lk * H * D, H * D, D
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = Lk * H * D, H * D, D
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = Lq * H * D, H * D, D
    p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim = B, H, H, Lq, Lk, D
    p.scale = 0.1
    p.window_left = p.window_right = -1
    p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[torch.bfloat16]
    assert _hip.workspace_bytes(p, 2048) > STATIC_SCRATCH_BYTES
    lib = _hip.load()
    rc = lib.mfa_fwd_splitkv_static(ctypes.byref(p), 2048, None)
    assert rc == _hip.MFA_ERR_INVALID
    assert b"static scratch" in lib.mfa_last_error()


@pytest.mark.parametrize("i", range(16))
def test_static_scratch_random_shapes(i):
    # seeded draws over batch, query rows, key length, grouped-query ratio,
    # head dim (padded and not), dtype, causal and chunk length (any multiple
    # of 64): every call reuses the scratch the previous one left behind
    import random
    rng = random.Random(7000 + i)
    B, Lq = rng.randint(1, 3), rng.choice([1, 2, 4, rng.randint(1, 64), rng.randint(1, 256)])
    Lk, Hkv = rng.randint(100, 20000), rng.choice([1, 2, 4])
    Hq, D = Hkv * rng.choice([1, 2, 4]), rng.choice([32, 40, 64, 96, 128])
    causal, chunk = rng.random() < 0.5, 64 * rng.randint(1, 64)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, dtype, seed=i)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for static in (True, False):
        o = torch.full((B, Lq, Hq, D), float("nan"), dtype=torch.float32, device="cuda")
        lse = torch.full((B, Hq, Lq), float("nan"), dtype=torch.float32, device="cuda")
        p = params_bshd(q, k, v, o, causal, lse)
        nbytes = _hip.workspace_bytes(p, chunk)
        if not 0 < nbytes <= STATIC_SCRATCH_BYTES:
            pytest.skip(f"workspace {nbytes} bytes is outside the static scratch")
        if static:
            _hip.fwd_splitkv_static(p, chunk, stream)
        else:
            ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
            _hip.fwd_splitkv(p, chunk, ws.data_ptr(), nbytes, stream)
        torch.cuda.synchronize()
        outs.append((o, lse))
    (o_s, lse_s), (o_w, lse_w) = outs
    what = f"case {i}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} causal={causal} chunk={chunk} {dtype}"
    assert torch.isfinite(o_s).all(), what
    assert torch.equal(o_s, o_w) and torch.equal(lse_s, lse_w), what
