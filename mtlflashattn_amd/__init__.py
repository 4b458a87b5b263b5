"""MI355X-native flash-attention forward for PyTorch-ROCm -- CUDA flash-attn API surface.

Drop-in for mtlflashattn's public API (metal_flash_attn/__init__.py): the same
six functions, argument meanings and error contract.  Unsupported features
raise NotImplementedError so callers can fall back, rather than silently
approximating (metal_flash_attn/__init__.py:1-5).

Backward: the reference is inference-only (metal_flash_attn/__init__.py:3-4).
Here calls whose inputs require grad are differentiable through HIP
backward kernels (dq, dk, dv; the returned lse too): bf16/fp16 on the matrix
cores, fp32 in fp32 on the vector ALU.  Paged K/V stay forward-only: their
backward raises NotImplementedError, as do dropout_p > 0, deterministic=True
and return_attn_probs=True.

Two additions the reference raises for: `flash_attn_varlen_func` accepts a
paged K/V cache (`block_table`, CUDA flash-attn's layout), and
`flash_attn_func_with_lse` / `flash_attn_varlen_func_with_lse` also return the
softmax log-sum-exp, which `merge_attention_partials` uses to combine attention
over disjoint key sets (context-parallel shards, cache + new tokens).

Every call runs the gfx950 HIP kernels of libmtlfa_hip.so on the tensors'
ROCm device; there is no CPU path.
"""
from __future__ import annotations

import math
import os

import torch

from . import _kernel
from ._kernel import MAX_HEAD_DIM, flash_attn_forward, forward_bshd, forward_varlen
from ._version import __version__

__all__ = [
    "flash_attn_func",
    "flash_attn_varlen_func",
    "flash_attn_qkvpacked_func",
    "flash_attn_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func",
    "flash_attn_varlen_kvpacked_func",
    "flash_attn_forward",
    "flash_attn_func_with_lse",
    "flash_attn_varlen_func_with_lse",
    "merge_attention_partials",
    "__version__",
]

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _check_supported(q, k, v, dropout_p, window_size, softcap, alibi_slopes, deterministic, return_attn_probs):
    """Error contract of metal_flash_attn/__init__.py:28-59, checked in the same order."""
    if dropout_p:
        raise NotImplementedError("mtlflashattn_amd: dropout_p > 0 not supported (inference-only)")
    if (
        not isinstance(window_size, (tuple, list))
        or len(window_size) != 2
        or any(not isinstance(w, int) or isinstance(w, bool) or w < -1 for w in window_size)
    ):
        raise ValueError(
            "mtlflashattn_amd: window_size must be a (left, right) pair of ints >= -1 "
            "(-1 = unbounded on that side)"
        )
    if softcap < 0:
        raise ValueError("mtlflashattn_amd: softcap must be >= 0 (0 disables capping)")
    if alibi_slopes is not None and not torch.is_tensor(alibi_slopes):
        raise TypeError("mtlflashattn_amd: alibi_slopes must be a tensor of per-head slopes")
    if deterministic:
        raise NotImplementedError("mtlflashattn_amd: deterministic not supported")
    if return_attn_probs:
        raise NotImplementedError("mtlflashattn_amd: return_attn_probs not supported (probs never materialized)")
    if not _kernel._is_rocm_tensor(q):
        raise NotImplementedError(f"mtlflashattn_amd: device {q.device.type!r} not supported (ROCm GPU only)")
    if q.dtype not in _SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise NotImplementedError(f"mtlflashattn_amd: dtype {q.dtype} (q/k/v must match, fp16/bf16/fp32)")
    D = q.shape[-1]
    if D > MAX_HEAD_DIM:
        raise NotImplementedError(f"mtlflashattn_amd: head_dim {D} > {MAX_HEAD_DIM}")
    if k.shape[-1] != D or v.shape[-1] != D:
        raise ValueError("mtlflashattn_amd: q/k/v head_dim mismatch")


def flash_attn_func(
    q,
    k,
    v,
    dropout_p=0.0,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    alibi_slopes=None,
    deterministic=False,
    return_attn_probs=False,
):
    """Drop-in for flash_attn.flash_attn_func (forward only; metal_flash_attn/__init__.py:62-99).

    q: [B, Lq, Hq, D]; k, v: [B, Lk, Hkv, D] (heads-third, CUDA flash-attn layout).
    Hkv must divide Hq (GQA/MQA). Returns [B, Lq, Hq, D] in q.dtype.
    """
    _check_supported(q, k, v, dropout_p, window_size, softcap, alibi_slopes, deterministic, return_attn_probs)
    return _dense(q, k, v, softmax_scale, causal, window_size, softcap, alibi_slopes, False)


def flash_attn_func_with_lse(q, k, v, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                             alibi_slopes=None):
    """flash_attn_func that also returns the softmax log-sum-exp.

    Returns (out [B, Lq, Hq, D] in q.dtype, softmax_lse [B, Hq, Lq] fp32):
    lse = ln(sum_j exp(s_j)) over each row's valid keys (s the scaled,
    soft-capped, ALiBi-biased score; CUDA flash-attn's softmax_lse), -inf for a
    row with no valid key.  Same arguments and errors as flash_attn_func; the
    reference has no counterpart (its return_attn_probs raises,
    metal_flash_attn/__init__.py:49-50).
    """
    _check_supported(q, k, v, 0.0, window_size, softcap, alibi_slopes, False, False)
    return _dense(q, k, v, softmax_scale, causal, window_size, softcap, alibi_slopes, True)


def _dense(q, k, v, softmax_scale, causal, window_size, softcap, alibi_slopes, return_lse):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"mtlflashattn_amd: expected 4-D [B,S,H,D] tensors, got q.dim()={q.dim()}")
    _kernel._check_qkv_shapes(q, k, v, h_axis=2, s_axis=1)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    return forward_bshd(
        q, k, v, scale=scale, causal=causal, softcap=softcap,
        window_left=window_size[0], window_right=window_size[1], alibi_slopes=alibi_slopes, return_lse=return_lse,
    )


def flash_attn_varlen_func(
    q,
    k,
    v,
    cu_seqlens_q,
    cu_seqlens_k,
    max_seqlen_q,
    max_seqlen_k,
    dropout_p=0.0,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    alibi_slopes=None,
    deterministic=False,
    return_attn_probs=False,
    block_table=None,
):
    """Drop-in for flash_attn.flash_attn_varlen_func (forward only; metal_flash_attn/__init__.py:102-183).

    q: [total_q, Hq, D]; k, v: [total_k, Hkv, D] packed without padding;
    cu_seqlens_*: [B+1] int32 cumulative sequence lengths.
    Returns [total_q, Hq, D] in q.dtype.  All sequences run in one launch.

    block_table (paged K/V cache, CUDA flash-attn's layout; the reference
    raises NotImplementedError, metal_flash_attn/__init__.py:130-131): int32
    [B, max_pages]; k, v are then page pools [num_pages, page_block_size, Hkv,
    D] with page_block_size a multiple of 256, key j of sequence b is row
    j % page_block_size of page block_table[b, j // page_block_size], and
    cu_seqlens_k gives the key counts only.  Page ids are read on the device;
    an id outside [0, num_pages) reads zero keys and values without faulting,
    but those keys are not masked (they score 0 and dilute the softmax), so
    the rows that see them are wrong; MTLFLASHATTN_CHECK_PAGES=1 checks the
    ids on the host and raises ValueError instead.
    """
    _check_supported(q, k, v, dropout_p, window_size, softcap, alibi_slopes, deterministic, return_attn_probs)
    return _varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale, causal, window_size, softcap, alibi_slopes,
                   block_table, False)


def flash_attn_varlen_func_with_lse(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                    softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                                    alibi_slopes=None, block_table=None):
    """flash_attn_varlen_func that also returns the softmax log-sum-exp.

    Returns (out [total_q, Hq, D] in q.dtype, softmax_lse [Hq, total_q] fp32,
    CUDA flash-attn's varlen layout); lse as in flash_attn_func_with_lse.
    """
    _check_supported(q, k, v, 0.0, window_size, softcap, alibi_slopes, False, False)
    return _varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale, causal, window_size, softcap, alibi_slopes,
                   block_table, True)


def _varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale, causal, window_size, softcap, alibi_slopes,
            block_table, return_lse):
    paged = block_table is not None
    if q.dim() != 3 or k.dim() != (4 if paged else 3) or v.dim() != (4 if paged else 3):
        if paged:
            raise ValueError("mtlflashattn_amd: with block_table, q must be [total,H,D] and k/v "
                             "[num_pages,page_block_size,H,D]")
        raise ValueError(f"mtlflashattn_amd: expected 3-D [total,H,D] tensors, got q.dim()={q.dim()}")
    if cu_seqlens_q.shape[0] != cu_seqlens_k.shape[0]:
        raise ValueError(
            f"mtlflashattn_amd: cu_seqlens_q ({cu_seqlens_q.shape[0]}) and "
            f"cu_seqlens_k ({cu_seqlens_k.shape[0]}) imply different batch sizes"
        )
    Hq, Hkv = q.shape[1], k.shape[-2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"mtlflashattn_amd: num_heads_kv ({Hkv}) must divide num_heads_q ({Hq})")
    if k.shape[:-1] != v.shape[:-1]:
        raise ValueError("mtlflashattn_amd: k/v total token count mismatch")
    if paged:
        page = k.shape[1]
        if not torch.is_tensor(block_table) or block_table.dim() != 2 or block_table.dtype != torch.int32:
            raise ValueError("mtlflashattn_amd: block_table must be an int32 [batch, max_pages] tensor")
        if block_table.shape[0] != cu_seqlens_q.shape[0] - 1:
            raise ValueError(f"mtlflashattn_amd: block_table has {block_table.shape[0]} rows for "
                             f"{cu_seqlens_q.shape[0] - 1} sequences")
        if page == 0 or page % 256 != 0:
            raise ValueError(f"mtlflashattn_amd: page_block_size {page} must be a positive multiple of 256")

    # The prefix sums on the host (the reference reads them for the same
    # checks, metal_flash_attn/__init__.py:145-154); they also yield the true
    # longest lengths, so a too-small max_seqlen_* cannot drop rows.
    cu_q, cu_k = _host_prefix_sums(cu_seqlens_q, cu_seqlens_k)
    if cu_q[-1] != q.shape[0]:
        raise ValueError(f"mtlflashattn_amd: cu_seqlens_q[-1]={cu_q[-1]} != total_q={q.shape[0]}")
    if not paged and cu_k[-1] != k.shape[0]:
        raise ValueError(f"mtlflashattn_amd: cu_seqlens_k[-1]={cu_k[-1]} != total_k={k.shape[0]}")
    lens_q = [b - a for a, b in zip(cu_q[:-1], cu_q[1:])]
    lens_k = [b - a for a, b in zip(cu_k[:-1], cu_k[1:])]
    if any(x < 0 for x in lens_q) or any(x < 0 for x in lens_k) or cu_q[0] != 0 or cu_k[0] != 0:
        raise ValueError("mtlflashattn_amd: cu_seqlens must be non-decreasing prefix sums starting at 0")
    if paged:
        _check_block_table(block_table, lens_k, k.shape[1], k.shape[0])

    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    # (with no sequence of exactly one query row, the launch for such rows is skipped)
    return forward_varlen(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max(lens_q, default=0), max(lens_k, default=0),
        scale=scale, causal=causal, softcap=softcap, window_left=window_size[0],
        window_right=window_size[1], alibi_slopes=alibi_slopes, return_lse=return_lse, block_table=block_table,
        no_single_rows=1 not in lens_q,
    )


# Host copies of the last varlen call's prefix sums, with the two tensors
# they were read from and their version counters.  Reading them is a
# device-to-host copy that waits for all queued GPU work, so a loop of calls
# on the same cu_seqlens would leave the GPU idle between calls; the copy is
# reused while the same tensor objects come back with unchanged versions
# (PyTorch moves a tensor's version on every in-place write through it or
# through a view of it).  Writes that bypass the counter (through `.data`,
# or by another library through the raw pointer) are not seen: such a
# tensor must not be passed again.
_cu_host = None


def _host_prefix_sums(cu_seqlens_q, cu_seqlens_k):
    global _cu_host
    cached = _cu_host
    try:
        versions = (cu_seqlens_q._version, cu_seqlens_k._version)
    except RuntimeError:  # inference-mode tensors keep no version counter
        versions = None
    if (versions is not None and cached is not None and cached[0] is cu_seqlens_q and cached[1] is cu_seqlens_k
            and cached[2] == versions):
        return cached[3], cached[4]
    n = cu_seqlens_q.shape[0]
    cu = torch.cat([cu_seqlens_q.reshape(-1).to(torch.int64), cu_seqlens_k.reshape(-1).to(torch.int64)]).tolist()
    cu_q, cu_k = cu[:n], cu[n:]
    if versions is not None:
        _cu_host = (cu_seqlens_q, cu_seqlens_k, versions, cu_q, cu_k)
    return cu_q, cu_k


def _check_block_table(block_table, lens_k, page, num_pages):
    """The table has a column for every page a sequence uses (from the key
    counts already on the host).  The page ids themselves are read on the
    host only with MTLFLASHATTN_CHECK_PAGES=1 (a device-to-host copy and a
    stream sync per call); otherwise the kernel's guard applies: a page id
    outside [0, num_pages) reads as zeros, never out of bounds."""
    need = [-(-n // page) for n in lens_k]
    if max(need, default=0) > block_table.shape[1]:
        raise ValueError(f"mtlflashattn_amd: block_table has {block_table.shape[1]} pages per sequence, "
                         f"{max(need)} needed for {max(lens_k)} keys")
    if not need or max(need) == 0:
        return
    if os.environ.get("MTLFLASHATTN_CHECK_PAGES", "").lower() not in ("1", "on", "true", "yes"):
        return
    used = torch.arange(block_table.shape[1]).unsqueeze(0) < torch.tensor(need).unsqueeze(1)
    ids = block_table.cpu()[used]
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= num_pages):
        raise ValueError(f"mtlflashattn_amd: block_table holds page ids outside [0, {num_pages})")


def merge_attention_partials(outs, lses):
    """Combine attentions of the same queries over disjoint key sets.

    outs: list of [..., Lq, Hq, D] outputs (any float dtype), lses: the
    matching [..., Hq, Lq] fp32 log-sum-exps (flash_attn_func_with_lse
    layout).  Returns (out in outs[0].dtype, lse): out = sum_i w_i out_i with
    w_i = exp(lse_i - lse), lse = ln(sum_i exp(lse_i)); rows without a valid
    key in any part get out = 0, lse = -inf.  This is the merge a
    context-parallel forward (key/value shards on different GPUs) or a
    cache + new-token split needs; it runs as PyTorch elementwise ops.
    """
    if len(outs) != len(lses) or not outs:
        raise ValueError("mtlflashattn_amd: merge_attention_partials needs matching, non-empty outs and lses")
    lse_all = torch.stack([x.float() for x in lses])
    lse = torch.logsumexp(lse_all, dim=0)
    safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
    acc = None
    for o, l in zip(outs, lse_all):
        w = torch.exp(l - safe).masked_fill(torch.isinf(lse), 0.0)
        term = o.float() * w.transpose(-1, -2).unsqueeze(-1)
        acc = term if acc is None else acc + term
    return acc.to(outs[0].dtype), lse


def flash_attn_qkvpacked_func(qkv, *args, **kwargs):
    """Drop-in for flash_attn.flash_attn_qkvpacked_func. qkv: [B, S, 3, H, D]."""
    if qkv.dim() != 5 or qkv.shape[2] != 3:
        raise ValueError(f"mtlflashattn_amd: expected qkv [B,S,3,H,D], got {tuple(qkv.shape)}")
    q, k, v = qkv.unbind(dim=2)
    return flash_attn_func(q, k, v, *args, **kwargs)


def flash_attn_kvpacked_func(q, kv, *args, **kwargs):
    """Drop-in for flash_attn.flash_attn_kvpacked_func. kv: [B, Sk, 2, Hkv, D]."""
    if kv.dim() != 5 or kv.shape[2] != 2:
        raise ValueError(f"mtlflashattn_amd: expected kv [B,S,2,H,D], got {tuple(kv.shape)}")
    k, v = kv.unbind(dim=2)
    return flash_attn_func(q, k, v, *args, **kwargs)


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, *args, **kwargs):
    """Drop-in for flash_attn.flash_attn_varlen_qkvpacked_func. qkv: [total, 3, H, D]."""
    if qkv.dim() != 4 or qkv.shape[1] != 3:
        raise ValueError(f"mtlflashattn_amd: expected qkv [total,3,H,D], got {tuple(qkv.shape)}")
    q, k, v = qkv.unbind(dim=1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen, *args, **kwargs)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, *args, **kwargs):
    """Drop-in for flash_attn.flash_attn_varlen_kvpacked_func. kv: [total_k, 2, Hkv, D]."""
    if kv.dim() != 4 or kv.shape[1] != 2:
        raise ValueError(f"mtlflashattn_amd: expected kv [total,2,H,D], got {tuple(kv.shape)}")
    k, v = kv.unbind(dim=1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, *args, **kwargs)
