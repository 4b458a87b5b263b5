"""Dispatcher boundary and HIP launcher.

`flash_attn_forward` keeps the signature and contract of the reference's
internal boundary (metal_flash_attn/_kernel.py:1052-1153): heads-second
q [B,Hq,Lq,D], k/v [B,Hkv,Lk,D] with any strides in, contiguous
[B,Hq,Lq,D] in q.dtype out.  Behind it the reference's Metal tier dispatch
(v0/v1/v2/v2r/v2_dtype, _kernel.py:716-985, :1288-1420) is replaced by one
path: the C ABI of libmtlfa_hip.so (include/mfa.h), which launches the gfx950
FA-2 kernels on torch's current HIP stream.

There is no silent fallback: a tensor that is not on a ROCm GPU raises
NotImplementedError (as the reference raises for non-MPS devices,
metal_flash_attn/__init__.py:51-52) and a missing or broken HIP library
raises RuntimeError.
"""
from __future__ import annotations

import atexit
import os
import sys
import warnings
from collections import namedtuple

import torch
import torch.nn.functional as F

from . import _hip

# Bias/masking knobs threaded through the launcher (metal_flash_attn/_kernel.py:20-24).
# softcap: logit soft-cap (0 = off). window_left/window_right: sliding-window key
# bounds relative to the bottom-right diagonal (-1 = open). alibi: fp32 slopes or None.
_BiasParams = namedtuple("_BiasParams", "softcap window_left window_right alibi")

MAX_HEAD_DIM = 128  # metal_flash_attn/_kernel.py:26

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Every value the reference accepted for MTLFLASHATTN_KERNEL
# (metal_flash_attn/_kernel.py:1077-1153) selects the single HIP path here.
_KNOWN_MODES = frozenset(
    {"auto", "hip", "torch", "pytorch", "v0", "v1", "v2", "v2_fp32", "v2_bf16", "v2_dtype", "v2_typed"}
)
_warned_modes = set()


# Preferred C-ABI tile_hint for bf16/fp16 launches (0 = the library's choice);
# tests set it to run every case through each kernel.  A preference the launch
# cannot take (fp32; ping-pong with a head dim above 64 or a block table)
# falls back to 0.
_TILE_HINT = 0
_PP_HINTS = (_hip.MFA_TILE_PINGPONG, _hip.MFA_TILE_PINGPONG256)


def _pp_head_dim_ok(D: int) -> bool:
    """The ping-pong tiles exist for head dims padded to 32, 64 and 128 (not 96)."""
    return -(-D // 32) * 32 != 96
# Split-KV chunk in keys for bf16/fp16 calls: None = the library's choice
# (mfa_fwd_split_keys), 0 = never split, a multiple of 64 = that chunk
# (tests and tuning).
_SPLIT_KEYS = None


def _kernel_mode() -> str:
    mode = os.environ.get("MTLFLASHATTN_KERNEL", "auto").lower()
    if mode not in ("auto", "hip") and mode not in _warned_modes:
        _warned_modes.add(mode)
        what = "a Metal tier" if mode in _KNOWN_MODES else "unknown"
        warnings.warn(
            f"mtlflashattn_amd: MTLFLASHATTN_KERNEL={mode!r} is {what}; the ROCm build has a single HIP "
            "path and uses it for every mode",
            stacklevel=3,
        )
    return "hip"


# ---------------------------------------------------------------------------
# trace (metal_flash_attn/_kernel.py:988-1049): per-(dtype, D, Lq, Lk, causal,
# label) call counts, printed to stderr at exit when MTLFLASHATTN_TRACE is set.

_trace = {}


def _trace_enabled() -> bool:
    return os.environ.get("MTLFLASHATTN_TRACE", "").lower() in ("1", "on", "true", "yes")


def _effective_kernel_label(q, k, v) -> str:
    """Label of the path flash_attn_forward takes (one path: the HIP kernels)."""
    return "hip"


def _record_trace(dtype, D, Lq, Lk, causal, label="hip"):
    try:
        key = (str(dtype).replace("torch.", ""), int(D), int(Lq), int(Lk), bool(causal), label)
        _trace[key] = _trace.get(key, 0) + 1
    except Exception:
        pass  # tracing must never break a real run


def _trace_summary_lines():
    if not _trace:
        return []
    total = sum(_trace.values())
    lines = [f"[MTLFLASHATTN_TRACE] {total} attention call(s), {len(_trace)} distinct shape/kernel combos:"]
    for (dt, D, Lq, Lk, causal, label), n in sorted(_trace.items(), key=lambda kv: (-kv[1], kv[0])):
        lines.append(
            f"  calls={n:<6} {dt:<9} D={D:<4} Lq={Lq:<6} Lk={Lk:<6} causal={'T' if causal else 'F'}  -> {label}"
        )
    return lines


@atexit.register
def _trace_atexit():
    if _trace_enabled() and _trace:
        print("\n".join(_trace_summary_lines()), file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# argument preparation


def _alibi_arg(alibi_slopes, B, Hq, device):
    """Validate [Hq] / [B, Hq] slopes (metal_flash_attn/_kernel.py:1275-1285).

    Returns (contiguous fp32 slopes on `device`, batch stride) with batch
    stride 0 for per-head slopes and Hq for per-(batch, head) slopes, so no
    [B*Hq] broadcast copy is made.
    """
    if alibi_slopes is None:
        return None, 0
    s = alibi_slopes
    if s.dim() == 1 and s.shape[0] == Hq:
        bstride = 0
    elif s.dim() == 2 and tuple(s.shape) == (B, Hq):
        bstride = Hq
    else:
        raise ValueError(
            f"mtlflashattn_amd: alibi_slopes must be [Hq={Hq}] or [B={B}, Hq={Hq}], got {tuple(s.shape)}"
        )
    return s.to(device=device, dtype=torch.float32).contiguous(), bstride


def _check_qkv_shapes(q, k, v, h_axis, s_axis):
    """4-D q/k/v that agree on the batch size, k/v on head count and length,
    and a K/V head count that divides the query head count (CUDA flash-attn
    and stock SDPA reject the rest; the kernel takes B from q and the K/V
    head count from k, so a mismatch must never reach it)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"mtlflashattn_amd: expected 4-D q/k/v, got {q.dim()}/{k.dim()}/{v.dim()} dims")
    if not (q.shape[0] == k.shape[0] == v.shape[0]):
        raise ValueError(f"mtlflashattn_amd: batch mismatch (q {q.shape[0]}, k {k.shape[0]}, v {v.shape[0]})")
    Hq, Hkv = q.shape[h_axis], k.shape[h_axis]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"mtlflashattn_amd: num_heads_kv ({Hkv}) must divide num_heads_q ({Hq})")
    if v.shape[h_axis] != Hkv:
        raise ValueError(f"mtlflashattn_amd: k has {Hkv} heads, v {v.shape[h_axis]}")
    if k.shape[s_axis] != v.shape[s_axis]:
        raise ValueError("mtlflashattn_amd: k/v seqlen mismatch")


def _is_rocm_tensor(t) -> bool:
    """True for a tensor on a ROCm GPU (the only device the HIP path serves)."""
    return t.device.type == "cuda" and torch.version.hip is not None


def _check_device(*tensors):
    for t in tensors:
        if not _is_rocm_tensor(t):
            raise NotImplementedError(
                f"mtlflashattn_amd: device {t.device.type!r} not supported (ROCm GPU only)"
            )
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"mtlflashattn_amd: tensors on different devices ({dev} vs {t.device})")


def _fits_abi(x: torch.Tensor) -> bool:
    """16-byte aligned base and 16-byte multiple strides (size-1 dims ignored)."""
    if x.stride(-1) != 1 and x.shape[-1] > 1:
        return False
    if x.data_ptr() % 16:
        return False
    al = 16 // x.element_size()
    return all(st % al == 0 for st, n in zip(x.stride()[:-1], x.shape[:-1]) if n > 1)


def _abi_operand(x: torch.Tensor) -> torch.Tensor:
    """x itself when it meets the C ABI's layout rule (_fits_abi), else a
    fresh contiguous copy.  A contiguous tensor at a storage offset that is
    not 16-byte aligned (e.g. base[1:].view(...)) stays misaligned under
    .contiguous(), which returns it unchanged; a new allocation from torch's
    caching allocator is aligned."""
    if _fits_abi(x):
        return x
    y = x.contiguous()
    if y is x or not _fits_abi(y):
        y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        y.copy_(x)
    return y


def _strides_bsh(x: torch.Tensor):
    """(batch, seq, head) element strides of a [B, S, H, D] view; 0 for size-1 dims."""
    return tuple(int(st) if n > 1 else 0 for st, n in zip(x.stride()[:3], x.shape[:3]))


def _run(q, k, v, out, *, scale, causal, softcap, window_left, window_right, alibi, alibi_bstride,
         cu_q=None, cu_k=None, seqlen_q=None, seqlen_k=None, lse=None, block_table=None, no_single_rows=False):
    """Launch the HIP forward on [B, S, H, D] views q, k, v and write `out`.

    out: [B, Sq, Hq, D] tensor of q.dtype or float32 (full-precision output).
    Varlen: q/k/v/out are [1, total, H, D] views, cu_q/cu_k int32 device
    tensors, seqlen_q/seqlen_k the maximum per-sequence lengths.
    lse: optional fp32 softmax log-sum-exp output with contiguous rows,
    [B, Hq, Lq] (dense) or [Hq, total_q] (varlen).
    block_table: optional int32 [batch, pages per sequence] page table; k/v
    are then [num_pages, page_block_size, Hkv, D] and every sequence's key
    count comes from seqlen_k (dense) or cu_k (varlen).
    no_single_rows: (varlen) no sequence has exactly one query row, so the
    exact-row launch for such sequences is skipped.
    """
    _kernel_mode()
    B, Sq, Hq, D = q.shape
    Hkv = k.shape[2]
    varlen = cu_q is not None
    batch = (cu_q.shape[0] - 1) if varlen else B
    Lq = int(seqlen_q) if varlen else Sq
    Lk = int(seqlen_k) if (varlen or block_table is not None) else k.shape[1]
    if batch == 0 or Lq == 0 or Hq == 0 or out.numel() == 0:
        return out
    if k.shape[1] == 0 or Lk == 0:
        if lse is not None:
            lse.fill_(float("-inf"))  # log-sum-exp over no key
        return out.zero_()  # no keys: every row is fully masked -> 0
    lse_strides = (0 if varlen else lse.stride(0), lse.stride(-2)) if lse is not None else None
    paged = (int(block_table.stride(0)), k.shape[1], k.shape[0]) if block_table is not None else None

    Dp = -(-D // 8) * 8
    if Dp == D:
        # fast path: tensors used in place; the launch parameters of this
        # signature (everything but the data pointers) are prepared once
        key = (q.shape, q.stride(), k.shape, k.stride(), v.shape, v.stride(), out.shape, out.stride(), q.dtype,
               out.dtype, q.device.index, float(scale), bool(causal), float(softcap), int(window_left),
               int(window_right), alibi is not None, alibi_bstride,
               (cu_q.shape[0], Lq, Lk) if varlen else None, _TILE_HINT, _SPLIT_KEYS, lse_strides, paged)
        ent = _plans.get(key)
        if ent is None and all(_fits_strides(t) for t in (q, k, v, out)):
            ent = _prepare(q, k, v, out, batch, Hq, Hkv, Lq, Lk, Dp, varlen, scale, causal, softcap, window_left,
                           window_right, alibi is not None, alibi_bstride, lse_strides, paged)
            if len(_plans) >= _PLANS_MAX:
                _plans.clear()
            _plans[key] = ent
        if ent is not None and not ((q.data_ptr() | k.data_ptr() | v.data_ptr() | out.data_ptr()) & 15):
            p = _hip.MfaFwdParams.from_buffer_copy(ent[0])
            p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
            if varlen:
                p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
            if alibi is not None:
                p.alibi_slopes = alibi.data_ptr()
            if lse is not None:
                p.softmax_lse = lse.data_ptr()
            if paged is not None:
                p.block_table = block_table.data_ptr()
            p.varlen_no_single_rows = 1 if (varlen and no_single_rows) else 0
            _launch(p, ent[1], q.device)
            return out
    if Dp != D:  # the kernels read 16-byte chunks: zero-pad the head dim
        q, k, v = (F.pad(t, (0, Dp - D)) for t in (q, k, v))
    q, k, v = (_abi_operand(t) for t in (q, k, v))
    dst = out
    if Dp != D or not _fits_abi(out) or out.stride(-1) != 1:
        dst = torch.empty(out.shape[:-1] + (Dp,), dtype=out.dtype, device=out.device)

    p = _hip.MfaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), dst.data_ptr()
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = _strides_bsh(q)
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = _strides_bsh(k)
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = _strides_bsh(v)
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = _strides_bsh(dst)
    p.batch, p.heads_q, p.heads_kv = batch, Hq, Hkv
    p.seqlen_q, p.seqlen_k, p.head_dim = Lq, Lk, Dp
    if varlen:
        p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.scale = float(scale)
    p.softcap = float(softcap)
    p.window_left, p.window_right = int(window_left), int(window_right)
    p.causal = 1 if causal else 0
    if alibi is not None:
        p.alibi_slopes = alibi.data_ptr()
        p.alibi_batch_stride = alibi_bstride
    p.dtype_in = _hip.DTYPE_CODES[q.dtype]
    p.dtype_out = _hip.DTYPE_CODES[out.dtype]
    hint = _TILE_HINT
    if q.dtype == torch.float32 or (hint in _PP_HINTS and (not _pp_head_dim_ok(Dp) or paged is not None)):
        hint = _hip.MFA_TILE_AUTO
    p.tile_hint = hint
    if lse is not None:
        p.softmax_lse = lse.data_ptr()
        p.lse_batch_stride, p.lse_head_stride = lse_strides
    if paged is not None:
        p.block_table = block_table.data_ptr()
        p.block_table_batch_stride, p.page_block_size, p.num_pages = paged
    p.varlen_no_single_rows = 1 if (varlen and no_single_rows) else 0
    _launch(p, _split_choice(p, q.dtype, hint), q.device)
    if dst is not out:
        out.copy_(dst[..., :D])
    return out


# prepared launch parameters per call signature (see _run's fast path)
_plans = {}
_PLANS_MAX = 512


def _fits_strides(x: torch.Tensor) -> bool:
    """_fits_abi without the base-address test (strides only)."""
    if x.stride(-1) != 1 and x.shape[-1] > 1:
        return False
    al = 16 // x.element_size()
    return all(st % al == 0 for st, n in zip(x.stride()[:-1], x.shape[:-1]) if n > 1)


def _prepare(q, k, v, out, batch, Hq, Hkv, Lq, Lk, Dp, varlen, scale, causal, softcap, window_left, window_right,
             has_alibi, alibi_bstride, lse_strides=None, paged=None):
    """(parameter template without data pointers, split-KV choice) of a call."""
    p = _hip.MfaFwdParams()
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = _strides_bsh(q)
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = _strides_bsh(k)
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = _strides_bsh(v)
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = _strides_bsh(out)
    p.batch, p.heads_q, p.heads_kv = batch, Hq, Hkv
    p.seqlen_q, p.seqlen_k, p.head_dim = Lq, Lk, Dp
    if varlen:  # placeholders: the choice below only needs to see varlen
        p.cu_seqlens_q = p.cu_seqlens_k = 256
    p.scale, p.softcap = float(scale), float(softcap)
    p.window_left, p.window_right = int(window_left), int(window_right)
    p.causal = 1 if causal else 0
    if has_alibi:
        p.alibi_slopes = 256
        p.alibi_batch_stride = alibi_bstride
    p.dtype_in = _hip.DTYPE_CODES[q.dtype]
    p.dtype_out = _hip.DTYPE_CODES[out.dtype]
    hint = _TILE_HINT
    if q.dtype == torch.float32 or (hint in _PP_HINTS and (not _pp_head_dim_ok(Dp) or paged is not None)):
        hint = _hip.MFA_TILE_AUTO
    p.tile_hint = hint
    if lse_strides is not None:
        p.lse_batch_stride, p.lse_head_stride = lse_strides
    if paged is not None:
        p.block_table_batch_stride, p.page_block_size, p.num_pages = paged
    chunk = _split_choice(p, q.dtype, hint)
    p.cu_seqlens_q = p.cu_seqlens_k = p.alibi_slopes = None
    return p, chunk


def _split_choice(p, dtype, hint):
    if dtype == torch.float32 or hint in _PP_HINTS:
        return 0
    return _hip.split_keys(p) if _SPLIT_KEYS is None else _SPLIT_KEYS


def _launch(p, chunk, device):
    idx = device.index
    if idx != torch.cuda.current_device():
        with torch.cuda.device(device):
            return _launch(p, chunk, device)
    stream = torch._C._cuda_getCurrentRawStream(idx)
    if chunk:
        # split-KV: partials in a workspace from torch's stream-ordered
        # caching allocator (reused only after these kernels ran)
        nbytes = _hip.workspace_bytes(p, chunk)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _hip.fwd_splitkv(p, chunk, ws.data_ptr(), nbytes, stream)
    else:
        _hip.fwd(p, stream)


def _out_dtype(q, out_dtype):
    if out_dtype is None or out_dtype == q.dtype:
        return q.dtype
    if out_dtype != torch.float32:
        raise ValueError(f"mtlflashattn_amd: out_dtype must be None, q.dtype or torch.float32, got {out_dtype}")
    return torch.float32


def flash_attn_forward(q, k, v, scale, causal, softcap=0.0, window_left=-1, window_right=-1,
                       alibi_slopes=None, out_dtype=None, return_lse=False):
    """q: [B,Hq,Lq,D], k/v: [B,Hkv,Lk,D] (heads-second, any strides).

    Returns [B,Hq,Lq,D] contiguous, in q.dtype (metal_flash_attn/_kernel.py:1052-1056).
    out_dtype=torch.float32 returns the kernel's fp32 result before the
    final rounding to q.dtype (the parity mode for bf16/fp16 inputs).
    return_lse=True returns (out, lse) with the fp32 softmax log-sum-exp
    lse [B,Hq,Lq] (natural log, -inf for rows with no valid key); the
    reference has no such output.
    """
    if _trace_enabled():
        _record_trace(q.dtype, q.shape[-1], q.shape[2], k.shape[2], causal)
    if softcap < 0:
        # _kernel.py:1070-1073: reject here so direct callers cannot diverge
        raise ValueError("mtlflashattn_amd: softcap must be >= 0 (0 disables capping)")
    _check_qkv_shapes(q, k, v, h_axis=1, s_axis=2)
    B, Hq, Lq, D = q.shape
    alibi, bstride = _alibi_arg(alibi_slopes, B, Hq, q.device)
    _check_device(q, k, v)
    if q.dtype not in _SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise NotImplementedError(f"mtlflashattn_amd: dtype {q.dtype} (q/k/v must match, fp16/bf16/fp32)")
    if D > MAX_HEAD_DIM:
        raise NotImplementedError(f"mtlflashattn_amd: head_dim {D} > {MAX_HEAD_DIM}")
    if _needs_grad(q, k, v) and _out_dtype(q, out_dtype) == q.dtype:
        # differentiable path (heads-third views of the same tensors)
        o, lse = _FlashAttnFn.apply(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale, causal,
                                    softcap, window_left, window_right, alibi_slopes)
        o = o.transpose(1, 2).contiguous()
        return (o, lse) if return_lse else o
    out = torch.empty(B, Hq, Lq, D, dtype=_out_dtype(q, out_dtype), device=q.device)
    lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device) if return_lse else None
    _run(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), out.transpose(1, 2),
         scale=scale, causal=causal, softcap=softcap, window_left=window_left,
         window_right=window_right, alibi=alibi, alibi_bstride=bstride, lse=lse)
    return (out, lse) if return_lse else out


def forward_bshd(q, k, v, scale, causal, softcap=0.0, window_left=-1, window_right=-1,
                 alibi_slopes=None, out_dtype=None, return_lse=False):
    """Heads-third forward: q [B,Lq,Hq,D], k/v [B,Lk,Hkv,D] -> [B,Lq,Hq,D].

    Same result as flash_attn_forward on the transposed views followed by
    `.transpose(1, 2).contiguous()` (metal_flash_attn/__init__.py:93-99), but
    the kernel writes the heads-third output directly (no layout copies).
    return_lse=True returns (out, lse [B,Hq,Lq] fp32).
    """
    if _trace_enabled():
        _record_trace(q.dtype, q.shape[-1], q.shape[1], k.shape[1], causal)
    if softcap < 0:
        raise ValueError("mtlflashattn_amd: softcap must be >= 0 (0 disables capping)")
    _check_qkv_shapes(q, k, v, h_axis=2, s_axis=1)
    B, Lq, Hq, D = q.shape
    if _needs_grad(q, k, v) and _out_dtype(q, out_dtype) == q.dtype:
        _alibi_arg(alibi_slopes, B, Hq, q.device)  # validate before autograd records anything
        o, lse = _FlashAttnFn.apply(q, k, v, scale, causal, softcap, window_left, window_right, alibi_slopes)
        return (o, lse) if return_lse else o
    alibi, bstride = _alibi_arg(alibi_slopes, B, Hq, q.device)
    out = torch.empty(B, Lq, Hq, D, dtype=_out_dtype(q, out_dtype), device=q.device)
    lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device) if return_lse else None
    _run(q, k, v, out, scale=scale, causal=causal, softcap=softcap, window_left=window_left,
         window_right=window_right, alibi=alibi, alibi_bstride=bstride, lse=lse)
    return (out, lse) if return_lse else out


def forward_varlen(q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, softcap=0.0, window_left=-1,
                   window_right=-1, alibi_slopes=None, out_dtype=None, return_lse=False, block_table=None,
                   _grad=True, no_single_rows=False):
    """Packed varlen forward in ONE launch: q [Tq,Hq,D], k/v [Tk,Hkv,D].

    cu_q/cu_k: int32 [batch+1] device tensors; max_q/max_k: the longest
    sequence lengths.  Replaces the reference's per-sequence loop of B=1
    dispatches (metal_flash_attn/__init__.py:165-182) with the same result.
    return_lse=True returns (out, lse [Hq, Tq] fp32).  block_table: int32
    [batch, pages per sequence]; k/v are then a page pool
    [num_pages, page_block_size, Hkv, D] and cu_k gives the key counts only
    (paged calls are forward-only).  Inputs that require grad (and no block
    table, q.dtype output) go through the HIP backward.  no_single_rows: the
    caller knows no sequence has exactly one query row (the library then
    skips the exact-row launch for such sequences; a one-row sequence would
    be left unwritten).
    """
    batch = cu_q.shape[0] - 1
    Hq = q.shape[1]
    if alibi_slopes is not None and alibi_slopes.dim() == 2 and tuple(alibi_slopes.shape) != (batch, Hq):
        raise ValueError(
            f"mtlflashattn_amd: alibi_slopes must be [Hq={Hq}] or [B={batch}, Hq={Hq}], "
            f"got {tuple(alibi_slopes.shape)}"
        )
    alibi, bstride = _alibi_arg(alibi_slopes, batch, Hq, q.device)
    if _trace_enabled() and _grad:
        _record_trace(q.dtype, q.shape[-1], max_q, max_k, causal, "hip-varlen")
    if block_table is not None and _needs_grad(q, k, v) and _out_dtype(q, out_dtype) == q.dtype:
        raise NotImplementedError("mtlflashattn_amd: paged K/V (block_table) calls are forward-only; "
                                  "run them under torch.no_grad() or without inputs that require grad")
    if _grad and block_table is None and _needs_grad(q, k, v) and _out_dtype(q, out_dtype) == q.dtype:
        o, lse = _FlashAttnVarlenFn.apply(q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, softcap, window_left,
                                          window_right, alibi_slopes, no_single_rows)
        return (o, lse) if return_lse else o
    out = torch.empty(q.shape, dtype=_out_dtype(q, out_dtype), device=q.device)
    lse = torch.empty(Hq, q.shape[0], dtype=torch.float32, device=q.device) if return_lse else None
    cu_q = cu_q.to(device=q.device, dtype=torch.int32).contiguous()
    cu_k = cu_k.to(device=q.device, dtype=torch.int32).contiguous()
    if block_table is not None:
        block_table = block_table.to(device=q.device, dtype=torch.int32)
        if block_table.stride(1) != 1:
            block_table = block_table.contiguous()
    _run(q[None], k if block_table is not None else k[None], v if block_table is not None else v[None], out[None],
         scale=scale, causal=causal, softcap=softcap, window_left=window_left, window_right=window_right,
         alibi=alibi, alibi_bstride=bstride, cu_q=cu_q, cu_k=cu_k, seqlen_q=max_q, seqlen_k=max_k, lse=lse,
         block_table=block_table, no_single_rows=no_single_rows)
    return (out, lse) if return_lse else out


# ---------------------------------------------------------------------------
# backward (the reference is forward-only, metal_flash_attn/__init__.py:3-4;
# README.md:159-161): HIP kernels behind mfa_bwd, wired into autograd


def _needs_grad(*tensors):
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _run_bwd(q, k, v, out, dout, lse, *, scale, causal, softcap, window_left, window_right, alibi, alibi_bstride,
             cu_q=None, cu_k=None, seqlen_q=None, seqlen_k=None, grad_f32=False, dlse=None):
    """(dq, dk, dv) of the forward on [B, S, H, D] views (varlen: [1, T, H, D]).

    out: the forward's output in q.dtype; lse: its softmax_lse ([B, Hq, Lq]
    dense, [Hq, T] varlen); dlse: optional gradient of lse (same shape).
    Returns new tensors shaped like q, k, v in q.dtype (grad_f32=True: fp32,
    the parity mode).
    """
    _kernel_mode()
    _check_device(q, k, v, out, dout)
    B, Sq, Hq, D = q.shape
    Hkv = k.shape[2]
    varlen = cu_q is not None
    batch = (cu_q.shape[0] - 1) if varlen else B
    Lq = int(seqlen_q) if varlen else Sq
    Lk = int(seqlen_k) if varlen else k.shape[1]
    gdt = torch.float32 if grad_f32 else q.dtype
    if batch == 0 or Lq == 0 or Lk == 0 or Hq == 0 or q.numel() == 0 or k.numel() == 0:
        return tuple(torch.zeros(t.shape, dtype=gdt, device=t.device) for t in (q, k, v))
    Dp = -(-D // 8) * 8
    ts = [q, k, v, out, dout.to(q.dtype)]
    if Dp != D:
        ts = [F.pad(t, (0, Dp - D)) for t in ts]
    q_, k_, v_, o_, do_ = (_abi_operand(t) for t in ts)
    dq = torch.empty(q_.shape, dtype=gdt, device=q.device)
    dk = torch.empty(k_.shape, dtype=gdt, device=q.device)
    dv = torch.empty(v_.shape, dtype=gdt, device=q.device)

    bp = _hip.MfaBwdParams()
    p = bp.fwd
    p.q, p.k, p.v, p.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o_.data_ptr()
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = _strides_bsh(q_)
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = _strides_bsh(k_)
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = _strides_bsh(v_)
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = _strides_bsh(o_)
    p.batch, p.heads_q, p.heads_kv = batch, Hq, Hkv
    p.seqlen_q, p.seqlen_k, p.head_dim = Lq, Lk, Dp
    if varlen:
        p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.scale, p.softcap = float(scale), float(softcap)
    p.window_left, p.window_right = int(window_left), int(window_right)
    p.causal = 1 if causal else 0
    if alibi is not None:
        p.alibi_slopes = alibi.data_ptr()
        p.alibi_batch_stride = alibi_bstride
    p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[q.dtype]
    lse = lse.contiguous()
    p.softmax_lse = lse.data_ptr()
    if dlse is not None:
        dlse = dlse.to(device=q.device, dtype=torch.float32).contiguous()
        bp.dlse = dlse.data_ptr()
    p.lse_batch_stride, p.lse_head_stride = (0, lse.stride(0)) if varlen else (lse.stride(0), lse.stride(1))
    bp.dout = do_.data_ptr()
    bp.do_batch_stride, bp.do_seq_stride, bp.do_head_stride = _strides_bsh(do_)
    bp.dq = dq.data_ptr()
    bp.dq_batch_stride, bp.dq_seq_stride, bp.dq_head_stride = _strides_bsh(dq)
    bp.dk = dk.data_ptr()
    bp.dk_batch_stride, bp.dk_seq_stride, bp.dk_head_stride = _strides_bsh(dk)
    bp.dv = dv.data_ptr()
    bp.dv_batch_stride, bp.dv_seq_stride, bp.dv_head_stride = _strides_bsh(dv)
    bp.dtype_grad = _hip.DTYPE_CODES[gdt]
    device = q.device
    with torch.cuda.device(device):
        nbytes = _hip.bwd_workspace_bytes(bp)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _hip.bwd(bp, ws.data_ptr(), nbytes, torch._C._cuda_getCurrentRawStream(device.index))
    if Dp != D:
        dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
    return dq, dk, dv


class _FlashAttnFn(torch.autograd.Function):
    """Heads-third dense attention with the HIP backward; returns (out, lse),
    both differentiable (a gradient on lse enters the backward's row sums)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, softcap, window_left, window_right, alibi_slopes):
        B, Lq, Hq, D = q.shape
        alibi, bstride = _alibi_arg(alibi_slopes, B, Hq, q.device)
        out = torch.empty(B, Lq, Hq, D, dtype=q.dtype, device=q.device)
        lse = torch.empty(B, Hq, Lq, dtype=torch.float32, device=q.device)
        _run(q, k, v, out, scale=scale, causal=causal, softcap=softcap, window_left=window_left,
             window_right=window_right, alibi=alibi, alibi_bstride=bstride, lse=lse)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.cfg = dict(scale=scale, causal=causal, softcap=softcap, window_left=window_left,
                       window_right=window_right, alibi=alibi, alibi_bstride=bstride)
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, k, v, out, lse = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv = _run_bwd(q, k, v, out, dout, lse, dlse=dlse, **ctx.cfg)
        return dq, dk, dv, None, None, None, None, None, None


class _FlashAttnVarlenFn(torch.autograd.Function):
    """Packed varlen attention with the HIP backward; returns (out, lse [Hq, T]),
    both differentiable."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, softcap, window_left, window_right,
                alibi_slopes, no_single_rows=False):
        out, lse = forward_varlen(q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, softcap, window_left,
                                  window_right, alibi_slopes, return_lse=True, _grad=False,
                                  no_single_rows=no_single_rows)
        batch, Hq = cu_q.shape[0] - 1, q.shape[1]
        alibi, bstride = _alibi_arg(alibi_slopes, batch, Hq, q.device)
        cu_q = cu_q.to(device=q.device, dtype=torch.int32).contiguous()
        cu_k = cu_k.to(device=q.device, dtype=torch.int32).contiguous()
        ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_k)
        ctx.cfg = dict(scale=scale, causal=causal, softcap=softcap, window_left=window_left,
                       window_right=window_right, alibi=alibi, alibi_bstride=bstride, seqlen_q=max_q,
                       seqlen_k=max_k)
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, k, v, out, lse, cu_q, cu_k = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv = _run_bwd(q[None], k[None], v[None], out[None], dout[None], lse, cu_q=cu_q, cu_k=cu_k,
                              dlse=dlse, **ctx.cfg)
        return dq[0], dk[0], dv[0], None, None, None, None, None, None, None, None, None, None, None


def split_chunk(q, k):
    """Split-KV chunk (keys) the library picks for heads-third q/k (0: single pass)."""
    if q.dtype == torch.float32:
        return 0
    p = _hip.MfaFwdParams()
    p.batch, p.heads_q, p.heads_kv = q.shape[0], q.shape[2], k.shape[2]
    p.seqlen_q, p.seqlen_k = q.shape[1], k.shape[1]
    p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[q.dtype]
    p.tile_hint = _TILE_HINT
    return _hip.split_keys(p) if _SPLIT_KEYS is None else _SPLIT_KEYS


def launch_info(q, k, v, causal=False, softcap=0.0, alibi=False, window_left=-1, window_right=-1):
    """Kernel geometry (name, grid, tile) for heads-third q/k/v; no launch."""
    B, Lq, Hq, D = q.shape
    p = _hip.MfaFwdParams()
    p.q = p.k = p.v = p.o = 256  # placeholder aligned addresses: nothing is read
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = Lq * Hq * D, Hq * D, D
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = k.shape[1] * k.shape[2] * D, k.shape[2] * D, D
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = p.k_batch_stride, p.k_seq_stride, p.k_head_stride
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = p.q_batch_stride, p.q_seq_stride, p.q_head_stride
    p.batch, p.heads_q, p.heads_kv = B, Hq, k.shape[2]
    p.seqlen_q, p.seqlen_k, p.head_dim = Lq, k.shape[1], -(-D // 8) * 8
    p.scale = 1.0
    p.softcap = float(softcap)
    p.window_left, p.window_right, p.causal = window_left, window_right, int(causal)
    p.alibi_slopes = 256 if alibi else None
    p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[q.dtype]
    hint = _TILE_HINT
    if q.dtype == torch.float32 or (hint in _PP_HINTS and not _pp_head_dim_ok(p.head_dim)):
        hint = _hip.MFA_TILE_AUTO
    p.tile_hint = hint
    return _hip.launch_info(p)


def launch_info_varlen(q, k, nseq, max_seqlen_q, max_seqlen_k, causal=False, softcap=0.0, alibi=False,
                       window_left=-1, window_right=-1):
    """launch_info for a varlen call: q [total_q, Hq, D], k [total_k, Hkv, D],
    nseq sequences of at most max_seqlen_q / max_seqlen_k rows (the plan
    reads no prefix sums)."""
    Hq, D = q.shape[1], q.shape[2]
    Hkv = k.shape[1]
    p = _hip.MfaFwdParams()
    p.q = p.k = p.v = p.o = 256  # placeholder aligned addresses: nothing is read
    p.q_seq_stride, p.q_head_stride = Hq * D, D
    p.k_seq_stride, p.k_head_stride = Hkv * D, D
    p.v_seq_stride, p.v_head_stride = Hkv * D, D
    p.o_seq_stride, p.o_head_stride = Hq * D, D
    p.batch, p.heads_q, p.heads_kv = nseq, Hq, Hkv
    p.seqlen_q, p.seqlen_k, p.head_dim = max_seqlen_q, max_seqlen_k, -(-D // 8) * 8
    p.cu_seqlens_q = p.cu_seqlens_k = 256
    p.scale = 1.0
    p.softcap = float(softcap)
    p.window_left, p.window_right, p.causal = window_left, window_right, int(causal)
    p.alibi_slopes = 256 if alibi else None
    p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[q.dtype]
    hint = _TILE_HINT
    if q.dtype == torch.float32 or (hint in _PP_HINTS and not _pp_head_dim_ok(p.head_dim)):
        hint = _hip.MFA_TILE_AUTO
    p.tile_hint = hint
    return _hip.launch_info(p)
