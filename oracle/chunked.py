"""ORACLE -- test infrastructure only, never product code.

CPU restatement of the reference's chunked-fp32 torch path, the path every
result of mtlflashattn_amd is checked against.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker or the CPU baseline.

Follows, step for step:
  * metal_flash_attn/_kernel.py:1165-1208 (`_flash_torch`): fp32 upcast
    (:1172-1174); GQA by repeat_interleave of K/V (:1175-1178); query chunks of
    MTLFLASHATTN_TORCH_CHUNK rows, default 2048 (:1156-1162, :1188); per chunk
    scores = (q @ k^T) * scale (:1190) -> softcap (:1191-1192) -> ALiBi
    (:1193-1196) -> causal / window masks (:1197-1204) -> softmax (:1205) ->
    nan_to_num (:1206) -> @ V (:1207); cast to q.dtype (:1208, done by callers
    through `cast_like`).
  * metal_flash_attn/_kernel.py:1275-1285 (`_broadcast_alibi_slopes`).
  * metal_flash_attn/__init__.py:62-99 (heads-third API, default scale
    1/sqrt(D)) and :102-183 (varlen: one B=1 call per sequence, empty query
    sequences skipped, [B, Hq] ALiBi rows picked per sequence).
  * metal_flash_attn/sdpa.py:86-130 (`_uneven_v_attention`, the exact path of
    the SDPA patch for value head dim != query/key head dim): GQA expansion
    only with enable_gqa, fp32 scores in query chunks, bool / additive masks,
    TOP-LEFT causal (torch SDPA's convention), nan_to_num, @ V, cast to V's
    dtype (`uneven_v_attention`).

Pinned by tests/test_oracle_pinning.py against torch's SDPA (a library
routine), an independent float64 C restatement of the streaming kernel
(oracle/stream_ref.c), closed forms, and the committed fixtures in
tests/golden/.
"""
from __future__ import annotations

import math

import torch

DEFAULT_CHUNK = 2048


def broadcast_alibi(alibi_slopes, B, Hq):
    """[Hq] or [B, Hq] slopes -> contiguous [B*Hq] fp32 (_kernel.py:1275-1285)."""
    s = alibi_slopes.detach().to(device="cpu", dtype=torch.float32)
    if s.dim() == 1 and s.shape[0] == Hq:
        s = s.unsqueeze(0).expand(B, Hq)
    elif not (s.dim() == 2 and tuple(s.shape) == (B, Hq)):
        raise ValueError(f"alibi_slopes must be [Hq={Hq}] or [B={B}, Hq={Hq}], got {tuple(s.shape)}")
    return s.reshape(-1).contiguous()


def flash_torch(q, k, v, scale, causal, softcap=0.0, window_left=-1, window_right=-1, alibi=None,
                chunk=DEFAULT_CHUNK, rows=None, return_lse=False, grad=False, dtype=torch.float32):
    """Heads-second q [B,Hq,Lq,D], k/v [B,Hkv,Lk,D] (CPU) -> fp32 [B,Hq,Lq,D].

    `alibi` is the broadcast [B*Hq] fp32 slope vector or None.  The result is
    the reference's fp32 `out` before its final cast.  `rows` optionally
    restricts the computation to the query chunks whose start index is in
    `rows` (other rows are left as NaN); each chunk is computed exactly as in
    the full run, so the subset equals the corresponding rows of the full
    result.

    return_lse=True also returns the fp32 [B,Hq,Lq] log-sum-exp of the same
    masked scores the softmax at _kernel.py:1205 normalises,
    torch.logsumexp(scores, -1) (-inf for a row whose keys are all masked).
    The reference computes but never returns this normaliser; it is the
    oracle of the build's softmax_lse output.

    grad=True keeps q, k, v in the autograd graph (no detach; they must be CPU
    tensors) so torch autograd gives the gradients of the reference's math --
    the oracle of the build's backward; `dtype` is the compute precision
    (float64 for gradcheck).
    """
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"num_heads_kv ({Hkv}) must divide num_heads_q ({Hq})")
    if grad:
        qf, kf, vf = q.to(dtype), k.to(dtype), v.to(dtype)
    else:
        qf, kf, vf = (t.detach().cpu().to(dtype) for t in (q, k, v))
    if Hkv != Hq:
        rep = Hq // Hkv
        kf = kf.repeat_interleave(rep, dim=1)
        vf = vf.repeat_interleave(rep, dim=1)
    kt = kf.transpose(-1, -2)
    out = torch.full((B, Hq, Lq, D), float("nan"), dtype=dtype)
    lse = torch.full((B, Hq, Lq), float("nan"), dtype=dtype)
    chunk = max(1, int(chunk))
    wl, wr = int(window_left), int(window_right)
    windowed = wl >= 0 or wr >= 0
    key_pos = torch.arange(Lk)[None, :] if (causal or windowed) else None
    for start in range(0, Lq, chunk):
        if rows is not None and start not in rows:
            continue
        end = min(start + chunk, Lq)
        scores = (qf[:, :, start:end] @ kt) * scale
        if softcap:
            scores = softcap * torch.tanh(scores / softcap)
        if alibi is not None:
            center_a = torch.arange(start, end)[:, None] + (Lk - Lq)
            key_a = torch.arange(Lk)[None, :]
            scores = scores - alibi.to(dtype).reshape(B, Hq, 1, 1) * (center_a - key_a).abs().to(dtype)
        if causal or windowed:
            center = torch.arange(start, end)[:, None] + (Lk - Lq)
            if causal:
                scores = scores.masked_fill(key_pos > center, float("-inf"))
            if wl >= 0:
                scores = scores.masked_fill(key_pos < center - wl, float("-inf"))
            if wr >= 0:
                scores = scores.masked_fill(key_pos > center + wr, float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        probs = torch.nan_to_num(probs, nan=0.0)
        out[:, :, start:end] = probs @ vf
        if return_lse:
            lse[:, :, start:end] = torch.logsumexp(scores, dim=-1)
    return (out, lse) if return_lse else out


def cast_like(out_f32, dtype):
    """The reference's final `.to(q.dtype)` (_kernel.py:1208)."""
    return out_f32.to(dtype)


def flash_attn_func(q, k, v, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                    alibi_slopes=None, chunk=DEFAULT_CHUNK, rows=None, return_lse=False):
    """Heads-third q [B,Lq,Hq,D], k/v [B,Lk,Hkv,D] -> fp32 [B,Lq,Hq,D] (__init__.py:62-99).

    return_lse=True: (out, lse [B,Hq,Lq]) -- see flash_torch.
    """
    B, _, Hq, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    alibi = broadcast_alibi(alibi_slopes, B, Hq) if alibi_slopes is not None else None
    res = flash_torch(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale, causal, softcap,
                      window_size[0], window_size[1], alibi, chunk=chunk, rows=rows, return_lse=return_lse)
    if return_lse:
        return res[0].transpose(1, 2).contiguous(), res[1]
    return res.transpose(1, 2).contiguous()


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale=None, causal=False,
                           window_size=(-1, -1), softcap=0.0, alibi_slopes=None, chunk=DEFAULT_CHUNK,
                           return_lse=False):
    """Packed q [Tq,Hq,D], k/v [Tk,Hkv,D] -> fp32 [Tq,Hq,D] (__init__.py:102-183).

    Rows of empty query sequences do not exist; rows of sequences with no
    keys are 0 (lse -inf).  return_lse=True: (out, lse [Hq, Tq]).
    """
    cu_q = [int(x) for x in torch.as_tensor(cu_seqlens_q).tolist()]
    cu_k = [int(x) for x in torch.as_tensor(cu_seqlens_k).tolist()]
    Hq, D = q.shape[1], q.shape[2]
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    out = torch.zeros(q.shape, dtype=torch.float32)
    lse = torch.full((Hq, q.shape[0]), float("-inf"), dtype=torch.float32)
    for i in range(len(cu_q) - 1):
        qs = q[cu_q[i]:cu_q[i + 1]]
        ks = k[cu_k[i]:cu_k[i + 1]]
        vs = v[cu_k[i]:cu_k[i + 1]]
        if qs.shape[0] == 0:
            continue
        seq_alibi = alibi_slopes
        if alibi_slopes is not None and alibi_slopes.dim() == 2:
            seq_alibi = alibi_slopes[i]
        alibi = broadcast_alibi(seq_alibi, 1, Hq) if seq_alibi is not None else None
        if ks.shape[0] == 0:
            continue  # no keys: zero rows (lse stays -inf)
        o, l = flash_torch(qs.permute(1, 0, 2)[None], ks.permute(1, 0, 2)[None], vs.permute(1, 0, 2)[None],
                           scale, causal, softcap, window_size[0], window_size[1], alibi, chunk=chunk,
                           return_lse=True)
        out[cu_q[i]:cu_q[i + 1]] = o[0].permute(1, 0, 2)
        lse[:, cu_q[i]:cu_q[i + 1]] = l[0]
    return (out, lse) if return_lse else out


def attention_grads(q, k, v, dout, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                    alibi_slopes=None, dtype=torch.float32, dlse=None):
    """Gradients (dq, dk, dv) of sum(out * dout) (+ sum(lse * dlse) when dlse,
    [B,Hq,Lq], is given) for heads-third q [B,Lq,Hq,D], k/v [B,Lk,Hkv,D], by
    torch autograd through flash_torch (CPU, `dtype`).

    The reference has no backward (metal_flash_attn/__init__.py:3-4); these
    are the exact gradients of its forward math (_kernel.py:1165-1208), GQA
    heads summed through repeat_interleave's backward.
    """
    B, _, Hq, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    alibi = broadcast_alibi(alibi_slopes, B, Hq) if alibi_slopes is not None else None
    qd, kd, vd = (t.detach().cpu().to(dtype).requires_grad_(True) for t in (q, k, v))
    with torch.enable_grad():
        out, lse = flash_torch(qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2), scale, causal, softcap,
                               window_size[0], window_size[1], alibi, grad=True, dtype=dtype, return_lse=True)
        loss = (out * dout.detach().cpu().to(dtype).transpose(1, 2)).sum()
        if dlse is not None:
            # rows without a valid key have lse = -inf and no gradient
            ld = dlse.detach().cpu().to(dtype)
            loss = loss + torch.where(torch.isinf(lse), torch.zeros_like(lse), lse * ld).sum()
        loss.backward()
    return qd.grad, kd.grad, vd.grad


def attention_grads_varlen(q, k, v, dout, cu_seqlens_q, cu_seqlens_k, softmax_scale=None, causal=False,
                           window_size=(-1, -1), softcap=0.0, alibi_slopes=None, dtype=torch.float32):
    """attention_grads for packed varlen q [Tq,Hq,D], k/v [Tk,Hkv,D] (one
    sequence at a time, as flash_attn_varlen_func)."""
    cu_q = [int(x) for x in torch.as_tensor(cu_seqlens_q).tolist()]
    cu_k = [int(x) for x in torch.as_tensor(cu_seqlens_k).tolist()]
    dq = torch.zeros(q.shape, dtype=dtype)
    dk = torch.zeros(k.shape, dtype=dtype)
    dv = torch.zeros(v.shape, dtype=dtype)
    for i in range(len(cu_q) - 1):
        a, b, c, d = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
        if b == a or d == c:
            continue
        seq_alibi = alibi_slopes
        if alibi_slopes is not None and alibi_slopes.dim() == 2:
            seq_alibi = alibi_slopes[i]
        g = attention_grads(q[None, a:b], k[None, c:d], v[None, c:d], dout[None, a:b], softmax_scale, causal,
                            window_size, softcap, seq_alibi, dtype)
        dq[a:b], dk[c:d], dv[c:d] = g[0][0], g[1][0], g[2][0]
    return dq, dk, dv


def gather_pages(k_pages, block_table, seqlens_k):
    """Paged K (or V) -> packed [sum(seqlens_k), H, D] (CPU).

    k_pages: [num_pages, page_block_size, H, D]; key j of sequence b is row
    j % page_block_size of page block_table[b, j // page_block_size] -- the
    block_table convention of CUDA flash-attn 2.x's flash_attn_varlen_func
    (the API the reference mirrors and whose version its shim reports, 2.7.4,
    metal_flash_attn/_version.py:6; flash-attn itself is not a dependency and
    is absent here), which the reference rejects
    (metal_flash_attn/__init__.py:130-131).  With this gather, the paged call
    equals flash_attn_varlen_func on the packed K/V.
    """
    kp = k_pages.detach().cpu()
    bt = torch.as_tensor(block_table).cpu().long()
    page = kp.shape[1]
    parts = []
    for b, n in enumerate(int(x) for x in seqlens_k):
        j = torch.arange(n)
        parts.append(kp[bt[b, j // page], j % page])
    if not parts:
        return kp.new_zeros((0,) + tuple(kp.shape[2:]))
    return torch.cat(parts, dim=0)


def uneven_v_attention(query, key, value, attn_mask=None, is_causal=False, scale=None, enable_gqa=False,
                       q_chunk=4096):
    """[B, H, L, D] SDPA semantics with value head dim Dv != D (sdpa.py:86-130).

    Returns [B, Hq, Lq, Dv] in value.dtype.  Causal is top-left aligned (key j
    visible to query i iff j <= i), as in torch SDPA."""
    Hq, Hkv = query.shape[1], key.shape[1]
    if Hq != Hkv:
        if not (enable_gqa and Hkv != 0 and Hq % Hkv == 0):
            raise ValueError(f"SDPA query/kv head mismatch (Hq={Hq}, Hkv={Hkv}); pass enable_gqa=True")
        key = key.repeat_interleave(Hq // Hkv, dim=1)
        value = value.repeat_interleave(Hq // Hkv, dim=1)
    s = scale if scale is not None else 1.0 / math.sqrt(query.shape[-1])
    Lq, Lk = query.shape[-2], key.shape[-2]
    bias = None
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            bias = torch.zeros(attn_mask.shape, dtype=torch.float32).masked_fill(~attn_mask.cpu(), float("-inf"))
        else:
            bias = attn_mask.detach().cpu().float()
    key_t = key.detach().cpu().float().transpose(-2, -1)
    value_f = value.detach().cpu().float()
    outs = []
    for i in range(0, Lq, q_chunk):
        qi = query[..., i:i + q_chunk, :].detach().cpu().float()
        scores = torch.matmul(qi, key_t) * s
        if bias is not None:
            scores = scores + (bias[..., i:i + qi.shape[-2], :] if bias.shape[-2] == Lq else bias)
        if is_causal:
            qpos = torch.arange(i, i + qi.shape[-2]).unsqueeze(-1)
            kpos = torch.arange(Lk).unsqueeze(0)
            scores = scores.masked_fill(kpos > qpos, float("-inf"))
        probs = torch.nan_to_num(scores.softmax(dim=-1), nan=0.0)
        outs.append(torch.matmul(probs, value_f))
    return torch.cat(outs, dim=-2).to(value.dtype)
