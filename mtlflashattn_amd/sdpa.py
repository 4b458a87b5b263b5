"""Gated F.scaled_dot_product_attention patch for PyTorch-ROCm.

Same API and gate structure as the reference's patch
(metal_flash_attn/sdpa.py:133-193): `install(min_score_gb, min_seq,
fast_min_seq)` swaps F.scaled_dot_product_attention for `_sdpa`, which
routes a call to the HIP kernels when it is eligible and one of three gates
fires, and otherwise -- or when the kernel raises -- calls the original op.
It never crashes the caller.  Kill switch: MTLFLASHATTN_SDPA=off.

Gates (any one fires; thresholds from the arguments or the
MTLFLASHATTN_SDPA_* environment variables):
  1. "correctness-large-seq": max(Lq, Lk) >= min_seq (default 4096).  On MPS
     this shielded a stock-SDPA accuracy bug; on ROCm it keeps long sequences
     on the O(L*D)-memory kernel (faster than stock there for every dtype).
  2. "fast-tier": max(Lq, Lk) >= fast_min_seq (default 512) and the inputs
     take an MFMA path that beats stock ROCm SDPA: fp16/bf16 or fp32 with
     head_dim a multiple of 8.
  3. "oom-rescue": the Lq x Lk score matrix would take >= min_score_gb
     (default 12 GB) as fp16.
The fast-tier floor and tiers are re-derived for ROCm (the reference's 1024
floor and its tier set were measured against stock MPS SDPA): on MI355X with
torch 2.10 the HIP path matches or beats stock SDPA from 512 tokens in
fp16/bf16 (0.94-2.3x at 512, 1.0-2.0x beyond) and from 256 in fp32, and loses
below 512 in fp16/bf16 (host launch cost dominates there).

Value head dim != query/key head dim (the reference's uneven-V shield,
metal_flash_attn/sdpa.py:76-130, :145-149, an exact torch path): gated like
the even case and computed by the HIP kernel, exactly, on zero-padded head
dims (zero query/key columns add nothing to a score; padded value columns are
dropped), one launch per 128 value columns.  Calls the kernel cannot express
(attention masks, top-left causal with Lq != Lk) go to the original op, which
handles uneven V on ROCm.
"""
from __future__ import annotations

import math
import os

import torch
import torch.nn.functional as F

from ._kernel import MAX_HEAD_DIM, flash_attn_forward

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# tiers of the single HIP path that beat stock ROCm SDPA (see _select_tier)
_FAST_TIERS = frozenset({"hip", "hip-fp32"})

_orig = None
_min_score_bytes = None
_min_seq = None
_fast_min_seq = None


def _on_rocm_gpu(t) -> bool:
    return t.device.type == "cuda" and torch.version.hip is not None


def _select_tier(q, k, v) -> str:
    """Which flavour of the HIP path serves these inputs.

    "hip": 16-bit inputs, head_dim a multiple of 8 (MFMA bf16/f16 path);
    "hip-fp32": fp32 inputs (fp32 MFMA, about 16x lower peak);
    "hip-padded": head_dim not a multiple of 8 (inputs are zero-padded first).
    """
    if q.shape[-1] % 8 != 0:
        return "hip-padded"
    if q.dtype == torch.float32:
        return "hip-fp32"
    return "hip"


def _gate(B, Hq, Lq, Lk, tier):
    """Return (eligible, reason) for the three routing gates."""
    maxlen = max(Lq, Lk)
    if maxlen >= _min_seq:
        return True, "correctness-large-seq"
    if maxlen >= _fast_min_seq and tier in _FAST_TIERS:
        return True, "fast-tier"
    score_bytes = B * Hq * Lq * Lk * 2
    if score_bytes >= _min_score_bytes:
        return True, "oom-rescue"
    return False, f"fits({score_bytes / 1024 ** 3:.2f}GB)"


def _eligibility(q, k, v, attn_mask, dropout_p, is_causal):
    """Return (eligible, reason); reason names the disqualifying gate (sdpa.py:33-73)."""
    if not _on_rocm_gpu(q):
        return False, "not-rocm"
    if attn_mask is not None:
        return False, "attn_mask"
    if dropout_p:
        return False, "dropout"
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return False, f"ndim({q.dim()})"
    if q.dtype not in _SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        return False, f"dtype({q.dtype})"
    D = q.shape[-1]
    if D > MAX_HEAD_DIM or k.shape[-1] != D or v.shape[-1] < 1:
        return False, f"head_dim({D})"
    Hq, Hkv = q.shape[1], k.shape[1]
    if Hkv == 0 or Hq % Hkv != 0:
        return False, f"heads({Hq}/{Hkv})"
    if not (q.shape[0] == k.shape[0] == v.shape[0]) or v.shape[1] != Hkv:
        return False, "batch-or-heads-mismatch"
    if k.shape[2] != v.shape[2]:
        return False, "kv-len-mismatch"
    # fp32 calls that autograd will differentiate stay on stock SDPA (its
    # gradients flow): the HIP fp32 backward is exact but runs on the vector
    # ALU, not the matrix cores
    if q.dtype == torch.float32 and torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return False, "grad-fp32"
    Lq, Lk = q.shape[2], k.shape[2]
    # SDPA's is_causal is TOP-LEFT aligned, the kernel's BOTTOM-RIGHT: equal only when Lq == Lk
    if is_causal and Lq != Lk:
        return False, "causal-cross-length"
    return _gate(q.shape[0], Hq, Lq, Lk, _select_tier(q, k, v))


def _uneven_v(q, k, v, scale, causal):
    """[B,H,L,D] attention with value head dim Dv != D on the HIP kernel: the
    narrower of (q/k, v) is zero-padded to the wider, Dv in blocks of at most
    MAX_HEAD_DIM columns (one launch each); exact (zero columns add nothing)."""
    D, Dv = q.shape[-1], v.shape[-1]
    outs = []
    for c0 in range(0, Dv, MAX_HEAD_DIM):
        vc = v[..., c0:c0 + MAX_HEAD_DIM]
        w = max(D, vc.shape[-1])
        qp, kp = (F.pad(t, (0, w - D)) if w > D else t for t in (q, k))
        vp = F.pad(vc, (0, w - vc.shape[-1])) if w > vc.shape[-1] else vc
        outs.append(flash_attn_forward(qp, kp, vp, scale=scale, causal=causal)[..., :vc.shape[-1]])
    return outs[0] if len(outs) == 1 else torch.cat(outs, dim=-1)


def _sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, **kwargs):
    eligible, _ = _eligibility(query, key, value, attn_mask, dropout_p, is_causal)
    if eligible:
        try:
            s = scale if scale is not None else 1.0 / math.sqrt(query.shape[-1])
            if value.shape[-1] != query.shape[-1]:
                return _uneven_v(query, key, value, s, is_causal)
            return flash_attn_forward(query, key, value, scale=s, causal=is_causal)
        except Exception as e:  # never crash: fall back to stock SDPA
            print(f"[mtlflashattn_amd/sdpa] kernel fell back ({e}); using stock SDPA")
    return _orig(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal, scale=scale,
                 **kwargs)


def install(min_score_gb=None, min_seq=None, fast_min_seq=None):
    """Patch F.scaled_dot_product_attention. Returns True if newly installed (sdpa.py:154-179)."""
    global _orig, _min_score_bytes, _min_seq, _fast_min_seq
    if _orig is not None:
        return False
    if os.environ.get("MTLFLASHATTN_SDPA", "auto").lower() in ("off", "0", "false"):
        return False
    if min_score_gb is None:
        min_score_gb = float(os.environ.get("MTLFLASHATTN_SDPA_MIN_GB", "12"))
    if min_seq is None:
        min_seq = int(os.environ.get("MTLFLASHATTN_SDPA_MIN_SEQ", "4096"))
    if fast_min_seq is None:
        fast_min_seq = int(os.environ.get("MTLFLASHATTN_SDPA_FAST_MIN_SEQ", "512"))
    _min_score_bytes = int(min_score_gb * (1024 ** 3))
    _min_seq = min_seq
    _fast_min_seq = fast_min_seq
    _orig = F.scaled_dot_product_attention
    F.scaled_dot_product_attention = _sdpa
    torch.nn.functional.scaled_dot_product_attention = _sdpa
    return True


def uninstall():
    """Restore the original op. Returns True if a patch was removed (sdpa.py:182-193)."""
    global _orig, _min_score_bytes, _min_seq, _fast_min_seq
    if _orig is None:
        return False
    F.scaled_dot_product_attention = _orig
    torch.nn.functional.scaled_dot_product_attention = _orig
    _orig = None
    _min_score_bytes = None
    _min_seq = None
    _fast_min_seq = None
    return True
