"""ctypes binding of the C ABI in include/mfa.h (libmtlfa_hip.so).

This module replaces the reference's per-tier shader libraries and their
cached parameter tensors (metal_flash_attn/_kernel.py:716-925, :1211-1272):
the kernel parameters travel in one POD struct (`MfaFwdParams`) that the
library copies into the kernel arguments, so a call allocates no device
memory besides the output the caller provides.

The library must be built in-tree first (`python -m mtlflashattn_amd._build`,
or `__graft_entry__.build()`); loading fails loudly otherwise.  torch is
imported before the library is opened so that the library binds to the HIP
runtime torch already loaded (both carry the soname libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must load torch's HIP runtime first)

from ._build import LIB_PATH

MFA_ABI_VERSION = 7
MFA_DTYPE_F16 = 0
MFA_DTYPE_BF16 = 1
MFA_DTYPE_F32 = 2
MFA_OK = 0
MFA_ERR_INVALID = -1
MFA_ERR_UNSUPPORTED = -2
MFA_ERR_LAUNCH = -3
MFA_TILE_AUTO = 0
MFA_TILE_256 = 1
MFA_TILE_PINGPONG = 2
MFA_TILE_PINGPONG256 = 3

DTYPE_CODES = {
    torch.float16: MFA_DTYPE_F16,
    torch.bfloat16: MFA_DTYPE_BF16,
    torch.float32: MFA_DTYPE_F32,
}

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_ptr = ctypes.c_void_p


class MfaFwdParams(ctypes.Structure):
    """Mirror of `mfa_fwd_params` (include/mfa.h)."""

    _fields_ = [
        ("q", _c_ptr), ("k", _c_ptr), ("v", _c_ptr), ("o", _c_ptr),
        ("q_batch_stride", _c_i64), ("q_seq_stride", _c_i64), ("q_head_stride", _c_i64),
        ("k_batch_stride", _c_i64), ("k_seq_stride", _c_i64), ("k_head_stride", _c_i64),
        ("v_batch_stride", _c_i64), ("v_seq_stride", _c_i64), ("v_head_stride", _c_i64),
        ("o_batch_stride", _c_i64), ("o_seq_stride", _c_i64), ("o_head_stride", _c_i64),
        ("batch", _c_i32), ("heads_q", _c_i32), ("heads_kv", _c_i32),
        ("seqlen_q", _c_i32), ("seqlen_k", _c_i32), ("head_dim", _c_i32),
        ("cu_seqlens_q", _c_ptr), ("cu_seqlens_k", _c_ptr),
        ("scale", ctypes.c_float), ("softcap", ctypes.c_float),
        ("window_left", _c_i32), ("window_right", _c_i32), ("causal", _c_i32),
        ("alibi_slopes", _c_ptr), ("alibi_batch_stride", _c_i32),
        ("dtype_in", _c_i32), ("dtype_out", _c_i32), ("tile_hint", _c_i32),
        ("softmax_lse", _c_ptr), ("lse_batch_stride", _c_i64), ("lse_head_stride", _c_i64),
        ("block_table", _c_ptr), ("block_table_batch_stride", _c_i64),
        ("page_block_size", _c_i32), ("num_pages", _c_i32), ("varlen_no_single_rows", _c_i32),
    ]


class MfaBwdParams(ctypes.Structure):
    """Mirror of `mfa_bwd_params` (include/mfa.h)."""

    _fields_ = [
        ("fwd", MfaFwdParams),
        ("dout", _c_ptr), ("do_batch_stride", _c_i64), ("do_seq_stride", _c_i64), ("do_head_stride", _c_i64),
        ("dq", _c_ptr), ("dq_batch_stride", _c_i64), ("dq_seq_stride", _c_i64), ("dq_head_stride", _c_i64),
        ("dk", _c_ptr), ("dk_batch_stride", _c_i64), ("dk_seq_stride", _c_i64), ("dk_head_stride", _c_i64),
        ("dv", _c_ptr), ("dv_batch_stride", _c_i64), ("dv_seq_stride", _c_i64), ("dv_head_stride", _c_i64),
        ("dtype_grad", _c_i32), ("reserved", _c_i32), ("dlse", _c_ptr),
    ]


class MfaLaunchInfo(ctypes.Structure):
    """Mirror of `mfa_launch_info` (include/mfa.h)."""

    _fields_ = [
        ("grid_x", _c_i32), ("block_x", _c_i32), ("rows_per_block", _c_i32),
        ("keys_per_block", _c_i32), ("lds_bytes", _c_i32),
        ("kernel_name", ctypes.c_char * 96),
    ]


class HipLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale or failed a call."""


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return os.environ.get("MTLFLASHATTN_HIP_LIB", LIB_PATH)


def load():
    """Open libmtlfa_hip.so once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise HipLibraryError(
                f"mtlflashattn_amd: HIP kernel library not found at {path}; build it with "
                "`python -m mtlflashattn_amd._build` (or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:
            raise HipLibraryError(f"mtlflashattn_amd: cannot load {path}: {e}") from e
        lib.mfa_abi_version.restype = ctypes.c_int
        lib.mfa_abi_version.argtypes = []
        lib.mfa_params_size.restype = ctypes.c_int
        lib.mfa_params_size.argtypes = []
        lib.mfa_last_error.restype = ctypes.c_char_p
        lib.mfa_last_error.argtypes = []
        lib.mfa_supported.restype = ctypes.c_int
        lib.mfa_supported.argtypes = [_c_i32, _c_i32]
        lib.mfa_fwd.restype = ctypes.c_int
        lib.mfa_fwd.argtypes = [ctypes.POINTER(MfaFwdParams), _c_ptr]
        lib.mfa_fwd_launch_info.restype = ctypes.c_int
        lib.mfa_fwd_launch_info.argtypes = [ctypes.POINTER(MfaFwdParams), ctypes.POINTER(MfaLaunchInfo)]
        lib.mfa_fwd_split_keys.restype = _c_i32
        lib.mfa_fwd_split_keys.argtypes = [ctypes.POINTER(MfaFwdParams)]
        lib.mfa_fwd_workspace_bytes.restype = ctypes.c_int64
        lib.mfa_fwd_workspace_bytes.argtypes = [ctypes.POINTER(MfaFwdParams), _c_i32]
        lib.mfa_fwd_splitkv.restype = ctypes.c_int
        lib.mfa_fwd_splitkv.argtypes = [ctypes.POINTER(MfaFwdParams), _c_i32, _c_ptr, ctypes.c_int64, _c_ptr]
        lib.mfa_fwd_splitkv_static.restype = ctypes.c_int
        lib.mfa_fwd_splitkv_static.argtypes = [ctypes.POINTER(MfaFwdParams), _c_i32, _c_ptr]
        lib.mfa_bwd_params_size.restype = ctypes.c_int
        lib.mfa_bwd_params_size.argtypes = []
        lib.mfa_bwd_supported.restype = ctypes.c_int
        lib.mfa_bwd_supported.argtypes = [_c_i32, _c_i32]
        lib.mfa_bwd_workspace_bytes.restype = ctypes.c_int64
        lib.mfa_bwd_workspace_bytes.argtypes = [ctypes.POINTER(MfaBwdParams)]
        lib.mfa_bwd.restype = ctypes.c_int
        lib.mfa_bwd.argtypes = [ctypes.POINTER(MfaBwdParams), _c_ptr, ctypes.c_int64, _c_ptr]
        if lib.mfa_abi_version() != MFA_ABI_VERSION:
            raise HipLibraryError(
                f"mtlflashattn_amd: {path} has ABI {lib.mfa_abi_version()}, expected {MFA_ABI_VERSION}; rebuild it"
            )
        if lib.mfa_bwd_params_size() != ctypes.sizeof(MfaBwdParams):
            raise HipLibraryError(
                f"mtlflashattn_amd: mfa_bwd_params is {lib.mfa_bwd_params_size()} bytes in {path} but "
                f"{ctypes.sizeof(MfaBwdParams)} in the ctypes mirror; rebuild it"
            )
        if lib.mfa_params_size() != ctypes.sizeof(MfaFwdParams):
            raise HipLibraryError(
                f"mtlflashattn_amd: mfa_fwd_params is {lib.mfa_params_size()} bytes in {path} but "
                f"{ctypes.sizeof(MfaFwdParams)} in the ctypes mirror; rebuild it"
            )
        _lib = lib
        return lib


def is_loaded() -> bool:
    return _lib is not None


def last_error() -> str:
    return load().mfa_last_error().decode(errors="replace")


def supported(dtype: torch.dtype, head_dim: int) -> bool:
    code = DTYPE_CODES.get(dtype)
    return code is not None and bool(load().mfa_supported(code, int(head_dim)))


def fwd(params: MfaFwdParams, stream: int) -> None:
    lib = load()
    rc = lib.mfa_fwd(ctypes.byref(params), _c_ptr(stream))
    if rc != MFA_OK:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_fwd failed ({rc})")


def split_keys(params: MfaFwdParams) -> int:
    """The library's split-KV chunk size for this call (0: no split)."""
    return int(load().mfa_fwd_split_keys(ctypes.byref(params)))


def workspace_bytes(params: MfaFwdParams, chunk: int) -> int:
    lib = load()
    n = lib.mfa_fwd_workspace_bytes(ctypes.byref(params), int(chunk))
    if n < 0:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_fwd_workspace_bytes failed ({n})")
    return int(n)


def fwd_splitkv(params: MfaFwdParams, chunk: int, workspace: int, workspace_bytes_: int, stream: int) -> None:
    lib = load()
    rc = lib.mfa_fwd_splitkv(ctypes.byref(params), int(chunk), _c_ptr(workspace), int(workspace_bytes_),
                             _c_ptr(stream))
    if rc != MFA_OK:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_fwd_splitkv failed ({rc})")


def fwd_splitkv_static(params: MfaFwdParams, chunk: int, stream: int) -> None:
    """mfa_fwd_splitkv with the library's static per-GPU scratch as workspace
    (allocates nothing; calls that overlap on one GPU race)."""
    lib = load()
    rc = lib.mfa_fwd_splitkv_static(ctypes.byref(params), int(chunk), _c_ptr(stream))
    if rc != MFA_OK:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_fwd_splitkv_static failed ({rc})")


def bwd_workspace_bytes(params: MfaBwdParams) -> int:
    lib = load()
    n = lib.mfa_bwd_workspace_bytes(ctypes.byref(params))
    if n < 0:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_bwd_workspace_bytes failed ({n})")
    return int(n)


def bwd(params: MfaBwdParams, workspace: int, workspace_bytes_: int, stream: int) -> None:
    lib = load()
    rc = lib.mfa_bwd(ctypes.byref(params), _c_ptr(workspace), int(workspace_bytes_), _c_ptr(stream))
    if rc != MFA_OK:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_bwd failed ({rc})")


def launch_info(params: MfaFwdParams) -> MfaLaunchInfo:
    lib = load()
    info = MfaLaunchInfo()
    rc = lib.mfa_fwd_launch_info(ctypes.byref(params), ctypes.byref(info))
    if rc != MFA_OK:
        raise HipLibraryError(lib.mfa_last_error().decode(errors="replace") or f"mfa_fwd_launch_info failed ({rc})")
    return info
