"""The C ABI of libmtlfa_hip.so (include/mfa.h) on CPU: the library loads,
exports every function the header declares, agrees with the ctypes mirror of
its parameter struct, and rejects invalid requests with an error code and a
message before anything is launched.  No call here reaches a GPU: every
mfa_fwd call fails validation or has an empty problem."""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from mtlflashattn_amd import _build, _hip, _kernel

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mfa.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    return _hip.load()


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mfa_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_entry_points():
    assert set(declared_functions()) >= {"mfa_abi_version", "mfa_last_error", "mfa_supported", "mfa_fwd",
                                         "mfa_fwd_launch_info", "mfa_params_size", "mfa_fwd_split_keys",
                                         "mfa_fwd_workspace_bytes", "mfa_fwd_splitkv"}


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_build.LIB_PATH)
    for name in declared_functions():
        assert hasattr(raw, name), f"{name} declared in include/mfa.h but not exported"


def test_abi_version_and_struct_size(lib):
    assert lib.mfa_abi_version() == _hip.MFA_ABI_VERSION
    assert lib.mfa_params_size() == ctypes.sizeof(_hip.MfaFwdParams)
    src = open(HEADER).read()
    assert f"#define MFA_ABI_VERSION {_hip.MFA_ABI_VERSION}" in src
    for name in ("MFA_DTYPE_F16", "MFA_DTYPE_BF16", "MFA_DTYPE_F32", "MFA_ERR_INVALID", "MFA_ERR_UNSUPPORTED",
                 "MFA_TILE_AUTO", "MFA_TILE_256", "MFA_TILE_PINGPONG"):
        val = int(re.search(rf"#define {name} (-?\d+)", src).group(1))
        assert val == getattr(_hip, name)


def test_supported_table(lib):
    for dt in (_hip.MFA_DTYPE_F16, _hip.MFA_DTYPE_BF16, _hip.MFA_DTYPE_F32):
        assert all(lib.mfa_supported(dt, d) for d in (8, 32, 64, 96, 128))
        assert not lib.mfa_supported(dt, 130) and not lib.mfa_supported(dt, 33) and not lib.mfa_supported(dt, 0)
    assert not lib.mfa_supported(7, 64)
    # the backward: the same table (fp32 on its vector-ALU kernels)
    for dt in (_hip.MFA_DTYPE_F16, _hip.MFA_DTYPE_BF16, _hip.MFA_DTYPE_F32):
        assert all(lib.mfa_bwd_supported(dt, d) for d in (8, 32, 64, 96, 128))
        assert not lib.mfa_bwd_supported(dt, 130) and not lib.mfa_bwd_supported(dt, 33)
    assert not lib.mfa_bwd_supported(7, 64)


def good_params(B=1, L=256, H=4, Hkv=4, D=64, dtype=_hip.MFA_DTYPE_BF16):
    p = _hip.MfaFwdParams()
    p.q = p.k = p.v = p.o = 4096
    p.q_batch_stride, p.q_seq_stride, p.q_head_stride = L * H * D, H * D, D
    p.k_batch_stride, p.k_seq_stride, p.k_head_stride = L * Hkv * D, Hkv * D, D
    p.v_batch_stride, p.v_seq_stride, p.v_head_stride = L * Hkv * D, Hkv * D, D
    p.o_batch_stride, p.o_seq_stride, p.o_head_stride = L * H * D, H * D, D
    p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim = B, H, Hkv, L, L, D
    p.scale, p.softcap = 0.125, 0.0
    p.window_left = p.window_right = -1
    p.dtype_in = p.dtype_out = dtype
    return p


@pytest.mark.parametrize("mutate,code,msg", [
    (lambda p: setattr(p, "dtype_in", 9), _hip.MFA_ERR_INVALID, "dtype_in"),
    (lambda p: setattr(p, "dtype_out", _hip.MFA_DTYPE_F16), _hip.MFA_ERR_INVALID, "dtype_out"),
    (lambda p: setattr(p, "head_dim", 160), _hip.MFA_ERR_UNSUPPORTED, "head_dim"),
    (lambda p: setattr(p, "head_dim", 36), _hip.MFA_ERR_UNSUPPORTED, "multiple of 8"),
    (lambda p: setattr(p, "heads_kv", 3), _hip.MFA_ERR_INVALID, "must divide"),
    (lambda p: setattr(p, "softcap", -1.0), _hip.MFA_ERR_INVALID, "softcap"),
    (lambda p: setattr(p, "window_left", -2), _hip.MFA_ERR_INVALID, "window"),
    (lambda p: setattr(p, "q", 4098), _hip.MFA_ERR_INVALID, "aligned"),
    (lambda p: setattr(p, "k_seq_stride", 68), _hip.MFA_ERR_INVALID, "strides"),
    # 16-bit O is stored in 16-byte row pieces: o strides of 4 (not 8) elements are refused
    (lambda p: setattr(p, "o_seq_stride", 4 * 64 + 4), _hip.MFA_ERR_INVALID, "o strides"),
    # a padded o head stride (D + 4) on a single-row grouped-query decode, whose
    # packed rows are addressed through the head stride
    (lambda p: (setattr(p, "seqlen_q", 1), setattr(p, "heads_kv", 1), setattr(p, "o_head_stride", 68),
                setattr(p, "o_seq_stride", 4 * 68), setattr(p, "o_batch_stride", 4 * 68)),
     _hip.MFA_ERR_INVALID, "o strides"),
    (lambda p: setattr(p, "o", None), _hip.MFA_ERR_INVALID, "NULL"),
    (lambda p: setattr(p, "cu_seqlens_q", 256), _hip.MFA_ERR_INVALID, "cu_seqlens"),
    (lambda p: setattr(p, "tile_hint", 4), _hip.MFA_ERR_INVALID, "tile_hint"),
    (lambda p: (setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG256), setattr(p, "head_dim", 96),
                setattr(p, "q_head_stride", 96)), _hip.MFA_ERR_UNSUPPORTED, "ping-pong"),
    (lambda p: (setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG), setattr(p, "dtype_in", _hip.MFA_DTYPE_F32),
                setattr(p, "dtype_out", _hip.MFA_DTYPE_F32)), _hip.MFA_ERR_UNSUPPORTED, "ping-pong"),
    (lambda p: (setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG), setattr(p, "head_dim", 80),
                setattr(p, "q_head_stride", 80)), _hip.MFA_ERR_UNSUPPORTED, "ping-pong"),
    (lambda p: setattr(p, "k_seq_stride", -64), _hip.MFA_ERR_INVALID, "sequence strides"),
    (lambda p: (setattr(p, "block_table", 256), setattr(p, "page_block_size", 256), setattr(p, "num_pages", 4),
                setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG)), _hip.MFA_ERR_UNSUPPORTED, "block_table"),
    (lambda p: setattr(p, "seqlen_k", -1), _hip.MFA_ERR_INVALID, "negative"),
    (lambda p: (setattr(p, "block_table", 256), setattr(p, "page_block_size", 100), setattr(p, "num_pages", 4)),
     _hip.MFA_ERR_INVALID, "page_block_size"),
    (lambda p: (setattr(p, "block_table", 256), setattr(p, "page_block_size", 256)), _hip.MFA_ERR_INVALID,
     "num_pages"),
    (lambda p: (setattr(p, "block_table", 256), setattr(p, "page_block_size", 512), setattr(p, "num_pages", 4),
                setattr(p, "block_table_batch_stride", -1)), _hip.MFA_ERR_INVALID, "block_table_batch_stride"),
    (lambda p: (setattr(p, "softmax_lse", 256), setattr(p, "lse_head_stride", -1)), _hip.MFA_ERR_INVALID,
     "lse strides"),
])
def test_invalid_requests_are_rejected_before_launch(lib, mutate, code, msg):
    p = good_params()
    mutate(p)
    assert lib.mfa_fwd(ctypes.byref(p), None) == code
    assert msg in lib.mfa_last_error().decode()
    with pytest.raises(_hip.HipLibraryError, match=msg):
        _hip.fwd(p, 0)


def test_null_params(lib):
    assert lib.mfa_fwd(None, None) == _hip.MFA_ERR_INVALID
    assert b"NULL" in lib.mfa_last_error()


def test_empty_problem_is_a_no_op(lib):
    p = good_params(B=0)
    assert lib.mfa_fwd(ctypes.byref(p), None) == _hip.MFA_OK
    assert lib.mfa_last_error() == b""
    p = good_params()
    p.seqlen_q = 0
    assert lib.mfa_fwd(ctypes.byref(p), None) == _hip.MFA_OK


def test_launch_geometry_of_the_baseline_configs(lib):
    bf = torch.empty(1, 8192, 16, 64, dtype=torch.bfloat16)
    info = _kernel.launch_info(bf, bf, bf)
    # config 2 fills the chip with 512-row ping-pong tiles (8 wavefronts)
    assert info.block_x == 512 and info.grid_x * info.rows_per_block >= 8192 * 16
    assert info.kernel_name.startswith(b"mfa_fwd16pp<bf16,d64")
    # XCD-grouped schedule: grid is a multiple of 8 and covers every (head, tile)
    assert info.grid_x % 8 == 0
    # too few 512-row tiles for 256 CUs: the 256-row kernel
    small = torch.empty(1, 2048, 16, 64, dtype=torch.bfloat16)
    info = _kernel.launch_info(small, small, small)
    assert info.block_x == 256 and info.kernel_name.startswith(b"mfa_fwd16<bf16,d64")
    # many short or single-row sequences: half-empty 512-row tiles lose to the
    # 256-row kernel even on a full grid (HBM-bound shapes)
    for lq, lk in ((256, 256), (1, 4096), (768, 768)):
        qs = torch.empty(64, lq, 16, 64, dtype=torch.bfloat16)
        ks = torch.empty(64, lk, 16, 64, dtype=torch.bfloat16)
        assert _kernel.launch_info(qs, ks, ks).block_x == 256, (lq, lk)
        assert _kernel.launch_info(qs, ks, ks, causal=True).block_x == 256, (lq, lk)
    long = torch.empty(8, 1280, 16, 64, dtype=torch.bfloat16)
    assert _kernel.launch_info(long, long, long).block_x == 512
    # the tile hint overrides the automatic choice
    p = good_params(L=2048, H=16)
    p.tile_hint = _hip.MFA_TILE_PINGPONG
    li = _hip.launch_info(p)
    assert li.block_x == 512 and li.rows_per_block == 512
    p.tile_hint = _hip.MFA_TILE_256
    assert _hip.launch_info(p).block_x == 256
    p.tile_hint = _hip.MFA_TILE_PINGPONG256
    li = _hip.launch_info(p)
    assert li.block_x == 512 and li.rows_per_block == 256
    # causal: when every 512-row tile would run at once (256 of them here) the
    # heaviest sets the time, and the 256-row ping-pong tiles are chosen
    c8k = torch.empty(1, 8192, 16, 64, dtype=torch.bfloat16)
    li = _kernel.launch_info(c8k, c8k, c8k, causal=True)
    assert li.block_x == 512 and li.rows_per_block == 256, li.kernel_name
    assert _kernel.launch_info(c8k, c8k, c8k).rows_per_block == 512  # non-causal: equal tiles
    # sliding windows, and causal calls with a bias, run on the 4-wavefront kernel
    assert _kernel.launch_info(c8k, c8k, c8k, window_left=1024, window_right=0).block_x == 256
    assert _kernel.launch_info(c8k, c8k, c8k, causal=True, softcap=30.0).block_x == 256
    assert _kernel.launch_info(c8k, c8k, c8k, softcap=30.0).block_x == 512  # equal tiles: ping-pong
    # causal with few 512-row tiles per head over several rounds: 4-wavefront kernel
    c4k = torch.empty(1, 4096, 16, 64, dtype=torch.bfloat16)  # 128 tiles of 512 rows, 256 of 256
    li = _kernel.launch_info(c4k, c4k, c4k, causal=True)
    assert li.block_x == 512 and li.rows_per_block == 256
    assert _kernel.launch_info(c4k, c4k, c4k).rows_per_block == 256  # non-causal: the same tiles
    assert _kernel.launch_info(c4k, c4k, c4k, softcap=30.0).block_x == 256  # bias: 4-wavefront kernel
    c1k = torch.empty(8, 1024, 32, 64, dtype=torch.bfloat16)
    assert _kernel.launch_info(c1k, c1k, c1k, causal=True).block_x == 256
    assert _kernel.launch_info(c1k, c1k, c1k).block_x == 512  # non-causal: ping-pong
    for D in (32, 64):  # one 512-row tile per head: the 4-wavefront kernel
        c512 = torch.empty(32, 512, 16, D, dtype=torch.bfloat16)
        assert _kernel.launch_info(c512, c512, c512).block_x == 256
        one_round = torch.empty(32, 512, 8, D, dtype=torch.bfloat16)  # 256 tiles of 512 rows, causal
        assert _kernel.launch_info(one_round, one_round, one_round, causal=True).block_x == 256
        # 3/4 to one round of 256-row tiles: the 256-row ping-pong tiles
        for B, L, causal in ((16, 512, False), (12, 512, True), (10, 768, False)):
            t = torch.empty(B, L, 8, D, dtype=torch.bfloat16)
            li = _kernel.launch_info(t, t, t, causal=causal)
            assert li.block_x == 512 and li.rows_per_block == 256, (B, L, causal, li.kernel_name)
        for B, L in ((18, 512), (11, 768), (8, 512)):  # past one round; under 3/4 of one
            t = torch.empty(B, L, 8, D, dtype=torch.bfloat16)
            assert _kernel.launch_info(t, t, t).block_x == 256, (B, L)
    c16k = torch.empty(1, 16384, 16, 64, dtype=torch.bfloat16)  # 512 tiles: balanced by the schedule
    assert _kernel.launch_info(c16k, c16k, c16k, causal=True).rows_per_block == 512
    f16 = torch.empty(1, 8192, 16, 128, dtype=torch.float16)
    info = _kernel.launch_info(f16, f16, f16, causal=True)  # dense, 512 tiles of 256 rows: ping-pong
    assert info.kernel_name.startswith(b"mfa_fwd16pp<f16,d128") and info.rows_per_block == 256
    # head dim 128: narrow windows, windows under a soft-cap / ALiBi and small
    # grids stay on the 4-wavefront kernel; windows of >= 2048 keys take the
    # ping-pong tiles
    assert _kernel.launch_info(f16, f16, f16, window_left=256, window_right=256).kernel_name.startswith(
        b"mfa_fwd16<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, window_left=1024, window_right=1024).kernel_name.startswith(
        b"mfa_fwd16pp<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, causal=True, window_left=4096, window_right=0).kernel_name.startswith(
        b"mfa_fwd16pp<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, causal=True, window_left=1024, window_right=0).kernel_name.startswith(
        b"mfa_fwd16<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, causal=True, softcap=30.0, window_left=4096,
                               window_right=0).kernel_name.startswith(b"mfa_fwd16<f16,d128")
    # dense rows: >= 2 tiles of 256 rows per head go to the ping-pong tiles,
    # >= 8 when causal
    def d128(B, L, causal):
        t = torch.empty(B, L, 16, 128, dtype=torch.float16)
        return _kernel.launch_info(t, t, t, causal=causal).kernel_name
    assert d128(64, 256, False).startswith(b"mfa_fwd16<f16,d128")  # 1 tile per head
    assert d128(32, 512, False).startswith(b"mfa_fwd16pp<f16,d128")
    assert d128(16, 1024, True).startswith(b"mfa_fwd16<f16,d128")  # 4 tiles per head
    assert d128(16, 1536, True).startswith(b"mfa_fwd16<f16,d128")  # 6
    assert d128(8, 2048, True).startswith(b"mfa_fwd16pp<f16,d128")  # 8
    assert d128(32, 384, False).startswith(b"mfa_fwd16<f16,d128")  # 512 padded rows against 384
    # packed grouped-query tiles (4 query heads per K/V head): rows of >= 512
    # positions, 1280 when causal
    def gqa(B, L, causal):
        q = torch.empty(B, L, 32, 128, dtype=torch.float16)
        kv = torch.empty(B, L, 8, 128, dtype=torch.float16)
        return _kernel.launch_info(q, kv, kv, causal=causal).kernel_name
    assert gqa(32, 512, False).startswith(b"mfa_fwd16pp<f16,d128")
    assert gqa(64, 256, False).startswith(b"mfa_fwd16<f16,d128")
    assert gqa(16, 1024, True).startswith(b"mfa_fwd16<f16,d128")
    assert gqa(12, 1536, True).startswith(b"mfa_fwd16pp<f16,d128")
    # windows: >= 1536 keys wide, >= 512 on packed grouped-query tiles
    q4 = torch.empty(4, 4096, 32, 128, dtype=torch.float16)
    kv4 = torch.empty(4, 4096, 8, 128, dtype=torch.float16)
    assert _kernel.launch_info(q4, kv4, kv4, window_left=256, window_right=256).kernel_name.startswith(
        b"mfa_fwd16pp<f16,d128")
    assert _kernel.launch_info(q4, kv4, kv4, window_left=200, window_right=200).kernel_name.startswith(
        b"mfa_fwd16<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, window_left=768, window_right=767).kernel_name.startswith(
        b"mfa_fwd16pp<f16,d128")
    assert _kernel.launch_info(f16, f16, f16, window_left=512, window_right=511).kernel_name.startswith(
        b"mfa_fwd16<f16,d128")
    small128 = torch.empty(1, 2048, 16, 128, dtype=torch.float16)
    assert _kernel.launch_info(small128, small128, small128).kernel_name.startswith(b"mfa_fwd16<f16,d128")
    big = torch.empty(1, 32768, 16, 128, dtype=torch.bfloat16)
    info = _kernel.launch_info(big, big, big, causal=True, softcap=30.0, alibi=True, window_left=2048, window_right=0)
    assert info.kernel_name.endswith(b"+bias")
    f32 = torch.empty(1, 512, 2, 64, dtype=torch.float32)
    info = _kernel.launch_info(f32, f32, f32)
    assert info.kernel_name.startswith(b"mfa_fwd32<f32,d64")
    assert info.grid_x == 2 * (512 // info.rows_per_block)  # linear schedule: heads x tiles


def test_varlen_d128_kernel_choice(lib):
    # varlen calls give the longest sequence only: at head dim 128 the
    # ping-pong tiles need >= 5 tiles of 256 rows non-causal, 16 causal;
    # grouped-query calls whose tiles pack 2, 4 or 8 query heads need rows
    # of >= 1024 positions (1280 causal)
    def varlen(nseq, longest, Hq, Hkv, causal):
        p = good_params(B=nseq, L=longest, H=Hq, Hkv=Hkv, D=128)
        p.q_batch_stride = p.k_batch_stride = p.v_batch_stride = p.o_batch_stride = 0
        p.cu_seqlens_q = p.cu_seqlens_k = 256  # placeholder: planning reads no device memory
        p.causal = int(causal)
        return _hip.launch_info(p).kernel_name
    assert varlen(8, 3501, 32, 8, False).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(8, 3501, 32, 8, True).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(32, 2048, 32, 8, False).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(64, 1024, 32, 8, True).startswith(b"mfa_fwd16<bf16,d128")
    assert varlen(64, 1024, 32, 8, False).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(64, 960, 32, 8, False).startswith(b"mfa_fwd16<bf16,d128")  # 15 tiles of 64
    assert varlen(64, 1280, 32, 8, True).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(8, 3501, 16, 16, True).startswith(b"mfa_fwd16<bf16,d128")  # one head per K/V head: 14 < 16
    assert varlen(4, 8192, 16, 16, True).startswith(b"mfa_fwd16pp<bf16,d128")
    assert varlen(64, 1024, 16, 16, False).startswith(b"mfa_fwd16<bf16,d128")  # 4 tiles
    assert varlen(32, 1280, 16, 16, False).startswith(b"mfa_fwd16pp<bf16,d128")  # 5 tiles
    assert varlen(16, 2048, 16, 16, True).startswith(b"mfa_fwd16<bf16,d128")  # causal: 8 < 16
    # the Python helper plans the same call (config 4's geometry)
    q = torch.empty(18373, 32, 128, dtype=torch.bfloat16)
    k = torch.empty(18373, 8, 128, dtype=torch.bfloat16)
    info = _kernel.launch_info_varlen(q, k, 8, 3501, 3501, causal=True)
    assert info.kernel_name.startswith(b"mfa_fwd16pp<bf16,d128") and info.block_x == 512


def test_oversized_grids_are_rejected_not_wrapped(lib):
    # batch * heads_q = 2^32 wraps a 32-bit product to 0 (an empty grid that
    # would return OK without writing the output): both passes must reject it
    p = good_params(B=65536, L=256, H=65536, Hkv=65536)
    assert lib.mfa_fwd(ctypes.byref(p), None) == _hip.MFA_ERR_INVALID
    assert b"too large" in lib.mfa_last_error()
    info = _hip.MfaLaunchInfo()
    assert lib.mfa_fwd_launch_info(ctypes.byref(p), ctypes.byref(info)) == _hip.MFA_ERR_INVALID
    bp = _hip.MfaBwdParams()
    bp.fwd = good_params(B=65536, L=256, H=65536, Hkv=65536)
    bp.fwd.softmax_lse = 4096
    bp.fwd.lse_batch_stride, bp.fwd.lse_head_stride = 65536 * 256, 256
    for name, pre in (("dout", "do"), ("dq", "dq"), ("dk", "dk"), ("dv", "dv")):
        setattr(bp, name, 4096)
        setattr(bp, f"{pre}_batch_stride", bp.fwd.q_batch_stride)
        setattr(bp, f"{pre}_seq_stride", bp.fwd.q_seq_stride)
        setattr(bp, f"{pre}_head_stride", bp.fwd.q_head_stride)
    bp.dtype_grad = _hip.MFA_DTYPE_BF16
    assert lib.mfa_bwd_workspace_bytes(ctypes.byref(bp)) < 0
    assert b"too large" in lib.mfa_last_error()
    bp.fwd.batch, bp.fwd.heads_q, bp.fwd.heads_kv = 1, 4, 4  # the same call at a normal size plans
    assert lib.mfa_bwd_workspace_bytes(ctypes.byref(bp)) > 0


def test_backward_rejects_strides_whose_128_row_span_overflows(lib):
    # the dK/dV kernel stages 128 query rows per step above head dim 64: a
    # query row stride of 10M elements spans < 2 GiB over 64 rows but not
    # over 128, so the planner must reject it rather than wrap the offset
    def bwd(qs):
        bp = _hip.MfaBwdParams()
        bp.fwd = good_params(B=1, L=256, H=4, Hkv=4, D=128)
        bp.fwd.q_seq_stride = qs
        bp.fwd.softmax_lse = 4096
        bp.fwd.lse_batch_stride, bp.fwd.lse_head_stride = 4 * 256, 256
        for name, pre in (("dout", "do"), ("dq", "dq"), ("dk", "dk"), ("dv", "dv")):
            setattr(bp, name, 4096)
            setattr(bp, f"{pre}_batch_stride", bp.fwd.k_batch_stride)
            setattr(bp, f"{pre}_seq_stride", bp.fwd.k_seq_stride)
            setattr(bp, f"{pre}_head_stride", bp.fwd.k_head_stride)
        bp.dtype_grad = _hip.MFA_DTYPE_BF16
        return lib.mfa_bwd_workspace_bytes(ctypes.byref(bp))
    assert bwd(4 * 128) > 0
    assert bwd(10_000_000) < 0
    assert b"128 rows" in lib.mfa_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("MTLFLASHATTN_HIP_LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_hip, "_lib", None)
    with pytest.raises(_hip.HipLibraryError, match="not found"):
        _hip.load()


def test_split_kv_choice(lib):
    # decode-like: few query rows, more keys than one 2048-key chunk
    for B in (1, 8):
        p = good_params(B=B, L=4096, H=16)
        p.seqlen_q = 1
        assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 2048
        p.seqlen_q = 256
        assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 2048
        p.seqlen_q = 257
        assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 0
    p = good_params(L=2048)
    p.seqlen_q = 1
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 0
    p.seqlen_k = 2049
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 2048
    # a dense batch that fills the chip on its own keeps the single pass; a
    # varlen batch (or B=1) is chunked by its lengths alone
    p = good_params(B=64, L=4096, H=16)
    p.seqlen_q = 1
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 0
    p.cu_seqlens_q = p.cu_seqlens_k = 256
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 2048
    p = good_params(B=1, L=4096, H=1024)
    p.seqlen_q = 1
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 2048
    p = good_params(L=8192, dtype=_hip.MFA_DTYPE_F32)
    p.seqlen_q = 1
    assert lib.mfa_fwd_split_keys(ctypes.byref(p)) == 0
    assert lib.mfa_fwd_split_keys(None) == 0


def test_split_kv_workspace_size(lib):
    p = good_params(B=2, L=3000, H=8, Hkv=2, D=64)
    p.seqlen_q = 3
    # ceil(3000 / 1024) = 3 chunks x (2*8 units) x 3 rows: O rows of 64 floats + lse (256-byte aligned)
    rows = 3 * 16 * 3
    assert lib.mfa_fwd_workspace_bytes(ctypes.byref(p), 1024) == rows * 64 * 4 + -(-rows * 4 // 256) * 256
    assert lib.mfa_fwd_workspace_bytes(ctypes.byref(p), 0) == 0
    p.head_dim = 40  # padded to 64-float rows
    assert lib.mfa_fwd_workspace_bytes(ctypes.byref(p), 1024) == rows * 64 * 4 + -(-rows * 4 // 256) * 256


@pytest.mark.parametrize("chunk,mutate,code,msg", [
    (100, None, _hip.MFA_ERR_INVALID, "multiple of 64"),
    (-64, None, _hip.MFA_ERR_INVALID, "multiple of 64"),
    (1024, lambda p: setattr(p, "dtype_in", _hip.MFA_DTYPE_F32) or setattr(p, "dtype_out", _hip.MFA_DTYPE_F32),
     _hip.MFA_ERR_UNSUPPORTED, "fp32"),
    (1024, lambda p: setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG), _hip.MFA_ERR_UNSUPPORTED, "256-row"),
    (1024, lambda p: setattr(p, "tile_hint", _hip.MFA_TILE_PINGPONG256), _hip.MFA_ERR_UNSUPPORTED, "256-row"),
    (64, lambda p: setattr(p, "seqlen_k", 64 * 1025), _hip.MFA_ERR_INVALID, "exceed"),
    (192, lambda p: (setattr(p, "block_table", 256), setattr(p, "page_block_size", 256), setattr(p, "num_pages", 16)),
     _hip.MFA_ERR_INVALID, "multiple of 256 with a block_table"),
])
def test_split_kv_invalid_requests(lib, chunk, mutate, code, msg):
    p = good_params(L=4096)
    p.seqlen_q = 1
    if mutate:
        mutate(p)
    assert lib.mfa_fwd_workspace_bytes(ctypes.byref(p), chunk) == code
    assert lib.mfa_fwd_splitkv(ctypes.byref(p), chunk, ctypes.c_void_p(1 << 20), 1 << 30, None) == code
    assert msg in lib.mfa_last_error().decode()


def test_split_kv_rejects_a_small_or_misaligned_workspace(lib):
    p = good_params(L=4096)
    p.seqlen_q = 1
    need = lib.mfa_fwd_workspace_bytes(ctypes.byref(p), 1024)
    assert need > 0
    assert lib.mfa_fwd_splitkv(ctypes.byref(p), 1024, ctypes.c_void_p(1 << 20), need - 1, None) == _hip.MFA_ERR_INVALID
    assert b"needed" in lib.mfa_last_error()
    assert lib.mfa_fwd_splitkv(ctypes.byref(p), 1024, ctypes.c_void_p((1 << 20) + 16), need, None) == \
        _hip.MFA_ERR_INVALID
    assert b"aligned" in lib.mfa_last_error()
    assert lib.mfa_fwd_splitkv(ctypes.byref(p), 1024, None, need, None) == _hip.MFA_ERR_INVALID


def test_plan_uses_the_device_geometry():
    """Tile and split-KV choices compare grids against the device's CU count
    (queried per device; MI355X 256 CUs / 8 XCDs by default, the env override
    stands in for a partitioned device here).  On a 32-CU, 1-XCD part a
    B=1 L=2048 H=16 D=64 call fills the chip with 512-row ping-pong tiles,
    which on 256 CUs would leave CUs idle (4-wavefront kernel there), and a
    B=4 Hq=32 decode already fills it without split-KV."""
    import subprocess
    import sys
    import textwrap

    code = textwrap.dedent("""
        import torch
        from mtlflashattn_amd import _hip, _kernel
        q = torch.empty(1, 2048, 16, 64, dtype=torch.bfloat16)
        print(_kernel.launch_info(q, q, q).kernel_name.decode())
        p = _hip.MfaFwdParams()
        p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k = 4, 32, 32, 1, 8192
        p.dtype_in = p.dtype_out = _hip.DTYPE_CODES[torch.bfloat16]
        print(_hip.split_keys(p))
    """)
    out = {}
    for cus, xcds in ((None, None), (32, 1)):
        env = dict(os.environ)
        env.pop("MTLFLASHATTN_CHIP_CUS", None)
        env.pop("MTLFLASHATTN_CHIP_XCDS", None)
        if cus:
            env["MTLFLASHATTN_CHIP_CUS"], env["MTLFLASHATTN_CHIP_XCDS"] = str(cus), str(xcds)
        env["PYTHONPATH"] = REPO
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        out[cus] = r.stdout.strip().splitlines()
    if torch.cuda.is_available():
        pytest.skip("the default leg assumes 256 CUs; a visible device reports its own")
    assert out[None][0].startswith("mfa_fwd16<bf16,d64") and out[None][1] == "2048"
    assert out[32][0].startswith("mfa_fwd16pp<bf16,d64,2,2>") and out[32][1] == "0"


def test_exact_row_kernel_choice(lib):
    # single-row 16-bit calls (one row per head, or packed grouped-query
    # decode rows) run the exact-row kernel whatever the tile hint; fp32 keeps
    # its own kernel; longer rows never take it as their main kernel
    def name(**kw):
        p = good_params(B=kw.pop("B", 4), L=4096, H=kw.pop("H", 16), Hkv=kw.pop("Hkv", 16), D=kw.pop("D", 128),
                        dtype=kw.pop("dtype", _hip.MFA_DTYPE_BF16))
        p.seqlen_q = kw.pop("Lq", 1)
        for f, val in kw.items():
            setattr(p, f, val)
        return _hip.launch_info(p).kernel_name
    assert name().startswith(b"mfa_fwd16x<bf16,d128>")
    assert name(Hkv=2).startswith(b"mfa_fwd16x<bf16,d128>")  # packed: 8 rows per K/V head
    assert name(D=64, dtype=_hip.MFA_DTYPE_F16).startswith(b"mfa_fwd16x<f16,d64>")
    assert name(D=64, tile_hint=_hip.MFA_TILE_PINGPONG).startswith(b"mfa_fwd16x<bf16,d64>")
    assert name(softcap=5.0).startswith(b"mfa_fwd16x<bf16,d128>")
    assert name(dtype=_hip.MFA_DTYPE_F32).startswith(b"mfa_fwd32")
    assert not name(Lq=2).startswith(b"mfa_fwd16x")
    assert not name(Lq=4096).startswith(b"mfa_fwd16x")
    # varlen: one query row per sequence at most -> exact kernel; longer
    # sequences -> their kernel (the single-row ones get the exact kernel's
    # second launch)
    assert name(Lq=1, cu_seqlens_q=256, cu_seqlens_k=256).startswith(b"mfa_fwd16x")
    assert not name(Lq=64, cu_seqlens_q=256, cu_seqlens_k=256).startswith(b"mfa_fwd16x")
