"""Error contract and argument plumbing of the public API, on CPU.

Mirrors the reference's argument checks (metal_flash_attn/__init__.py:28-59,
:84-90, :130-164, :186-229; metal_flash_attn/_kernel.py:1070-1075,
:1275-1285) and its unsupported-kwarg tests (tests/test_flash_attn_func.py:
126-147, :247-252, :337-358; tests/test_flash_attn_varlen_func.py:111-131;
tests/test_packed_funcs.py:43-54, :80-86).  Checks that come after the device
check run with the device predicate patched to accept CPU tensors and the
launcher replaced by a recording fake, so nothing reaches the GPU.
"""
from __future__ import annotations

import math

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _kernel


def t(*shape, dtype=torch.float16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.fixture
def fake_device(monkeypatch):
    """Treat CPU tensors as ROCm tensors and record launches instead of running them."""
    calls = []

    def fake_run(q, k, v, out, **kw):
        calls.append(dict(q=q, k=k, v=v, out=out, **kw))
        return out

    monkeypatch.setattr(_kernel, "_is_rocm_tensor", lambda x: True)
    monkeypatch.setattr(_kernel, "_run", fake_run)
    return calls


QKV = (t(1, 32, 4, 64), t(1, 32, 4, 64), t(1, 32, 4, 64))


class TestCheckSupportedOrder:
    @pytest.mark.parametrize("kwargs,exc", [
        (dict(dropout_p=0.1), NotImplementedError),
        (dict(window_size=(-2, 0)), ValueError),
        (dict(window_size=(1,)), ValueError),
        (dict(window_size=(True, 0)), ValueError),
        (dict(window_size=(1.5, 0)), ValueError),
        (dict(window_size="ab"), ValueError),
        (dict(softcap=-1.0), ValueError),
        (dict(alibi_slopes=[0.5, 0.25, 0.125, 0.0625]), TypeError),
        (dict(deterministic=True), NotImplementedError),
        (dict(return_attn_probs=True), NotImplementedError),
    ])
    def test_argument_errors(self, kwargs, exc):
        with pytest.raises(exc):
            mfa.flash_attn_func(*QKV, **kwargs)

    def test_dropout_checked_before_window(self):
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_func(*QKV, dropout_p=0.5, window_size=(-5, 0))

    def test_cpu_tensors_raise_not_implemented(self):
        with pytest.raises(NotImplementedError, match="ROCm GPU only"):
            mfa.flash_attn_func(*QKV)
        with pytest.raises(NotImplementedError):
            _kernel.flash_attn_forward(t(1, 2, 8, 16), t(1, 2, 8, 16), t(1, 2, 8, 16), 0.25, False)

    def test_window_lists_accepted(self, fake_device):
        mfa.flash_attn_func(*QKV, window_size=[3, -1])
        assert fake_device[-1]["window_left"] == 3 and fake_device[-1]["window_right"] == -1


class TestAfterDeviceCheck:
    def test_dtype_mismatch_and_unsupported(self, fake_device):
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_func(t(1, 8, 2, 64), t(1, 8, 2, 64, dtype=torch.float32), t(1, 8, 2, 64))
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_func(*(t(1, 8, 2, 64, dtype=torch.float64) for _ in range(3)))

    def test_head_dim_gt_128(self, fake_device):
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_func(*(t(1, 16, 1, 160) for _ in range(3)))

    def test_head_dim_mismatch(self, fake_device):
        with pytest.raises(ValueError):
            mfa.flash_attn_func(t(1, 8, 2, 64), t(1, 8, 2, 32), t(1, 8, 2, 32))

    def test_rank_heads_and_lengths(self, fake_device):
        with pytest.raises(ValueError):
            mfa.flash_attn_func(t(8, 2, 64), t(8, 2, 64), t(8, 2, 64))
        with pytest.raises(ValueError):
            mfa.flash_attn_func(t(1, 8, 6, 64), t(1, 8, 4, 64), t(1, 8, 4, 64))
        with pytest.raises(ValueError):
            mfa.flash_attn_func(t(1, 8, 4, 64), t(1, 9, 4, 64), t(1, 8, 4, 64))
        assert not fake_device

    def test_batch_and_value_head_mismatch(self, fake_device):
        # the kernel takes the batch from q and the K/V head count from k: a
        # k/v batch or a v head count that differs must raise, never launch
        with pytest.raises(ValueError, match="batch"):
            mfa.flash_attn_func(t(4, 8, 4, 64), t(2, 8, 4, 64), t(2, 8, 4, 64))
        with pytest.raises(ValueError, match="batch"):
            mfa.flash_attn_func(t(2, 8, 4, 64), t(2, 8, 4, 64), t(1, 8, 4, 64))
        with pytest.raises(ValueError, match="heads"):
            mfa.flash_attn_func(t(1, 8, 4, 64), t(1, 8, 2, 64), t(1, 8, 1, 64))
        # heads-second boundary and the heads-third launcher check the same
        with pytest.raises(ValueError, match="batch"):
            _kernel.flash_attn_forward(t(4, 4, 8, 32), t(2, 4, 8, 32), t(2, 4, 8, 32), 0.25, False)
        with pytest.raises(ValueError, match="heads"):
            _kernel.flash_attn_forward(t(1, 4, 8, 32), t(1, 2, 8, 32), t(1, 1, 8, 32), 0.25, False)
        with pytest.raises(ValueError, match="seqlen"):
            _kernel.flash_attn_forward(t(1, 4, 8, 32), t(1, 4, 8, 32), t(1, 4, 9, 32), 0.25, False)
        with pytest.raises(ValueError, match="batch"):
            _kernel.forward_bshd(t(3, 8, 4, 32), t(1, 8, 4, 32), t(1, 8, 4, 32), 0.25, False)
        assert not fake_device

    def test_default_scale_and_forwarded_arguments(self, fake_device):
        q, k, v = t(2, 10, 8, 48), t(2, 12, 2, 48), t(2, 12, 2, 48)
        slopes = torch.rand(8)
        out = mfa.flash_attn_func(q, k, v, causal=True, window_size=(5, 0), softcap=7.0, alibi_slopes=slopes)
        c = fake_device[-1]
        assert c["scale"] == pytest.approx(1 / math.sqrt(48))
        assert c["causal"] is True and c["softcap"] == 7.0
        assert (c["window_left"], c["window_right"]) == (5, 0)
        assert c["alibi_bstride"] == 0 and torch.equal(c["alibi"], slopes)
        assert out.shape == q.shape and out.dtype == q.dtype
        # heads-third inputs are passed as views: no layout copy on the way in
        assert c["q"].data_ptr() == q.data_ptr() and c["k"].data_ptr() == k.data_ptr()
        mfa.flash_attn_func(q, k, v, softmax_scale=0.3)
        assert fake_device[-1]["scale"] == 0.3

    def test_alibi_shapes(self, fake_device):
        q = t(2, 8, 4, 32)
        mfa.flash_attn_func(q, q, q, alibi_slopes=torch.rand(2, 4))
        assert fake_device[-1]["alibi_bstride"] == 4
        assert fake_device[-1]["alibi"].dtype == torch.float32
        with pytest.raises(ValueError):
            mfa.flash_attn_func(q, q, q, alibi_slopes=torch.ones(3))
        with pytest.raises(ValueError):
            mfa.flash_attn_func(q, q, q, alibi_slopes=torch.ones(3, 4))

    def test_flash_attn_forward_boundary(self, fake_device):
        q = t(2, 4, 8, 32)  # heads-second
        out = _kernel.flash_attn_forward(q, q[:, :2], q[:, :2], 0.25, True)
        assert out.shape == (2, 4, 8, 32) and out.is_contiguous()
        with pytest.raises(ValueError):
            _kernel.flash_attn_forward(q, q, q, 0.25, False, softcap=-1.0)
        with pytest.raises(ValueError):
            _kernel.flash_attn_forward(q, q[:, :3], q[:, :3], 0.25, False)
        with pytest.raises(ValueError):
            _kernel.flash_attn_forward(q, q, q, 0.25, False, alibi_slopes=torch.ones(5))
        out32 = _kernel.flash_attn_forward(q, q, q, 0.25, False, out_dtype=torch.float32)
        assert out32.dtype == torch.float32
        with pytest.raises(ValueError):
            _kernel.flash_attn_forward(q, q, q, 0.25, False, out_dtype=torch.float64)


class TestVarlenContract:
    def make(self, lens_q=(5, 7), lens_k=(6, 3), Hq=4, Hkv=2, D=32):
        q, k, v = t(sum(lens_q), Hq, D), t(sum(lens_k), Hkv, D), t(sum(lens_k), Hkv, D)
        cu_q = torch.tensor([0, *torch.tensor(lens_q).cumsum(0).tolist()], dtype=torch.int32)
        cu_k = torch.tensor([0, *torch.tensor(lens_k).cumsum(0).tolist()], dtype=torch.int32)
        return q, k, v, cu_q, cu_k

    def test_unsupported_kwargs(self):
        q, k, v, cu_q, cu_k = self.make()
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6, dropout_p=0.5)

    def test_block_table_contract(self, fake_device, monkeypatch):
        # the reference raises NotImplementedError for block_table
        # (metal_flash_attn/__init__.py:130-131); this build implements the paged
        # layout of CUDA flash-attn and validates it before any launch
        q, k, v, cu_q, cu_k = self.make()
        pool = t(3, 256, 2, 32)
        bt = torch.tensor([[0], [2]], dtype=torch.int32)
        with pytest.raises(ValueError):  # k/v not page pools
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6, block_table=bt)
        with pytest.raises(ValueError):  # page size not a multiple of 256
            mfa.flash_attn_varlen_func(q, t(3, 100, 2, 32), t(3, 100, 2, 32), cu_q, cu_k, 7, 6, block_table=bt)
        with pytest.raises(ValueError):  # int64 table
            mfa.flash_attn_varlen_func(q, pool, pool, cu_q, cu_k, 7, 6, block_table=bt.long())
        with pytest.raises(ValueError):  # one row per sequence
            mfa.flash_attn_varlen_func(q, pool, pool, cu_q, cu_k, 7, 6, block_table=bt[:1])
        bad_ids = torch.tensor([[0], [3]], dtype=torch.int32)
        monkeypatch.setenv("MTLFLASHATTN_CHECK_PAGES", "1")
        with pytest.raises(ValueError):  # page id outside the pool (host check on request)
            mfa.flash_attn_varlen_func(q, pool, pool, cu_q, cu_k, 7, 6, block_table=bad_ids)
        with pytest.raises(ValueError):  # too few pages for 300 keys
            mfa.flash_attn_varlen_func(q, pool, pool, cu_q, torch.tensor([0, 300, 303], dtype=torch.int32),
                                       7, 300, block_table=bt)
        assert not fake_device
        # unused entries (past a sequence's last page) are never checked or read
        out = mfa.flash_attn_varlen_func(q, pool, pool, cu_q, cu_k, 7, 6,
                                         block_table=torch.tensor([[1, -5], [2, 99]], dtype=torch.int32))
        call = fake_device[-1]
        assert out.shape == q.shape and call["k"].shape == pool.shape and call["block_table"] is not None
        assert call["seqlen_k"] == 6 and call["lse"] is None
        # by default the page ids are not read on the host (no per-call device
        # sync): an id outside the pool reaches the kernel, whose guard reads
        # zeros for it
        monkeypatch.delenv("MTLFLASHATTN_CHECK_PAGES")
        n = len(fake_device)
        mfa.flash_attn_varlen_func(q, pool, pool, cu_q, cu_k, 7, 6, block_table=bad_ids)
        assert len(fake_device) == n + 1

    def test_with_lse_layouts(self, fake_device):
        q, k, v, cu_q, cu_k = self.make()
        out, lse = mfa.flash_attn_varlen_func_with_lse(q, k, v, cu_q, cu_k, 7, 6, causal=True)
        assert out.shape == q.shape and lse.shape == (4, 12) and lse.dtype == torch.float32
        assert fake_device[-1]["lse"] is lse
        qd, kd, vd = t(2, 9, 4, 32), t(2, 5, 2, 32), t(2, 5, 2, 32)
        out, lse = mfa.flash_attn_func_with_lse(qd, kd, vd)
        assert out.shape == qd.shape and lse.shape == (2, 4, 9) and lse.dtype == torch.float32
        with pytest.raises(ValueError):
            mfa.flash_attn_func_with_lse(qd, kd, vd, softcap=-1.0)

    def test_shape_errors(self, fake_device):
        q, k, v, cu_q, cu_k = self.make()
        with pytest.raises(ValueError):
            mfa.flash_attn_varlen_func(q[None], k[None], v[None], cu_q, cu_k, 7, 6)
        with pytest.raises(ValueError):  # different batch sizes
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k[:2], 7, 6)
        with pytest.raises(ValueError):  # heads
            mfa.flash_attn_varlen_func(t(12, 3, 32), k, v, cu_q, cu_k, 7, 6)
        with pytest.raises(ValueError):  # k/v totals
            mfa.flash_attn_varlen_func(q, k, v[:-1], cu_q, cu_k, 7, 6)
        with pytest.raises(ValueError):  # cu_seqlens_q[-1] != total_q
            mfa.flash_attn_varlen_func(q[:-1], k, v, cu_q, cu_k, 7, 6)
        with pytest.raises(ValueError):  # cu_seqlens_k[-1] != total_k
            mfa.flash_attn_varlen_func(q, k[:-1], v[:-1], cu_q, cu_k, 7, 6)
        with pytest.raises(ValueError):  # non-monotonic
            mfa.flash_attn_varlen_func(q, k, v, torch.tensor([0, 9, 12], dtype=torch.int32),
                                       torch.tensor([0, 10, 9], dtype=torch.int32), 9, 10)
        with pytest.raises(ValueError):  # 2-D ALiBi must be [batch, Hq]
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6, alibi_slopes=torch.ones(3, 4))
        assert not fake_device

    def test_prefix_sums_read_once_per_tensor_version(self, fake_device, monkeypatch):
        # repeated calls on the same cu_seqlens read them on the host once; an
        # in-place write (a new version) or other tensors are read again
        q, k, v, cu_q, cu_k = self.make()
        reads = []
        real_cat = torch.cat
        monkeypatch.setattr(torch, "cat", lambda ts, *a, **kw: (reads.append(1), real_cat(ts, *a, **kw))[1])
        mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6)
        mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6, causal=True)
        assert len(reads) == 1 and len(fake_device) == 2
        with pytest.raises(ValueError):  # the cached sums are checked against each call's totals
            mfa.flash_attn_varlen_func(q[:-1], k, v, cu_q, cu_k, 7, 6)
        assert len(reads) == 1
        cu_q[1] = 13  # non-monotonic now: the new version is read and rejected
        with pytest.raises(ValueError):
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6)
        assert len(reads) == 2
        cu_q[1] = 4  # lengths (4, 8): the true longest query length follows the write
        mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 7, 6)
        assert len(reads) == 3 and fake_device[-1]["seqlen_q"] == 8
        mfa.flash_attn_varlen_func(q, k, v, cu_q.clone(), cu_k, 7, 6)  # another tensor
        assert len(reads) == 4

    def test_one_launch_with_true_max_lengths(self, fake_device):
        q, k, v, cu_q, cu_k = self.make(lens_q=(5, 0, 7), lens_k=(6, 4, 3))
        slopes = torch.rand(3, 4)
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 1, 1, alibi_slopes=slopes, causal=True)
        assert len(fake_device) == 1
        c = fake_device[0]
        # understated max_seqlen_* is replaced by the true longest lengths
        assert (c["seqlen_q"], c["seqlen_k"]) == (7, 6)
        assert c["alibi_bstride"] == 4
        assert torch.equal(c["cu_q"], cu_q) and c["cu_q"].dtype == torch.int32
        assert out.shape == q.shape


class TestPackedContract:
    def test_shape_validation(self):
        with pytest.raises(ValueError):
            mfa.flash_attn_qkvpacked_func(t(1, 32, 2, 4, 64))
        with pytest.raises(ValueError):
            mfa.flash_attn_kvpacked_func(t(1, 32, 4, 64), t(1, 32, 3, 4, 64))
        with pytest.raises(ValueError):
            mfa.flash_attn_varlen_qkvpacked_func(t(32, 2, 4, 64), torch.tensor([0, 32], dtype=torch.int32), 32)
        with pytest.raises(ValueError):
            mfa.flash_attn_varlen_kvpacked_func(t(32, 4, 64), t(32, 3, 4, 64), torch.tensor([0, 32]),
                                                torch.tensor([0, 32]), 32, 32)

    def test_unsupported_kwargs_propagate(self):
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_qkvpacked_func(t(1, 32, 3, 4, 64), dropout_p=0.5)

    def test_packed_views_reach_the_launcher_uncopied(self, fake_device):
        qkv = t(2, 16, 3, 4, 64)
        mfa.flash_attn_qkvpacked_func(qkv, causal=True)
        c = fake_device[-1]
        q, k, v = qkv.unbind(dim=2)
        assert c["q"].data_ptr() == q.data_ptr() and c["v"].data_ptr() == v.data_ptr()
        assert c["causal"] is True


def test_public_surface():
    for name in ("flash_attn_func", "flash_attn_varlen_func", "flash_attn_qkvpacked_func",
                 "flash_attn_kvpacked_func", "flash_attn_varlen_qkvpacked_func", "flash_attn_varlen_kvpacked_func"):
        assert callable(getattr(mfa, name))
    from mtlflashattn_amd._version import FLASH_ATTN_SHIM_VERSION

    assert FLASH_ATTN_SHIM_VERSION == "2.7.4"
    assert _kernel.MAX_HEAD_DIM == 128


def test_trace_records_calls(monkeypatch, fake_device):
    monkeypatch.setenv("MTLFLASHATTN_TRACE", "1")
    _kernel._trace.clear()
    q = t(1, 128, 4, 64)
    mfa.flash_attn_func(q, q, q)
    mfa.flash_attn_func(q, q, q)
    assert list(_kernel._trace.values()) == [2]
    (dt, D, Lq, Lk, causal, label), = _kernel._trace
    assert (dt, D, Lq, Lk, causal, label) == ("float16", 64, 128, 128, False, "hip")
    assert any("float16" in line for line in _kernel._trace_summary_lines())
    monkeypatch.delenv("MTLFLASHATTN_TRACE")
    _kernel._trace.clear()
    mfa.flash_attn_func(q, q, q)
    assert _kernel._trace == {}


def test_kernel_mode_env_selects_the_single_path(monkeypatch, fake_device):
    monkeypatch.setenv("MTLFLASHATTN_KERNEL", "v2_bf16")
    _kernel._warned_modes.clear()
    with pytest.warns(UserWarning, match="single HIP"):
        assert _kernel._kernel_mode() == "hip"


class TestLauncherAlignment:
    """The C ABI takes 16-byte aligned bases and strides (include/mfa.h).  The
    reference has no alignment rule (metal_flash_attn/_kernel.py:1296-1298),
    so the launcher must copy a legal tensor that breaks it, including a
    contiguous one at a misaligned storage offset, where .contiguous() is a
    no-op."""

    @staticmethod
    def recorded_launch(monkeypatch):
        launches = []

        def fake_launch(p, chunk, device):
            launches.append(p)

        monkeypatch.setattr(_kernel, "_launch", fake_launch)
        monkeypatch.setattr(_kernel, "_split_choice", lambda p, dtype, hint: 0)
        _kernel._plans.clear()
        return launches

    def test_misaligned_contiguous_inputs_are_copied(self, monkeypatch):
        B, L, H, D = 2, 16, 4, 64
        base = torch.randn(1 + B * L * H * D, dtype=torch.float32).to(torch.bfloat16)
        q = base[1:].view(B, L, H, D)
        assert q.is_contiguous() and q.data_ptr() % 16 == 2 and q.contiguous() is q
        fixed = _kernel._abi_operand(q)
        assert fixed.data_ptr() % 16 == 0 and torch.equal(fixed, q)
        assert _kernel._abi_operand(fixed) is fixed  # aligned tensors pass through uncopied

        launches = self.recorded_launch(monkeypatch)
        out = torch.empty(B, L, H, D, dtype=torch.bfloat16)
        _kernel._run(q, q, q, out, scale=0.125, causal=False, softcap=0.0, window_left=-1, window_right=-1,
                     alibi=None, alibi_bstride=0)
        p = launches[-1]
        assert p.q % 16 == 0 and p.k % 16 == 0 and p.v % 16 == 0 and p.o % 16 == 0
        assert (p.q_seq_stride, p.q_head_stride) == (H * D, D)

    def test_misaligned_output_goes_through_a_staging_buffer(self, monkeypatch):
        B, L, H, D = 1, 8, 2, 32
        q = torch.zeros(B, L, H, D, dtype=torch.float16)
        obase = torch.zeros(1 + B * L * H * D, dtype=torch.float16)
        out = obase[1:].view(B, L, H, D)
        launches = self.recorded_launch(monkeypatch)
        _kernel._run(q, q, q, out, scale=0.125, causal=False, softcap=0.0, window_left=-1, window_right=-1,
                     alibi=None, alibi_bstride=0)
        assert launches[-1].o % 16 == 0 and launches[-1].o != out.data_ptr()
