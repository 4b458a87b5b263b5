"""GPU parity of the HIP forward against the oracle (the reference's chunked-fp32
torch path restated in oracle/chunked.py), on the reference test suite's cases
(tests/test_flash_attn_func.py, tests/test_flash_attn_varlen_func.py,
tests/test_packed_funcs.py of the reference) and on BASELINE configs 1-4 at full
size.  Every call goes through the C ABI of libmtlfa_hip.so."""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _hip, _kernel
from oracle import chunked
from gpu_util import (
    DEV, assert_output, assert_parity, default_scale, make_qkv, make_varlen, max_err, native_library_mapped,
)

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(params=[_hip.MFA_TILE_256, _hip.MFA_TILE_PINGPONG, _hip.MFA_TILE_PINGPONG256],
                ids=["tile256", "pingpong", "pingpong256"])
def tile(request, monkeypatch):
    """Run a test through each bf16/fp16 kernel: 256-row tiles and the 512- and
    256-row ping-pong tiles (head dims <= 64; other cases keep the library's
    choice)."""
    monkeypatch.setattr(_kernel, "_TILE_HINT", request.param)
    return request.param


def run_both(q, k, v, **kw):
    """(public API output in q.dtype, fp32-output parity mode)."""
    out = mfa.flash_attn_func(q, k, v, **kw)
    scale = kw.get("softmax_scale")
    scale = scale if scale is not None else default_scale(q.shape[-1])
    ws = kw.get("window_size", (-1, -1))
    out32 = _kernel.forward_bshd(q, k, v, scale, kw.get("causal", False), kw.get("softcap", 0.0), ws[0], ws[1],
                                 kw.get("alibi_slopes"), out_dtype=torch.float32)
    return out, out32


def check(q, k, v, what="", **kw):
    out, out32 = run_both(q, k, v, **kw)
    assert out.shape == q.shape and out.dtype == q.dtype
    ref = chunked.flash_attn_func(q.cpu(), k.cpu(), v.cpu(), softmax_scale=kw.get("softmax_scale"),
                                  causal=kw.get("causal", False), window_size=kw.get("window_size", (-1, -1)),
                                  softcap=kw.get("softcap", 0.0), alibi_slopes=kw.get("alibi_slopes"))
    e32 = assert_parity(out32, ref, q.dtype, what)
    eout = assert_output(out, ref, q.dtype, what)
    return e32, eout


def test_native_library_is_the_path():
    q, k, v = make_qkv(1, 64, 64, 2, 2, 64, torch.bfloat16)
    mfa.flash_attn_func(q, k, v)
    torch.cuda.synchronize()
    assert native_library_mapped(), "libmtlfa_hip.so is not mapped: the HIP path did not run"


@pytest.mark.parametrize("dtype", DTYPES)
def test_launch_parameter_reuse(dtype):
    # V with strides unlike K's (prepared parameters are per signature) and a
    # second call of the same signature on new data
    q, k, v = make_qkv(2, 64, 80, 4, 4, 64, dtype, seed=1)
    v2 = v.transpose(1, 2).contiguous().transpose(1, 2)
    assert v2.stride() != v.stride()
    assert torch.equal(mfa.flash_attn_func(q, k, v2), mfa.flash_attn_func(q, k, v))
    q, k, v = make_qkv(2, 64, 80, 4, 4, 64, dtype, seed=2)
    check(q, k, v, "second call of one signature")
    check(q, k, v.transpose(1, 2).contiguous().transpose(1, 2), "second call, strided V")


def test_config1_fp32_exact_inputs():
    # B=1, L=512, H=2, D=64, fp32, non-causal, scale 1/8, seed 0
    q, k, v = make_qkv(1, 512, 512, 2, 2, 64, torch.float32, seed=0)
    e32, _ = check(q, k, v, "config1", softmax_scale=0.125)
    print(f"config1 fp32 max abs err {e32:.3e}")


@pytest.mark.usefixtures("tile")
class TestFlashAttnFunc:
    @pytest.mark.parametrize("dtype", DTYPES)
    def test_mha_self_attn(self, dtype):
        q, k, v = make_qkv(2, 128, 128, 4, 4, 64, dtype)
        check(q, k, v)

    @pytest.mark.parametrize("dtype", DTYPES)
    @pytest.mark.parametrize("causal", [False, True])
    def test_cross_attn_lq_ne_lk(self, dtype, causal):
        q, k, v = make_qkv(1, 64, 192, 4, 4, 64, dtype)
        check(q, k, v, causal=causal)
        q, k, v = make_qkv(1, 200, 77, 4, 4, 64, dtype, seed=5)
        check(q, k, v, causal=causal)

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_causal_lq_gt_lk(self, dtype):
        q, k, v = make_qkv(1, 96, 48, 2, 2, 32, dtype)
        out = mfa.flash_attn_func(q, k, v, causal=True)
        # rows i < Lq - Lk see no key: exactly zero (metal_flash_attn/_kernel.py:85-86)
        assert torch.count_nonzero(out[:, :48]) == 0
        check(q, k, v, causal=True)

    @pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 1)])
    @pytest.mark.parametrize("dtype", DTYPES)
    def test_gqa_mqa(self, hq, hkv, dtype):
        q, k, v = make_qkv(2, 64, 64, hq, hkv, 64, dtype)
        check(q, k, v, causal=True)

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_gqa_bit_exact_vs_repeated_kv(self, dtype):
        q, k, v = make_qkv(2, 300, 300, 8, 2, 64, dtype, seed=3)
        a = mfa.flash_attn_func(q, k, v, causal=True)
        kr = k.repeat_interleave(4, dim=2)
        vr = v.repeat_interleave(4, dim=2)
        b = mfa.flash_attn_func(q, kr, vr, causal=True)
        assert torch.equal(a, b)

    @pytest.mark.parametrize("d", [8, 16, 32, 40, 64, 80, 96, 128, 33, 100])
    @pytest.mark.parametrize("dtype", DTYPES)
    def test_head_dims(self, d, dtype):
        q, k, v = make_qkv(1, 70, 90, 2, 2, d, dtype)
        check(q, k, v, f"D={d}")
        check(q, k, v, f"D={d} causal", causal=True)

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_single_key_block(self, dtype):
        # every tile walks one 64-key block, so its first MFMA phase is also
        # its last (head dim 128 ping-pong tiles: a QK-only phase, then a
        # PV-only one)
        for lq, lk, causal in ((300, 40, False), (64, 64, True), (200, 64, True), (1000, 17, False)):
            q, k, v = make_qkv(1, lq, lk, 2, 2, 128, dtype, seed=lq)
            check(q, k, v, f"Lq={lq} Lk={lk} causal={causal}", causal=causal)

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_custom_softmax_scale(self, dtype):
        q, k, v = make_qkv(1, 64, 64, 2, 2, 64, dtype)
        check(q, k, v, softmax_scale=0.25)
        check(q, k, v, "negative scale", softmax_scale=-0.2)

    def test_head_dim_gt_128_raises(self):
        q, k, v = make_qkv(1, 16, 16, 1, 1, 160, torch.float32)
        with pytest.raises(NotImplementedError):
            mfa.flash_attn_func(q, k, v)

    def test_non_contiguous_views(self):
        g = torch.Generator().manual_seed(9)
        base = torch.randn(2, 4, 96, 64, generator=g).to("cuda", torch.bfloat16)  # [B,H,L,D]
        q = base.transpose(1, 2)  # heads-third view with heads-second strides
        check(q, q, q, "transposed view")

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_misaligned_contiguous_inputs(self, dtype):
        # contiguous tensors at storage offsets that are not 16-byte aligned
        # (.contiguous() returns them unchanged): the launcher copies them
        # (the reference has no alignment rule, metal_flash_attn/_kernel.py:1296-1298)
        B, L, H, D = 2, 96, 4, 64
        g = torch.Generator().manual_seed(21)
        n = B * L * H * D
        base = torch.randn(3 * n + 3, generator=g).to("cuda", dtype)
        q = base[1:1 + n].view(B, L, H, D)
        k = base[2 + n:2 + 2 * n].view(B, L, H, D)
        v = base[3 + 2 * n:3 + 3 * n].view(B, L, H, D)
        assert q.is_contiguous() and q.data_ptr() % 16 != 0
        check(q, k, v, "misaligned", causal=True)
        assert torch.equal(mfa.flash_attn_func(q, k, v, causal=True),
                           mfa.flash_attn_func(q.clone(), k.clone(), v.clone(), causal=True))


@pytest.mark.usefixtures("tile")
class TestFeatures:
    @pytest.mark.parametrize("dtype", DTYPES)
    def test_softcap(self, dtype):
        q, k, v = make_qkv(2, 128, 128, 4, 4, 64, dtype)
        check(q, k, v, softcap=30.0)
        check(q, k, v, softcap=5.0, causal=True)

    @pytest.mark.parametrize("dtype", DTYPES)
    @pytest.mark.parametrize("win", [(48, 0), (16, 16), (32, -1), (-1, 0), (0, 0), (1000, 1000), (64, 16)])
    def test_window(self, dtype, win):
        q, k, v = make_qkv(1, 256, 256, 2, 2, 64, dtype)
        check(q, k, v, str(win), window_size=win)

    def test_causal_plus_window_cross_length(self):
        q, k, v = make_qkv(1, 200, 333, 2, 2, 64, torch.float32)
        check(q, k, v, causal=True, window_size=(32, -1))
        q, k, v = make_qkv(1, 64, 192, 2, 2, 64, torch.float32)
        check(q, k, v, window_size=(40, 8))

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_alibi(self, dtype):
        q, k, v = make_qkv(2, 128, 128, 4, 4, 64, dtype)
        slopes = torch.tensor([0.5, 0.25, 0.125, 0.0625], device="cuda")
        check(q, k, v, alibi_slopes=slopes)
        check(q, k, v, alibi_slopes=slopes, causal=True)
        batched = torch.tensor([[0.5, 0.25, 0.125, 0.0625], [0.1, 0.05, 0.3, 0.2]], device="cuda")
        check(q, k, v, alibi_slopes=batched)

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_feature_mix(self, dtype):
        q, k, v = make_qkv(1, 300, 300, 4, 2, 128, dtype, seed=7, scale_inputs=0.5)
        slopes = torch.tensor([2 ** (-8 * (i + 1) / 4) for i in range(4)], device="cuda")
        check(q, k, v, causal=True, window_size=(70, 0), softcap=30.0, alibi_slopes=slopes)

    def test_bad_alibi_shape_raises(self):
        q, k, v = make_qkv(1, 32, 32, 4, 4, 64, torch.float16)
        with pytest.raises(ValueError):
            mfa.flash_attn_func(q, k, v, alibi_slopes=torch.ones(3, device="cuda"))


@pytest.mark.usefixtures("tile")
class TestVarlen:
    def check_varlen(self, seqlens_q, seqlens_k, Hq=4, Hkv=4, D=64, dtype=torch.float32, causal=False,
                     alibi=None, **kw):
        q, k, v, cu_q, cu_k = make_varlen(seqlens_q, seqlens_k, Hq, Hkv, D, dtype)
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(seqlens_q), max(seqlens_k), causal=causal,
                                         alibi_slopes=alibi, **kw)
        assert out.shape == q.shape and out.dtype == q.dtype
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal,
                                             alibi_slopes=alibi.cpu() if alibi is not None else None, **kw)
        out32 = _kernel.forward_varlen(q, k, v, cu_q, cu_k, max(seqlens_q), max(seqlens_k),
                                       kw.get("softmax_scale") or default_scale(D), causal,
                                       alibi_slopes=alibi, out_dtype=torch.float32)
        assert_parity(out32, ref, dtype, "varlen")
        assert_output(out, ref, dtype, "varlen")
        return q, k, v, cu_q, cu_k, out

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_ragged_batch(self, dtype):
        self.check_varlen([37, 128, 5], [37, 128, 5], dtype=dtype)
        self.check_varlen([64, 17], [64, 17], dtype=dtype, causal=True)

    def test_prefix_sums_rewritten_in_place(self):
        # the host copy of cu_seqlens is reused only while the tensors keep
        # their version: rewriting them in place on the device (same totals,
        # other lengths) must give the call on fresh tensors, bit for bit
        q, k, v, cu_q, cu_k = make_varlen([100, 28], [100, 28], 4, 2, 64, torch.bfloat16, seed=41)
        first = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 100, 100, causal=True)
        again = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 100, 100, causal=True)
        assert torch.equal(first, again)
        cu = torch.tensor([0, 20, 128], dtype=torch.int32, device=DEV)
        cu_q.copy_(cu)
        cu_k.copy_(cu)
        moved = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 108, 108, causal=True)
        fresh = mfa.flash_attn_varlen_func(q, k, v, cu.clone(), cu.clone(), 108, 108, causal=True)
        assert torch.equal(moved, fresh)
        assert not torch.equal(moved, first)
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True)
        assert_output(moved, ref, torch.bfloat16, "rewritten cu_seqlens")

    def test_ragged_cross_lens(self):
        self.check_varlen([16, 33], [80, 7])
        self.check_varlen([16, 33, 0, 5], [80, 7, 9, 0], causal=True)  # empty q / empty k sequences

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_gqa(self, dtype):
        self.check_varlen([40, 24, 300], [40, 24, 300], Hq=8, Hkv=2, causal=True, dtype=dtype)

    def test_alibi_per_sequence(self):
        slopes = torch.tensor([[0.5, 0.25, 0.125, 0.0625], [0.1, 0.2, 0.3, 0.4]], device="cuda")
        self.check_varlen([40, 24], [40, 24], alibi=slopes)
        self.check_varlen([40, 24], [40, 24], alibi=slopes[0])

    @pytest.mark.parametrize("dtype", DTYPES)
    def test_boundaries_bit_exact(self, dtype):
        lens = [96, 257, 1, 130]
        q, k, v, cu_q, cu_k = make_varlen(lens, lens, 8, 2, 64, dtype, seed=4)
        out = mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens), max(lens), causal=True)
        starts = [0] + list(torch.tensor(lens).cumsum(0).tolist())
        for i in range(len(lens)):
            s, e = starts[i], starts[i + 1]
            dense = mfa.flash_attn_func(q[None, s:e], k[None, s:e], v[None, s:e], causal=True)[0]
            assert torch.equal(out[s:e], dense), f"sequence {i} differs from its dense B=1 call"
        # perturbing the other sequences leaves sequence 1 bit-identical
        q2, k2, v2 = q.clone(), k.clone(), v.clone()
        for t in (q2, k2, v2):
            t[: starts[1]] = 7.0
            t[starts[2]:] = -3.0
        out2 = mfa.flash_attn_varlen_func(q2, k2, v2, cu_q, cu_k, max(lens), max(lens), causal=True)
        assert torch.equal(out2[starts[1]:starts[2]], out[starts[1]:starts[2]])

    @pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
    def test_no_single_rows_flag(self, dtype):
        # with no sequence of one query row, the API skips the exact-row
        # launch (varlen_no_single_rows): the same bits as with it
        lens = [96, 257, 2, 130]
        q, k, v, cu_q, cu_k = make_varlen(lens, lens, 8, 2, 64, dtype, seed=5)
        a = _kernel.forward_varlen(q, k, v, cu_q, cu_k, 257, 257, 0.125, True, return_lse=True, no_single_rows=True)
        b = _kernel.forward_varlen(q, k, v, cu_q, cu_k, 257, 257, 0.125, True, return_lse=True)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert torch.equal(mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 257, 257, causal=True, softmax_scale=0.125),
                           b[0])

    def test_mismatched_batch_raises(self):
        q, k, v, cu_q, _ = make_varlen([32, 32], [32, 32], 4, 4, 64, torch.float16)
        cu_k_bad = torch.tensor([0, 64], dtype=torch.int32, device="cuda")
        with pytest.raises(ValueError):
            mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k_bad, 32, 64)


@pytest.mark.usefixtures("tile")
class TestPacked:
    def test_qkvpacked_matches_unpacked(self):
        g = torch.Generator().manual_seed(0)
        qkv = torch.randn(2, 96, 3, 4, 64, generator=g).to("cuda", torch.float16)
        out_p = mfa.flash_attn_qkvpacked_func(qkv, causal=True)
        q, k, v = qkv.unbind(dim=2)
        assert torch.equal(out_p, mfa.flash_attn_func(q, k, v, causal=True))
        assert torch.equal(out_p, mfa.flash_attn_func(q.contiguous(), k.contiguous(), v.contiguous(), causal=True))

    def test_kvpacked_matches_unpacked_gqa(self):
        g = torch.Generator().manual_seed(1)
        q = torch.randn(1, 64, 8, 64, generator=g).to("cuda", torch.float16)
        kv = torch.randn(1, 128, 2, 2, 64, generator=g).to("cuda", torch.float16)
        out_p = mfa.flash_attn_kvpacked_func(q, kv, softmax_scale=0.1)
        k, v = kv.unbind(dim=2)
        assert torch.equal(out_p, mfa.flash_attn_func(q, k, v, softmax_scale=0.1))

    def test_varlen_packed(self):
        g = torch.Generator().manual_seed(2)
        qkv = torch.randn(37 + 81, 3, 4, 64, generator=g).to("cuda", torch.float16)
        cu = torch.tensor([0, 37, 118], dtype=torch.int32, device="cuda")
        out_p = mfa.flash_attn_varlen_qkvpacked_func(qkv, cu, 81)
        q, k, v = qkv.unbind(dim=1)
        assert torch.equal(out_p, mfa.flash_attn_varlen_func(q, k, v, cu, cu, 81, 81))
        q = torch.randn(50, 4, 64, generator=g).to("cuda", torch.float16)
        kv = torch.randn(90, 2, 4, 64, generator=g).to("cuda", torch.float16)
        cu_q = torch.tensor([0, 20, 50], dtype=torch.int32, device="cuda")
        cu_k = torch.tensor([0, 60, 90], dtype=torch.int32, device="cuda")
        out_p = mfa.flash_attn_varlen_kvpacked_func(q, kv, cu_q, cu_k, 30, 60)
        k, v = kv.unbind(dim=1)
        assert torch.equal(out_p, mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 30, 60))


@pytest.mark.parametrize("L,H,kw", [
    (1000, 4, dict(causal=True)),
    (1536, 2, dict(causal=True, window_size=(300, 0))),
    (777, 3, dict(window_size=(100, 50), softcap=20.0)),
    (2048, 2, dict(causal=True, alibi=True)),
])
def test_pingpong_tile_heights_bit_exact(monkeypatch, L, H, kw):
    """The 512- and 256-row ping-pong tiles (the library picks the 256-row ones
    for causal calls with few tiles) give the same bits: each 32-row query
    block sees the same key blocks in the same order either way."""
    q, k, v = make_qkv(2, L, L, H, H, 64, torch.bfloat16, seed=L)
    kw = dict(kw)
    if kw.pop("alibi", False):
        kw["alibi_slopes"] = torch.rand(H, device="cuda") * 0.5
    outs = []
    for hint in (_hip.MFA_TILE_PINGPONG, _hip.MFA_TILE_PINGPONG256):
        monkeypatch.setattr(_kernel, "_TILE_HINT", hint)
        outs.append(mfa.flash_attn_func(q, k, v, **kw))
    assert torch.equal(outs[0], outs[1])


class TestBaselineConfigs:
    """BASELINE configs 2-5 at full size against the oracle (seconds of CPU each)."""

    def test_config2_bf16_d64_l8192(self):
        q, k, v = make_qkv(1, 8192, 8192, 16, 16, 64, torch.bfloat16, seed=1)
        e32, eout = check(q, k, v, "config2")
        print(f"config2 bf16: fp32-out err/max|ref| parity {e32:.3e}, bf16-out {eout:.3e}")

    def test_config3_fp16_d128_causal(self):
        q, k, v = make_qkv(1, 8192, 8192, 16, 16, 128, torch.float16, seed=2)
        e32, eout = check(q, k, v, "config3", causal=True)
        print(f"config3 fp16: fp32-out {e32:.3e}, fp16-out {eout:.3e}")

    def test_config4_varlen_gqa_causal(self):
        g = torch.Generator(device="cpu").manual_seed(3)
        lens = torch.randint(256, 4097, (8,), generator=g)
        assert lens.tolist() == [2706, 3501, 3030, 2221, 3090, 1748, 1214, 863]
        T = int(lens.sum())
        q = torch.randn(T, 32, 128, generator=g).to("cuda", torch.bfloat16)
        k = torch.randn(T, 8, 128, generator=g).to("cuda", torch.bfloat16)
        v = torch.randn(T, 8, 128, generator=g).to("cuda", torch.bfloat16)
        cu = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)]).to(torch.int32).to("cuda")
        out = mfa.flash_attn_varlen_func(q, k, v, cu, cu, int(lens.max()), int(lens.max()), causal=True)
        out32 = _kernel.forward_varlen(q, k, v, cu, cu, int(lens.max()), int(lens.max()), default_scale(128), True,
                                       out_dtype=torch.float32)
        ref = chunked.flash_attn_varlen_func(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True)
        e32 = assert_parity(out32, ref, torch.bfloat16, "config4")
        eout = assert_output(out, ref, torch.bfloat16, "config4")
        print(f"config4 bf16 varlen: fp32-out {e32:.3e}, bf16-out {eout:.3e}, max|ref| {ref.abs().max():.3f}")

    def test_config5_long_feature_mix_full_workload(self):
        """Config 5 at its workload: bf16 B=1 L=32768 H=16 D=128, causal, window
        (2048, 0), soft-cap 30, ALiBi 2^(-8(i+1)/16), inputs N(0,1)*0.5 from
        seed 4 (the reference's op order, _kernel.py:1188-1207: soft-cap
        :1191-1192 -> ALiBi :1193-1196 -> window masks :1201-1204).  The kernel
        runs on the whole sequence; the oracle checks five 512-row chunks of
        every head (before the window fills, as it fills, just after, the
        middle, the tail) one head at a time, which bounds its host memory."""
        L, H, D = 32768, 16, 128
        q, k, v = make_qkv(1, L, L, H, H, D, torch.bfloat16, seed=4, scale_inputs=0.5)
        slopes = torch.tensor([2 ** (-8 * (i + 1) / 16) for i in range(H)], dtype=torch.float32, device="cuda")
        kw = dict(causal=True, window_size=(2048, 0), softcap=30.0, alibi_slopes=slopes)
        out, out32 = run_both(q, k, v, **kw)
        torch.cuda.synchronize()
        chunk = 512
        starts = (0, 1536, 2048, 16384, L - chunk)
        rows = torch.cat([torch.arange(s0, s0 + chunk) for s0 in starts])
        qc, kc, vc, sc = q.cpu(), k.cpu(), v.cpu(), slopes.cpu()
        refs = []
        for h in range(H):
            ref = chunked.flash_attn_func(qc[:, :, h:h + 1], kc[:, :, h:h + 1], vc[:, :, h:h + 1], causal=True,
                                          window_size=(2048, 0), softcap=30.0, alibi_slopes=sc[h:h + 1],
                                          chunk=chunk, rows=set(starts))
            refs.append(ref[0, rows, 0])
        ref = torch.stack(refs, dim=1)  # [rows, H, D]
        assert not torch.isnan(ref).any()
        e32 = assert_parity(out32[0, rows], ref, torch.bfloat16, "config5 (fp32 output)")
        eout = assert_output(out[0, rows], ref, torch.bfloat16, "config5 (bf16 output)")
        rmax = ref.abs().max().item()
        print(f"config5 bf16: fp32-out err {e32:.3e} ({e32 / rmax:.3e} max|ref|), bf16-out {eout:.3e} "
              f"({eout / rmax:.3e} max|ref|), max|ref| {rmax:.3f}, rows checked {rows.numel()} x {H} heads")
