"""Gated F.scaled_dot_product_attention patch (the reference's
tests/test_sdpa_patch.py).  CPU tests cover install/uninstall, the kill switch,
the env-configurable gates and the never-crash fallback; GPU tests check that
eligible calls route to the HIP kernel and match the oracle."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from mtlflashattn_amd import _kernel, sdpa


@pytest.fixture
def patched():
    assert sdpa.install(min_score_gb=1e-9)
    yield sdpa
    sdpa.uninstall()


def test_install_uninstall_restores_original():
    orig = F.scaled_dot_product_attention
    assert sdpa.install(min_score_gb=1e-9)
    assert F.scaled_dot_product_attention is not orig
    assert torch.nn.functional.scaled_dot_product_attention is F.scaled_dot_product_attention
    assert not sdpa.install(min_score_gb=1e-9)  # idempotent
    assert sdpa.uninstall()
    assert F.scaled_dot_product_attention is orig
    assert not sdpa.uninstall()


def test_kill_switch_blocks_install(monkeypatch):
    monkeypatch.setenv("MTLFLASHATTN_SDPA", "off")
    orig = F.scaled_dot_product_attention
    assert not sdpa.install(min_score_gb=1e-9)
    assert F.scaled_dot_product_attention is orig


def test_cpu_calls_use_stock(patched):
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 2, 64, 32, generator=g) for _ in range(3))
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.equal(out, patched._orig(q, k, v, is_causal=True))
    assert patched._eligibility(q, k, v, None, 0.0, False) == (False, "not-rocm")


class TestGates:
    """_eligibility on CPU tensors with the device predicate patched to accept them."""

    @pytest.fixture(autouse=True)
    def rocm(self, monkeypatch):
        monkeypatch.setattr(sdpa, "_on_rocm_gpu", lambda t: True)

    def elig(self, q, k, v, mask=None, dropout=0.0, causal=False):
        return sdpa._eligibility(q, k, v, mask, dropout, causal)

    def test_disqualifiers(self):
        q = torch.zeros(1, 4, 64, 64, dtype=torch.float16)
        assert sdpa.install()
        try:
            assert self.elig(q, q, q, mask=torch.zeros(64, 64)) == (False, "attn_mask")
            assert self.elig(q, q, q, dropout=0.1) == (False, "dropout")
            assert self.elig(q[0], q[0], q[0])[1].startswith("ndim")
            assert self.elig(q.double(), q.double(), q.double())[1].startswith("dtype")
            big = torch.zeros(1, 4, 64, 160, dtype=torch.float16)
            assert self.elig(big, big, big)[1].startswith("head_dim")
            assert self.elig(q, q[:, :3], q[:, :3])[1].startswith("heads")
            assert self.elig(q, q, q[:, :, :32]) == (False, "kv-len-mismatch")
            # batch / value-head mismatches stay on stock SDPA (the kernel
            # would read past the K/V allocation)
            q4 = torch.zeros(4, 4, 64, 64, dtype=torch.float16)
            k2 = torch.zeros(2, 4, 64, 64, dtype=torch.float16)
            assert self.elig(q4, k2, k2) == (False, "batch-or-heads-mismatch")
            assert self.elig(q, q, q[:, :2]) == (False, "batch-or-heads-mismatch")
            kk = torch.zeros(1, 4, 96, 64, dtype=torch.float16)
            assert self.elig(q, kk, kk, causal=True) == (False, "causal-cross-length")
        finally:
            sdpa.uninstall()

    def test_fp32_under_autograd_stays_stock(self):
        # fp32 calls whose inputs need gradients go to stock SDPA (the HIP
        # fp32 backward runs on the vector ALU), 16-bit ones keep the kernel
        assert sdpa.install()
        try:
            q = torch.zeros(1, 2, 1024, 64, dtype=torch.float32, requires_grad=True)
            assert self.elig(q, q, q) == (False, "grad-fp32")
            with torch.no_grad():
                assert self.elig(q, q, q) == (True, "fast-tier")
            assert self.elig(q.detach(), q.detach(), q.detach()) == (True, "fast-tier")
            h = torch.zeros(1, 2, 1024, 64, dtype=torch.bfloat16, requires_grad=True)
            assert self.elig(h, h, h) == (True, "fast-tier")
        finally:
            sdpa.uninstall()

    def test_fast_tier_fires_when_memory_fits(self):
        q = torch.zeros(1, 4, 2048, 64, dtype=torch.float16)
        assert sdpa.install()
        try:
            assert self.elig(q, q, q) == (True, "fast-tier")
        finally:
            sdpa.uninstall()

    def test_rocm_derived_fast_floor_and_tiers(self):
        # fp16/bf16 from 512 tokens, fp32 too (measured against stock ROCm SDPA)
        assert sdpa.install()
        try:
            for dt in (torch.float16, torch.bfloat16, torch.float32):
                q = torch.zeros(1, 2, 512, 64, dtype=dt)
                assert self.elig(q, q, q) == (True, "fast-tier"), dt
                q = torch.zeros(1, 2, 511, 64, dtype=dt)
                assert self.elig(q, q, q)[1].startswith("fits"), dt
            # head dim not a multiple of 8 (padded copies): only the other gates
            q = torch.zeros(1, 2, 1024, 100, dtype=torch.float16)
            assert self.elig(q, q, q)[1].startswith("fits")
        finally:
            sdpa.uninstall()

    def test_uneven_value_head_dim_is_eligible(self):
        q = torch.zeros(1, 2, 1024, 64, dtype=torch.float16)
        assert sdpa.install()
        try:
            for dv in (32, 128, 200, 256):
                v = torch.zeros(1, 2, 1024, dv, dtype=torch.float16)
                assert self.elig(q, q, v) == (True, "fast-tier"), dv
            v = torch.zeros(1, 2, 1024, 128, dtype=torch.float16)
            assert self.elig(q, q, v, mask=torch.zeros(1024, 1024)) == (False, "attn_mask")
            k = torch.zeros(1, 2, 1000, 64, dtype=torch.float16)
            assert self.elig(q, k, v[:, :, :1000], causal=True) == (False, "causal-cross-length")
            big = torch.zeros(1, 2, 1024, 160, dtype=torch.float16)
            assert self.elig(big, big, v)[1].startswith("head_dim")
        finally:
            sdpa.uninstall()

    def test_tiny_stays_stock(self):
        q = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
        assert sdpa.install()
        try:
            ok, reason = self.elig(q, q, q)
        finally:
            sdpa.uninstall()
        assert not ok and reason.startswith("fits")

    def test_large_seq_fires_for_every_tier(self):
        q = torch.zeros(1, 2, 4096, 100, dtype=torch.float32)  # neither fast nor huge
        assert sdpa.install()
        try:
            assert self.elig(q, q, q) == (True, "correctness-large-seq")
        finally:
            sdpa.uninstall()

    def test_env_configurable_floors(self, monkeypatch):
        q = torch.zeros(1, 2, 300, 64, dtype=torch.float16)
        monkeypatch.setenv("MTLFLASHATTN_SDPA_FAST_MIN_SEQ", "256")
        assert sdpa.install()
        try:
            assert self.elig(q, q, q) == (True, "fast-tier")
        finally:
            sdpa.uninstall()
        q = torch.zeros(1, 2, 512, 100, dtype=torch.float32)
        monkeypatch.setenv("MTLFLASHATTN_SDPA_MIN_SEQ", "256")
        assert sdpa.install()
        try:
            assert self.elig(q, q, q) == (True, "correctness-large-seq")
        finally:
            sdpa.uninstall()

    def test_memory_gate(self):
        q = torch.zeros(2, 8, 512, 100, dtype=torch.float32)
        assert sdpa.install(min_score_gb=0.001)
        try:
            assert self.elig(q, q, q) == (True, "oom-rescue")
        finally:
            sdpa.uninstall()

    def test_kernel_error_falls_back_to_stock(self, monkeypatch, capsys):
        def boom(*a, **k):
            raise RuntimeError("boom")

        monkeypatch.setattr(sdpa, "flash_attn_forward", boom)
        g = torch.Generator().manual_seed(1)
        q, k, v = (torch.randn(1, 2, 64, 32, generator=g) for _ in range(3))
        assert sdpa.install(min_score_gb=1e-9)
        try:
            out = F.scaled_dot_product_attention(q, k, v)
            stock = sdpa._orig(q, k, v)
        finally:
            sdpa.uninstall()
        assert torch.equal(out, stock)
        assert "fell back (boom)" in capsys.readouterr().out


@pytest.mark.gpu
class TestSdpaOnGpu:
    def make(self, B, H, Lq, Lk, D, dtype=torch.float16, Hkv=None, seed=0):
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(B, H, Lq, D, generator=g).to("cuda", dtype)
        k = torch.randn(B, Hkv or H, Lk, D, generator=g).to("cuda", dtype)
        v = torch.randn(B, Hkv or H, Lk, D, generator=g).to("cuda", dtype)
        return q, k, v

    def ref(self, q, k, v, causal=False, scale=None):
        from oracle import chunked

        s = scale if scale is not None else q.shape[-1] ** -0.5
        return chunked.flash_torch(q.cpu(), k.cpu(), v.cpu(), s, causal)

    def test_eligible_routes_to_kernel(self, patched, monkeypatch):
        calls = []
        orig = sdpa.flash_attn_forward

        def spy(*a, **kw):
            calls.append(1)
            return orig(*a, **kw)

        monkeypatch.setattr(sdpa, "flash_attn_forward", spy)
        q, k, v = self.make(1, 4, 128, 128, 64)
        out = F.scaled_dot_product_attention(q, k, v)
        assert calls
        ref = self.ref(q, k, v)
        assert (out.float().cpu() - ref).abs().max() <= 4e-3 * ref.abs().max()

    def test_causal_gqa_and_scale(self, patched):
        q, k, v = self.make(1, 8, 96, 96, 64, dtype=torch.float32, Hkv=2)
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        assert (out.cpu() - self.ref(q, k, v, causal=True)).abs().max() <= 1e-5
        out = F.scaled_dot_product_attention(q, k, v, scale=0.5, enable_gqa=True)
        assert (out.cpu() - self.ref(q, k, v, scale=0.5)).abs().max() <= 1e-5

    def test_cross_length_causal_falls_back(self, patched):
        q, k, v = self.make(1, 2, 32, 96, 64)
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        assert torch.equal(out, patched._orig(q, k, v, is_causal=True))

    def test_attn_mask_falls_back(self, patched):
        q, k, v = self.make(1, 2, 64, 64, 64)
        mask = torch.zeros(64, 64, device="cuda", dtype=torch.float16)
        mask[:, 32:] = float("-inf")
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        assert torch.equal(out, patched._orig(q, k, v, attn_mask=mask))

    @pytest.mark.parametrize("d,dv", [(128, 64), (64, 128), (64, 200), (40, 96)])
    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    def test_uneven_value_head_dim_on_the_kernel(self, patched, monkeypatch, d, dv, dtype):
        from oracle import chunked

        calls = []
        orig = sdpa.flash_attn_forward
        monkeypatch.setattr(sdpa, "flash_attn_forward", lambda *a, **kw: calls.append(1) or orig(*a, **kw))
        g = torch.Generator().manual_seed(d + dv)
        q = torch.randn(1, 8, 96, d, generator=g).to("cuda", dtype)
        k = torch.randn(1, 2, 96, d, generator=g).to("cuda", dtype)
        v = torch.randn(1, 2, 96, dv, generator=g).to("cuda", dtype)
        for causal in (False, True):
            calls.clear()
            out = F.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True)
            assert calls, "uneven-V call did not reach the HIP kernel"
            assert len(calls) == -(-dv // 128)  # one launch per 128 value columns
            assert out.shape == (1, 8, 96, dv) and out.dtype == dtype
            ref = chunked.uneven_v_attention(q.float(), k.float(), v.float(), is_causal=causal, enable_gqa=True)
            err = (out.float().cpu() - ref).abs().max().item()
            bar = 1e-5 if dtype == torch.float32 else 4e-3 * ref.abs().max().item()
            assert err <= bar, f"D={d} Dv={dv} causal={causal}: err {err:.3e} > {bar:.3e}"

    def test_fp32_gradients_flow_through_the_patch(self, patched):
        # fp32 training through the patched op: stock SDPA serves it and the
        # gradients match stock's; bf16 gradients come from the HIP backward
        g = torch.Generator().manual_seed(5)
        base = [torch.randn(1, 2, 1024, 64, generator=g) for _ in range(3)]
        q, k, v = (x.to("cuda").requires_grad_(True) for x in base)
        F.scaled_dot_product_attention(q, k, v).sum().backward()
        q2, k2, v2 = (x.to("cuda").requires_grad_(True) for x in base)
        patched._orig(q2, k2, v2).sum().backward()
        for a, b in ((q, q2), (k, k2), (v, v2)):
            assert torch.equal(a.grad, b.grad)
        qh, kh, vh = (x.to("cuda", torch.bfloat16).requires_grad_(True) for x in base)
        F.scaled_dot_product_attention(qh, kh, vh).float().sum().backward()
        assert all(t.grad is not None and torch.isfinite(t.grad.float()).all() for t in (qh, kh, vh))

    def test_uneven_value_head_dim_with_mask_stays_stock(self, patched):
        q, k, _ = self.make(1, 2, 64, 64, 64)
        v = torch.randn(1, 2, 64, 96, device="cuda", dtype=torch.float16)
        mask = torch.zeros(64, 64, device="cuda", dtype=torch.float16)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        assert torch.equal(out, patched._orig(q, k, v, attn_mask=mask))
