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
            kk = torch.zeros(1, 4, 96, 64, dtype=torch.float16)
            assert self.elig(q, kk, kk, causal=True) == (False, "causal-cross-length")
        finally:
            sdpa.uninstall()

    def test_fast_tier_fires_when_memory_fits(self):
        q = torch.zeros(1, 4, 2048, 64, dtype=torch.float16)
        assert sdpa.install()
        try:
            assert self.elig(q, q, q) == (True, "fast-tier")
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
        q = torch.zeros(1, 2, 512, 64, dtype=torch.float16)
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
