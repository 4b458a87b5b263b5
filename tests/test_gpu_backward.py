"""GPU parity of the backward pass (dq, dk, dv through torch autograd and the
mfa_bwd C ABI).  The reference is forward-only (metal_flash_attn/__init__.py:
3-4), so the oracle is torch autograd through the restated forward
(oracle.chunked.attention_grads, fp32 on the CPU), itself pinned against
finite differences in test_oracle_pinning.py.

Bar: every gradient within GRAD_REL * max|ref grad| of the oracle, judged on
fp32 gradients (the C ABI's dtype_grad = fp32).  Beyond the forward's
rounding of P to 16 bits, the backward rounds dS = P * (dP - Dsum) to 16 bits
for the dQ and dK products, and Dsum comes from the forward output O rounded
to 16 bits; the bar allows for those roundings (bf16: 2^-8 relative each).
The bf16/fp16 gradients returned by autograd are held to twice that bar.
Properties: two runs are bit-identical (no atomics), each varlen sequence's
gradients equal its dense B=1 call bit for bit, grouped-query dK/dV equal
the sum over the group's query heads of the repeated-K/V gradients (within
the bar), and the SDPA patch carries gradients.
"""
from __future__ import annotations

import pytest
import torch

import mtlflashattn_amd as mfa
from mtlflashattn_amd import _kernel
from oracle import chunked
from gpu_util import DEV, default_scale, make_qkv, make_varlen

pytestmark = pytest.mark.gpu

GRAD_REL = {torch.bfloat16: 6e-3, torch.float16: 1.5e-3}
DTYPES16 = [torch.bfloat16, torch.float16]


def grads_of(fn, q, k, v, dout):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out = fn(q, k, v)
    out.backward(dout)
    return out, q.grad, k.grad, v.grad


def rel_err(got, ref):
    ref = ref.float()
    scale = max(ref.abs().max().item(), 1e-6)
    return (got.detach().float().cpu() - ref).abs().max().item() / scale


def check_grads(got, ref, dtype, what, factor=1.0):
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        assert g.shape == r.shape, (what, name)
        e = rel_err(g, r)
        assert e <= factor * GRAD_REL[dtype], f"{what} {name}: rel err {e:.2e} > {factor * GRAD_REL[dtype]:.1e}"


def fp32_grads(q, k, v, dout, scale, **kw):
    """Gradients as fp32 straight from the C ABI (dtype_grad = fp32)."""
    out, lse = _kernel.forward_bshd(q, k, v, scale, kw.get("causal", False), kw.get("softcap", 0.0),
                                    kw.get("wl", -1), kw.get("wr", -1), kw.get("alibi"), return_lse=True)
    alibi, bstride = _kernel._alibi_arg(kw.get("alibi"), q.shape[0], q.shape[2], q.device)
    return _kernel._run_bwd(q, k, v, out, dout, lse, scale=scale, causal=kw.get("causal", False),
                            softcap=kw.get("softcap", 0.0), window_left=kw.get("wl", -1),
                            window_right=kw.get("wr", -1), alibi=alibi, alibi_bstride=bstride, grad_f32=True)


FEATURES = [
    dict(),
    dict(causal=True),
    dict(causal=True, window_size=(100, 0)),
    dict(window_size=(60, 30)),
    dict(softcap=5.0),
    dict(alibi=True, causal=True),
    dict(softcap=8.0, alibi=True, window_size=(90, 10)),
    dict(softmax_scale=-0.09),
]


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
@pytest.mark.parametrize("shape", [(2, 200, 333, 4, 2, 64), (1, 300, 150, 2, 2, 128)], ids=["lq<lk-gqa", "lq>lk-d128"])
def test_grads_match_oracle(dtype, feat, shape):
    B, Lq, Lk, Hq, Hkv, D = shape
    q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, dtype, seed=Lq + D)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(7)).to(DEV, dtype)
    kw = dict(feat)
    if kw.pop("alibi", False):
        kw["alibi_slopes"] = torch.linspace(0.05, 0.4, Hq, device=DEV)
    out, *got = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, **kw), q, k, v, dout)
    assert out.grad_fn is not None
    ref = chunked.attention_grads(q, k, v, dout, kw.get("softmax_scale"), kw.get("causal", False),
                                  kw.get("window_size", (-1, -1)), kw.get("softcap", 0.0),
                                  kw["alibi_slopes"].cpu() if "alibi_slopes" in kw else None)
    errs = [rel_err(g, r) for g, r in zip(got, ref)]
    print(f"\n[bwd] {dtype} {feat} {shape} rel err dq/dk/dv (16-bit grads) = " + ", ".join(f"{e:.2e}" for e in errs))
    check_grads(got, ref, dtype, f"{feat} {shape} 16-bit grads", factor=2.0)
    scale = kw.get("softmax_scale") or default_scale(D)
    ws = kw.get("window_size", (-1, -1))
    g32 = fp32_grads(q, k, v, dout, scale, causal=kw.get("causal", False), softcap=kw.get("softcap", 0.0),
                     wl=ws[0], wr=ws[1], alibi=kw.get("alibi_slopes"))
    errs = [rel_err(g, r) for g, r in zip(g32, ref)]
    print(f"[bwd] fp32 grads rel err = " + ", ".join(f"{e:.2e}" for e in errs))
    check_grads(g32, ref, dtype, f"{feat} {shape} fp32 grads")


@pytest.mark.parametrize("d", [8, 40, 96, 100])
def test_head_dims(d):
    q, k, v = make_qkv(1, 130, 170, 2, 1, d, torch.bfloat16, seed=d)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(8)).to(DEV, torch.bfloat16)
    _, *got = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True), q, k, v, dout)
    ref = chunked.attention_grads(q, k, v, dout, causal=True)
    check_grads(got, ref, torch.bfloat16, f"D={d}", factor=2.0)


@pytest.mark.parametrize("hq,hkv,D", [(4, 2, 64), (8, 2, 128), (16, 2, 128)])
def test_deterministic(hq, hkv, D):
    # D=128: the eight-wavefront dK/dV kernel; 16 query heads per 2 K/V heads
    # at this size also take the head-group partials and their summing kernel
    q, k, v = make_qkv(2, 257, 300, hq, hkv, D, torch.bfloat16, seed=9)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(9)).to(DEV, torch.bfloat16)
    f = lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True)  # noqa: E731
    a = grads_of(f, q, k, v, dout)
    b = grads_of(f, q, k, v, dout)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("dtype", DTYPES16)
def test_varlen_grads(dtype):
    lens_q, lens_k = [5, 0, 130, 1, 64], [9, 7, 200, 0, 64]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 4, 2, 64, dtype, seed=10)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(10)).to(DEV, dtype)
    f = lambda q, k, v: mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k),  # noqa: E731
                                                   causal=True)
    _, *got = grads_of(f, q, k, v, dout)
    ref = chunked.attention_grads_varlen(q, k, v, dout, cu_q.cpu(), cu_k.cpu(), causal=True)
    check_grads(got, ref, dtype, "varlen", factor=2.0)
    # each sequence equals its dense B=1 call bit for bit
    sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
    sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
    for i in range(len(lens_q)):
        if lens_q[i] == 0 or lens_k[i] == 0:
            continue
        a, b, c, d = sq[i], sq[i + 1], sk[i], sk[i + 1]
        _, dq, dk, dv = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True),
                                 q[None, a:b], k[None, c:d], v[None, c:d], dout[None, a:b])
        assert torch.equal(got[0][a:b], dq[0]) and torch.equal(got[1][c:d], dk[0]) and \
            torch.equal(got[2][c:d], dv[0]), f"sequence {i}"
    # keys of a sequence whose queries are empty get zero gradients
    assert (got[1][sk[1]:sk[2]] == 0).all() and (got[2][sk[1]:sk[2]] == 0).all()


def test_packed_and_heads_second_paths_carry_gradients():
    q, k, v = make_qkv(1, 100, 100, 4, 4, 64, torch.float16, seed=11)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(11)).to(DEV, torch.float16)
    _, *ref = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True), q, k, v, dout)
    qkv = torch.stack([q, k, v], dim=2).detach().requires_grad_(True)
    mfa.flash_attn_qkvpacked_func(qkv, causal=True).backward(dout)
    assert torch.equal(qkv.grad[:, :, 0], ref[0]) and torch.equal(qkv.grad[:, :, 1], ref[1])
    _, *hs = grads_of(lambda q, k, v: mfa.flash_attn_forward(q.transpose(1, 2), k.transpose(1, 2),
                                                             v.transpose(1, 2), default_scale(64), True)
                      .transpose(1, 2), q, k, v, dout)
    for a, b in zip(hs, ref):
        assert torch.equal(a, b)


def test_sdpa_patch_carries_gradients(monkeypatch):
    from mtlflashattn_amd import sdpa
    import torch.nn.functional as F

    calls = []
    real = _kernel._run_bwd
    monkeypatch.setattr(_kernel, "_run_bwd", lambda *a, **kw: calls.append(1) or real(*a, **kw))

    q, k, v = (t.transpose(1, 2) for t in make_qkv(1, 600, 600, 4, 4, 64, torch.bfloat16, seed=12))
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(12)).to(DEV, torch.bfloat16)
    sdpa.install()
    try:
        _, *got = grads_of(lambda q, k, v: F.scaled_dot_product_attention(q, k, v, is_causal=True), q, k, v, dout)
    finally:
        sdpa.uninstall()
    ref = chunked.attention_grads(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), dout.transpose(1, 2),
                                  causal=True)
    assert calls, "the patched SDPA call did not run the HIP backward"
    check_grads([g.transpose(1, 2) for g in got], ref, torch.bfloat16, "sdpa", factor=2.0)


# fp32 gradients of fp32 inputs (the fp32 kernels: fp32 end to end), against
# float64 autograd of the oracle: within FP32_GRAD_REL * max|ref grad|.
FP32_GRAD_REL = 5e-6  # (measured: at most 1.1e-6 over these cases)


def check_fp32_grads(got, ref, what):
    errs = []
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        assert g.dtype == torch.float32 and g.shape == r.shape, (what, name)
        e = rel_err(g, r)
        errs.append(e)
        assert e <= FP32_GRAD_REL, f"{what} {name}: rel err {e:.2e} > {FP32_GRAD_REL:.0e}"
    return errs


@pytest.mark.parametrize("feat", FEATURES, ids=[str(i) for i in range(len(FEATURES))])
@pytest.mark.parametrize("shape", [(2, 200, 333, 4, 2, 64), (1, 300, 150, 2, 2, 128), (1, 130, 170, 2, 1, 40),
                                   (1, 90, 70, 3, 3, 96), (1, 50, 60, 2, 2, 33)],
                         ids=["lq<lk-gqa", "lq>lk-d128", "d40-mqa", "d96", "d33"])
def test_fp32_grads_match_oracle(feat, shape):
    B, Lq, Lk, Hq, Hkv, D = shape
    q, k, v = make_qkv(B, Lq, Lk, Hq, Hkv, D, torch.float32, seed=Lq + D)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(7)).to(DEV)
    kw = dict(feat)
    if kw.pop("alibi", False):
        kw["alibi_slopes"] = torch.linspace(0.05, 0.4, Hq, device=DEV)
    _, *got = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, **kw), q, k, v, dout)
    ref = chunked.attention_grads(q, k, v, dout, kw.get("softmax_scale"), kw.get("causal", False),
                                  kw.get("window_size", (-1, -1)), kw.get("softcap", 0.0),
                                  kw["alibi_slopes"].cpu() if "alibi_slopes" in kw else None, dtype=torch.float64)
    errs = check_fp32_grads(got, ref, f"fp32 {feat} {shape}")
    print(f"\n[bwd fp32] {feat} {shape} rel err dq/dk/dv = " + ", ".join(f"{e:.2e}" for e in errs))


def test_fp32_lse_gradient():
    # a loss on the returned lse enters the row sums (Dsum - dlse)
    q, k, v = make_qkv(1, 100, 120, 2, 2, 64, torch.float32, seed=21)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(21)).to(DEV)
    dlse = torch.randn(1, 2, 100, generator=torch.Generator().manual_seed(22)).to(DEV)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out, lse = mfa.flash_attn_func_with_lse(qg, kg, vg, causal=True)
    ((out * dout).sum() + (lse * dlse).sum()).backward()
    ref = chunked.attention_grads(q, k, v, dout, causal=True, dtype=torch.float64, dlse=dlse)
    check_fp32_grads((qg.grad, kg.grad, vg.grad), ref, "fp32 lse gradient")


def test_fp32_varlen_grads():
    lens_q, lens_k = [5, 0, 130, 1, 64], [9, 7, 200, 0, 64]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 4, 2, 64, torch.float32, seed=23)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(23)).to(DEV)
    f = lambda q, k, v: mfa.flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k),  # noqa: E731
                                                   causal=True, softcap=6.0)
    _, *got = grads_of(f, q, k, v, dout)
    ref = chunked.attention_grads_varlen(q, k, v, dout, cu_q.cpu(), cu_k.cpu(), causal=True, softcap=6.0,
                                         dtype=torch.float64)
    check_fp32_grads(got, ref, "fp32 varlen")
    _, *again = grads_of(f, q, k, v, dout)
    assert all(torch.equal(a, b) for a, b in zip(got, again))  # no atomics: bit-identical
    sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
    sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
    for i in range(len(lens_q)):
        if lens_q[i] == 0 or lens_k[i] == 0:
            continue
        a, b, c, d = sq[i], sq[i + 1], sk[i], sk[i + 1]
        _, dq, dk, dv = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True, softcap=6.0),
                                 q[None, a:b], k[None, c:d], v[None, c:d], dout[None, a:b])
        assert torch.equal(got[0][a:b], dq[0]) and torch.equal(got[1][c:d], dk[0]) and \
            torch.equal(got[2][c:d], dv[0]), f"sequence {i}"
    assert (got[1][sk[1]:sk[2]] == 0).all() and (got[2][sk[1]:sk[2]] == 0).all()


def test_gqa_grads_equal_summed_repeated_heads():
    q, k, v = make_qkv(1, 150, 170, 8, 2, 64, torch.bfloat16, seed=14)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(14)).to(DEV, torch.bfloat16)
    f = lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True)  # noqa: E731
    _, dq, dk, dv = grads_of(f, q, k, v, dout)
    _, dq_r, dk_r, dv_r = grads_of(f, q, k.repeat_interleave(4, dim=2), v.repeat_interleave(4, dim=2), dout)
    assert torch.equal(dq, dq_r)  # the dQ kernel does the same arithmetic per query head
    for g, r in ((dk, dk_r), (dv, dv_r)):
        summed = r.float().reshape(1, 170, 2, 4, 64).sum(3)
        assert rel_err(g, summed.cpu()) <= GRAD_REL[torch.bfloat16]


@pytest.mark.parametrize("B,L,hq,hkv", [(4, 2048, 16, 8), (1, 8192, 16, 4)], ids=["one-group", "two-groups"])
def test_gqa_head_groups_at_d128(B, L, hq, hkv):
    # grouped-query dK/dV at head dim 128 with one workgroup per K/V head
    # looping over its query heads (512 workgroups already) and with two
    # groups of query heads whose fp32 partials are summed
    q, k, v = make_qkv(B, L, L, hq, hkv, 128, torch.bfloat16, seed=L + hkv)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(L)).to(DEV, torch.bfloat16)
    f = lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=True)  # noqa: E731
    r = hq // hkv
    _, dq, dk, dv = grads_of(f, q, k, v, dout)
    _, dq_r, dk_r, dv_r = grads_of(f, q, k.repeat_interleave(r, dim=2), v.repeat_interleave(r, dim=2), dout)
    assert torch.equal(dq, dq_r)
    for g, rep in ((dk, dk_r), (dv, dv_r)):
        summed = rep.float().reshape(B, L, hkv, r, 128).sum(3)
        assert rel_err(g, summed.cpu()) <= GRAD_REL[torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES16)
def test_lse_gradient(dtype):
    # loss = sum(out * dout) + sum(lse * dlse): the lse gradient enters as Dsum - dlse
    q, k, v = make_qkv(1, 160, 220, 4, 2, 64, dtype, seed=15)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(15)).to(DEV, dtype)
    dlse = torch.randn(1, 4, 160, generator=torch.Generator().manual_seed(16)).to(DEV)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out, lse = mfa.flash_attn_func_with_lse(qg, kg, vg, causal=True)
    ((out.float() * dout.float()).sum() + (lse * dlse).sum()).backward()
    ref = chunked.attention_grads(q, k, v, dout, causal=True, dlse=dlse)
    check_grads((qg.grad, kg.grad, vg.grad), ref, dtype, "lse gradient", factor=2.0)


def test_merged_key_shards_train_like_full_attention():
    # context-parallel use: attention over key shards merged by lse, end to end
    # differentiable, gives the gradients of attention over all keys
    q, k, v = make_qkv(1, 120, 300, 4, 4, 64, torch.bfloat16, seed=17)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(17)).to(DEV, torch.bfloat16)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    parts = [mfa.flash_attn_func_with_lse(qg, kg[:, a:b], vg[:, a:b]) for a, b in ((0, 100), (100, 101), (101, 300))]
    out, _ = mfa.merge_attention_partials([o for o, _ in parts], [l for _, l in parts])
    (out.float() * dout.float()).sum().backward()
    ref = chunked.attention_grads(q, k, v, dout)
    check_grads((qg.grad, kg.grad, vg.grad), ref, torch.bfloat16, "merged shards", factor=2.0)


@pytest.mark.parametrize("lq,lk,causal", [(5, 1, False), (1, 1, True), (1, 700, True), (3, 2, True), (33, 65, False),
                                          (200, 7, True)])
def test_edge_lengths(lq, lk, causal):
    q, k, v = make_qkv(2, lq, lk, 4, 2, 64, torch.bfloat16, seed=lq * 100 + lk)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(lq + lk)).to(DEV, torch.bfloat16)
    _, *got = grads_of(lambda q, k, v: mfa.flash_attn_func(q, k, v, causal=causal), q, k, v, dout)
    ref = chunked.attention_grads(q, k, v, dout, causal=causal)
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        if r.abs().max() == 0:
            # identically zero in exact arithmetic (one key: dS = dP - Dsum = 0);
            # the kernel's two fp32 sums of dO.v differ only in rounding
            assert g.float().abs().max().item() <= 1e-3, f"{name} Lq={lq} Lk={lk}"
        else:
            e = rel_err(g, r)
            assert e <= 2 * GRAD_REL[torch.bfloat16], f"{name} Lq={lq} Lk={lk} causal={causal}: rel err {e:.2e}"


def test_varlen_with_empty_key_sequences_and_lse_gradient():
    lens_q, lens_k = [3, 4, 0, 2], [0, 50, 9, 300]
    q, k, v, cu_q, cu_k = make_varlen(lens_q, lens_k, 4, 4, 64, torch.float16, seed=18)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(18)).to(DEV, torch.float16)
    dlse = torch.randn(4, sum(lens_q), generator=torch.Generator().manual_seed(19)).to(DEV)
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out, lse = mfa.flash_attn_varlen_func_with_lse(qg, kg, vg, cu_q, cu_k, max(lens_q), max(lens_k), causal=True)
    assert torch.isneginf(lse[:, :3]).all()  # the first sequence has no key
    ((out.float() * dout.float()).sum() + (torch.where(torch.isinf(lse), 0, lse) * dlse).sum()).backward()
    sq = [0] + torch.tensor(lens_q).cumsum(0).tolist()
    sk = [0] + torch.tensor(lens_k).cumsum(0).tolist()
    ref = chunked.attention_grads_varlen(q, k, v, dout, cu_q.cpu(), cu_k.cpu(), causal=True)
    # the lse term per sequence through the dense oracle
    for i in range(len(lens_q)):
        a, b, c, d = sq[i], sq[i + 1], sk[i], sk[i + 1]
        if b == a or d == c:
            continue
        gi = chunked.attention_grads(q[None, a:b], k[None, c:d], v[None, c:d], torch.zeros_like(dout[None, a:b]),
                                     causal=True, dlse=dlse[None, :, a:b])
        ref[0][a:b] += gi[0][0]
        ref[1][c:d] += gi[1][0]
        ref[2][c:d] += gi[2][0]
    check_grads((qg.grad, kg.grad, vg.grad), ref, torch.float16, "varlen + lse gradient", factor=2.0)
    assert torch.count_nonzero(qg.grad[:3]) == 0


def test_long_rows_config3_shape():
    """Gradients at config 3's full shape (fp16, B=1, L=8192, H=16, D=128,
    causal; inputs from seed 2): every head runs on the kernels, and the full
    dq/dk/dv of heads 0 and 15 (8192-key rows, long causal tails) are checked
    against the oracle's autograd."""
    q, k, v = make_qkv(1, 8192, 8192, 16, 16, 128, torch.float16, seed=2)
    g = torch.Generator().manual_seed(3)
    dout = torch.randn(q.shape, generator=g).to(DEV, torch.float16)
    dq, dk, dv = fp32_grads(q, k, v, dout, default_scale(128), causal=True)
    torch.cuda.synchronize()
    for h in (0, 15):
        sl = slice(h, h + 1)
        ref = chunked.attention_grads(q[:, :, sl], k[:, :, sl], v[:, :, sl], dout[:, :, sl], causal=True)
        got = (dq[:, :, sl], dk[:, :, sl], dv[:, :, sl])
        errs = [rel_err(a, b) for a, b in zip(got, ref)]
        print(f"config3 shape head {h}: dq {errs[0]:.2e} dk {errs[1]:.2e} dv {errs[2]:.2e} (x max|ref|)")
        check_grads(got, ref, torch.float16, f"config3 shape head {h}")


def test_long_rows_config2_shape():
    """Gradients at config 2's shape (bf16, B=1, L=8192, H=16, D=64,
    non-causal; inputs from seed 1): the full dq/dk/dv of heads 0 and 15
    against the oracle's autograd."""
    q, k, v = make_qkv(1, 8192, 8192, 16, 16, 64, torch.bfloat16, seed=1)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(4)).to(DEV, torch.bfloat16)
    dq, dk, dv = fp32_grads(q, k, v, dout, default_scale(64))
    torch.cuda.synchronize()
    for h in (0, 15):
        sl = slice(h, h + 1)
        ref = chunked.attention_grads(q[:, :, sl], k[:, :, sl], v[:, :, sl], dout[:, :, sl])
        got = (dq[:, :, sl], dk[:, :, sl], dv[:, :, sl])
        errs = [rel_err(a, b) for a, b in zip(got, ref)]
        print(f"config2 shape head {h}: dq {errs[0]:.2e} dk {errs[1]:.2e} dv {errs[2]:.2e} (x max|ref|)")
        check_grads(got, ref, torch.bfloat16, f"config2 shape head {h}")


def test_config4_shape_varlen_gqa():
    """Gradients at config 4's shape (bf16 varlen, lengths from seed 3, Hq=32,
    Hkv=8, D=128, causal): every sequence and head runs on the kernels (dK/dV
    of a K/V head summed over its 4 query heads from fp32 partials); the
    oracle checks K/V head groups 0 and 7 (query heads 0-3 and 28-31) of the
    longest (3501) and the shortest (863) sequence in full."""
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(256, 4097, (8,), generator=g)
    T = int(lens.sum())
    q = torch.randn(T, 32, 128, generator=g).to(DEV, torch.bfloat16)
    k = torch.randn(T, 8, 128, generator=g).to(DEV, torch.bfloat16)
    v = torch.randn(T, 8, 128, generator=g).to(DEV, torch.bfloat16)
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)]).to(torch.int32).to(DEV)
    mx = int(lens.max())
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(5)).to(DEV, torch.bfloat16)
    out, lse = _kernel.forward_varlen(q, k, v, cu, cu, mx, mx, default_scale(128), True, return_lse=True)
    dq, dk, dv = _kernel._run_bwd(q[None], k[None], v[None], out[None], dout[None], lse, scale=default_scale(128),
                                  causal=True, softcap=0.0, window_left=-1, window_right=-1, alibi=None,
                                  alibi_bstride=0, cu_q=cu, cu_k=cu, seqlen_q=mx, seqlen_k=mx, grad_f32=True)
    torch.cuda.synchronize()
    starts = [0] + lens.cumsum(0).tolist()
    ls = lens.tolist()
    for i in (ls.index(max(ls)), ls.index(min(ls))):
        a, b = starts[i], starts[i + 1]
        for grp in (0, 7):
            hq, hk = slice(4 * grp, 4 * grp + 4), slice(grp, grp + 1)
            ref = chunked.attention_grads(q[None, a:b, hq], k[None, a:b, hk], v[None, a:b, hk], dout[None, a:b, hq],
                                          causal=True)
            got = (dq[:, a:b, hq], dk[:, a:b, hk], dv[:, a:b, hk])
            errs = [rel_err(x, y) for x, y in zip(got, ref)]
            print(f"config4 shape seq {i} (L={b - a}) kv head {grp}: dq {errs[0]:.2e} dk {errs[1]:.2e} "
                  f"dv {errs[2]:.2e} (x max|ref|)")
            check_grads(got, ref, torch.bfloat16, f"config4 shape seq {i} kv head {grp}")


def test_config5_shape_window_softcap_alibi():
    """Gradients at config 5's shape (bf16, B=1, L=32768, H=16, D=128, causal,
    window (2048, 0), soft-cap 30, ALiBi 2^(-8(i+1)/16), inputs N(0,1)*0.5
    from seed 4): every head runs on the kernels.  The oracle runs on slices
    of heads 0 and 15: rows [a, a+4096) against keys [a-2048, a+4096) keep
    every position difference i - j (bottom-right causal, window and ALiBi
    distances) of the full problem, so dq of those rows and dk/dv of keys
    [a, a+2048) -- whose every contributing row lies in the slice -- are
    exact; a = 0 (before the window fills) and a = 16384."""
    L, H, D = 32768, 16, 128
    q, k, v = make_qkv(1, L, L, H, H, D, torch.bfloat16, seed=4, scale_inputs=0.5)
    slopes = torch.tensor([2 ** (-8 * (i + 1) / 16) for i in range(H)], dtype=torch.float32, device=DEV)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(6)).to(DEV, torch.bfloat16)
    kw = dict(causal=True, softcap=30.0, wl=2048, wr=0, alibi=slopes)
    dq, dk, dv = fp32_grads(q, k, v, dout, default_scale(D), **kw)
    torch.cuda.synchronize()
    for a in (0, 16384):
        k0 = max(a - 2048, 0)
        for h in (0, 15):
            sl = slice(h, h + 1)
            ref = chunked.attention_grads(q[:, a:a + 4096, sl], k[:, k0:a + 4096, sl], v[:, k0:a + 4096, sl],
                                          dout[:, a:a + 4096, sl], causal=True, window_size=(2048, 0), softcap=30.0,
                                          alibi_slopes=slopes[sl].cpu())
            got = (dq[:, a:a + 4096, sl], dk[:, a:a + 2048, sl], dv[:, a:a + 2048, sl])
            ref = (ref[0], ref[1][:, a - k0:a - k0 + 2048], ref[2][:, a - k0:a - k0 + 2048])
            errs = [rel_err(x, y) for x, y in zip(got, ref)]
            print(f"config5 shape rows {a}.. head {h}: dq {errs[0]:.2e} dk {errs[1]:.2e} dv {errs[2]:.2e} (x max|ref|)")
            check_grads(got, ref, torch.bfloat16, f"config5 shape rows {a} head {h}")
