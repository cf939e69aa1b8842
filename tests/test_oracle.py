"""Pins the CPU oracle (oracle/hk_oracle.cpp) before it is trusted as the parity target.

The reference repository stores no golden vectors (all its inputs are generated at run time),
so every oracle function is pinned here by checks that a plausible slip (dropped term, wrong
sign, transposed operand, swapped bias correction) would fail:
  - published known-answer values of the generators (MT19937-64, SplitMix64);
  - the reference harness's own cross-check where it has one (GELU backward vs a central
    difference, kernels_test.cu:271-279; the reduce self-test's exact input,
    unified_reduce_standalone.cu:821);
  - independent library routines in float64 on the CPU (torch.nn.functional / torch.optim /
    numpy matmul), i.e. the textbook operation the reference formula implements;
  - invariants (softmax rows sum to one, CE gradient rows sum to zero, causal row 0 attends
    only to key 0, AdamW with zero gradient and zero decay leaves p unchanged).
All CPU-only; sizes keep the suite within seconds.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import max_rel

# ---------------------------------------------------------------------------------------------
# generators
# ---------------------------------------------------------------------------------------------


def _mt19937_64(seed: int):
    """MT19937-64 (Matsumoto & Nishimura, 2004), written from the published algorithm."""
    n, m, mask = 312, 156, (1 << 64) - 1
    mt = [0] * n
    mt[0] = seed & mask
    for i in range(1, n):
        mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & mask
    idx = n
    upper, lower = 0xFFFFFFFF80000000, 0x7FFFFFFF
    while True:
        if idx >= n:
            for i in range(n):
                x = (mt[i] & upper) | (mt[(i + 1) % n] & lower)
                xa = x >> 1
                if x & 1:
                    xa ^= 0xB5026F5AA96619E9
                mt[i] = mt[(i + m) % n] ^ xa
            idx = 0
        y = mt[idx]
        idx += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        yield y & mask


def test_mt19937_64_known_answer():
    # C++ [rand.predef]: the 10000th output of a default-constructed mt19937_64 (seed 5489).
    g = _mt19937_64(5489)
    for _ in range(9999):
        next(g)
    assert next(g) == 9981545732273789042


def test_rand_uniform_matches_libstdcxx_float_canonical(orc):
    # uniform_real_distribution<float>(lo, hi) over mt19937_64 in libstdc++: one 64-bit draw,
    # canonical = float(x) / 2^64 (float arithmetic, clamped below 1), value = canonical*(hi-lo)+lo.
    g = _mt19937_64(7)
    lo, hi = np.float32(-4.0), np.float32(4.0)
    expect = []
    for _ in range(64):
        c = np.float32(np.float32(next(g)) / np.float32(2.0**64))
        if c >= 1:
            c = np.nextafter(np.float32(1), np.float32(0))
        expect.append(np.float32(c * (hi - lo) + lo))
    got = orc.rand_uniform(64, 7, -4.0, 4.0)
    np.testing.assert_array_equal(got, np.array(expect, np.float32))


def test_splitmix_known_answers(orc):
    # Vigna's SplitMix64 with state 0 emits mix(gamma), mix(2 gamma): 0xe220a8397b1dcdaf,
    # 0x6e789e6aa1b965f4. The harness fill feeds mix(seed + i) and keeps the top 24 bits.
    gamma = 0x9E3779B97F4A7C15
    for mult, word in ((1, 0xE220A8397B1DCDAF), (2, 0x6E789E6AA1B965F4)):
        got = orc.splitmix_uniform(1, (mult * gamma) & ((1 << 64) - 1), 0.0, 1.0)
        assert got[0] == np.float32((word >> 40) / 16777216.0)


def test_normal_moments(orc):
    z = orc.normal(1 << 20, 3, 0.0, 1.0).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    assert abs(np.mean(z**4) - 3.0) < 0.05  # Gaussian kurtosis


def test_bf16_rounding_matches_torch(orc):
    x = np.concatenate([orc.normal(4096, 11, 0, 3), np.array(
        [0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf],
        np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.f32_to_bf16(x), want)
    np.testing.assert_array_equal(orc.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


def test_fp16_rounding_is_ieee_rne():
    # The 16-bit parity checks take numpy's fp32 -> fp16 conversion as RNE(ref). Pin it on the
    # cases that separate round-to-nearest-even from truncation or round-half-up: ties at
    # normal and subnormal spacing, the overflow threshold, and agreement with torch.
    x = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -11 + 2 ** -20, 2.0 ** -25,
                  3 * 2.0 ** -25, 65519.0, 65520.0, -65520.0, 2.0 ** -24], np.float32)
    want = np.array([1.0, 1 + 2 ** -9, 1 + 2 ** -10, 0.0, 2.0 ** -23, 65504.0, np.inf, -np.inf,
                     2.0 ** -24])
    with np.errstate(over="ignore"):  # 65520 -> inf is the case being pinned
        np.testing.assert_array_equal(x.astype(np.float16).astype(np.float64), want)
    y = np.random.default_rng(3).standard_normal(4096).astype(np.float32) * 100
    np.testing.assert_array_equal(y.astype(np.float16).view(np.uint16),
                                  torch.from_numpy(y).half().numpy().view(np.uint16))


def test_half_ulp_check_accepts_rounding_and_rejects_one_ulp(orc):
    from conftest import half_ulp_check

    ref = orc.normal(4096, 13)
    for fmt, bits in (("f16", ref.astype(np.float16).view(np.uint16)),
                      ("bf16", orc.f32_to_bf16(ref))):
        assert half_ulp_check(bits, ref, fmt)[0] == 0
        off = bits.copy()
        i = int(np.argmax(np.abs(ref)))
        off[i] += 2  # two ulps away from the rounding of the largest element
        with pytest.raises(AssertionError):
            half_ulp_check(off, ref, fmt, rel_tol=0.0)


# ---------------------------------------------------------------------------------------------
# GELU
# ---------------------------------------------------------------------------------------------


def test_gelu_forward_vs_torch_tanh_gelu(orc):
    x = orc.rand_uniform(1 << 16, 1, -4.0, 4.0)
    ref = F.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    assert max_rel(orc.gelu_forward(x), ref) < 2e-7
    # GELU(x) + GELU(-x) = x for the tanh form, GELU(0) = 0
    assert orc.gelu_forward(np.array([0.0], np.float32))[0] == 0.0


def test_gelu_backward_vs_autograd_and_harness_fd(orc):
    g = orc.rand_uniform(1 << 14, 2, -1.0, 1.0)
    x = orc.rand_uniform(1 << 14, 3, -4.0, 4.0)
    xt = torch.from_numpy(x).double().requires_grad_()
    F.gelu(xt, approximate="tanh").backward(torch.from_numpy(g).double())
    got = orc.gelu_backward(g, x)
    assert max_rel(got, xt.grad.numpy()) < 1e-6
    # the harness's own check: central difference of the forward, tolerance 5e-2
    assert np.max(np.abs(got - orc.gelu_backward_fd(g, x))) < 5e-2


def test_gelu_bf16_decodes_inputs(orc):
    x = orc.f32_to_bf16(orc.normal(4096, 5))
    xf = orc.bf16_to_f32(x)
    assert np.array_equal(orc.gelu_forward(x), orc.gelu_forward(xf))
    g = orc.f32_to_bf16(orc.normal(4096, 6))
    assert np.array_equal(orc.gelu_backward(g, x), orc.gelu_backward(orc.bf16_to_f32(g), xf))


# ---------------------------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(64, 768), (7, 33), (3, 5)])
def test_layer_norm_vs_torch(orc, rows, cols):
    x = orc.rand_uniform(rows * cols, 4).reshape(rows, cols)
    gamma = orc.rand_uniform(cols, 5, 0.5, 1.5)
    beta = orc.rand_uniform(cols, 6, -0.1, 0.1)
    dy = orc.rand_uniform(rows * cols, 7).reshape(rows, cols)
    y, mean, rstd = orc.layer_norm_forward(x, gamma, beta, 1e-5)
    xt = torch.from_numpy(x).double().requires_grad_()
    gt = torch.from_numpy(gamma).double().requires_grad_()
    bt = torch.from_numpy(beta).double().requires_grad_()
    yt = F.layer_norm(xt, (cols,), gt, bt, 1e-5)
    assert max_rel(y, yt.detach().numpy()) < 1e-6
    np.testing.assert_allclose(mean, x.astype(np.float64).mean(1), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(x.astype(np.float64).var(1) + 1e-5), rtol=1e-6)
    yt.backward(torch.from_numpy(dy).double())
    dx = orc.ln_backward_input(dy, x, mean, rstd, gamma)
    assert max_rel(dx, xt.grad.numpy()) < 1e-5
    dg, db = orc.ln_backward_gamma_beta(dy, x, mean, rstd)
    assert max_rel(dg, gt.grad.numpy()) < 1e-5
    assert max_rel(db, bt.grad.numpy()) < 1e-6
    # without gamma the input gradient is the gamma = 1 one
    dx1 = orc.ln_backward_input(dy, x, mean, rstd, None)
    assert np.array_equal(dx1, orc.ln_backward_input(dy, x, mean, rstd, np.ones(cols, np.float32)))


def test_layer_norm_single_column(orc):
    # one column: xhat = 0, so y = beta and the input gradient vanishes
    x = orc.rand_uniform(5, 8).reshape(5, 1)
    y, mean, rstd = orc.layer_norm_forward(x, np.array([2.0], np.float32), np.array([0.5], np.float32), 1e-5)
    np.testing.assert_array_equal(y, np.full((5, 1), 0.5, np.float32))
    np.testing.assert_array_equal(mean, x[:, 0])
    dx = orc.ln_backward_input(orc.rand_uniform(5, 9).reshape(5, 1), x, mean, rstd, None)
    assert np.max(np.abs(dx)) == 0.0


# ---------------------------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("vocab", [1, 3, 5, 257, 50257])
def test_sparse_ce_vs_torch(orc, vocab):
    rows = 8
    logits = orc.normal(rows * vocab, 12, 0.0, 2.0).reshape(rows, vocab)
    targets = (np.arange(rows) * 37 % vocab).astype(np.int32)
    targets[-1] = vocab - 1
    loss, mx, sm = orc.sparse_ce_forward(logits, targets)
    lt = torch.from_numpy(logits).double().requires_grad_()
    ref = F.cross_entropy(lt, torch.from_numpy(targets).long(), reduction="none")
    assert max_rel(loss, ref.detach().numpy()) < 1e-5
    np.testing.assert_array_equal(mx, logits.max(1))
    np.testing.assert_allclose(sm, np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True)).sum(1),
                               rtol=1e-6)
    ref.sum().backward()
    grad = orc.sparse_ce_backward(logits, targets, mx, sm, 1.0)
    assert max_rel(grad, lt.grad.numpy()) < 1e-6
    assert np.max(np.abs(grad.astype(np.float64).sum(1))) < 1e-5  # rows of softmax - onehot
    np.testing.assert_allclose(orc.sparse_ce_backward(logits, targets, mx, sm, 0.25), grad * 0.25,
                               rtol=1e-6, atol=1e-12)


# ---------------------------------------------------------------------------------------------
# AdamW
# ---------------------------------------------------------------------------------------------


def test_adamw_vs_torch_optim(orc):
    n = 10007
    p = orc.rand_uniform(n, 13)
    g = orc.rand_uniform(n, 14)
    m = orc.rand_uniform(n, 15, 0.0, 0.1)
    v = orc.rand_uniform(n, 16, 0.0, 0.1)
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    p2, m2, v2 = orc.adamw(p, g, m, v, lr, b1, b2, eps, wd, 1 - b1, 1 - b2)
    pt = torch.from_numpy(p).double().requires_grad_()
    opt = torch.optim.AdamW([pt], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    pt.grad = torch.from_numpy(g).double()
    opt.state[pt] = {"step": torch.tensor(0.0), "exp_avg": torch.from_numpy(m).double().clone(),
                     "exp_avg_sq": torch.from_numpy(v).double().clone()}
    opt.step()
    assert max_rel(m2, opt.state[pt]["exp_avg"].numpy()) < 1e-6
    assert max_rel(v2, opt.state[pt]["exp_avg_sq"].numpy()) < 1e-6
    assert max_rel(p2 - p, pt.detach().numpy() - p.astype(np.float64)) < 1e-4
    # zero gradient, zero decay, zero moments: parameters unchanged
    z = np.zeros(n, np.float32)
    p3, _, _ = orc.adamw(p, z, z, z, lr, b1, b2, eps, 0.0, 1 - b1, 1 - b2)
    assert np.array_equal(p3, p)


# ---------------------------------------------------------------------------------------------
# Reduce
# ---------------------------------------------------------------------------------------------


def test_reduce_selftest_input_exact(orc):
    rows, cols = 64, 100
    src = orc.reduce_selftest_input(rows * cols)
    np.testing.assert_array_equal(src[:18], (np.array([(i % 17) - 8 for i in range(18)]) * 0.25).astype(np.float32))
    inner = orc.reduce_inner(src, rows, cols)
    np.testing.assert_array_equal(inner, src.reshape(rows, cols).astype(np.float64).sum(1).astype(np.float32))
    outer = orc.reduce_outer(src, rows, rows, rows, rows, cols)
    np.testing.assert_array_equal(outer, src.reshape(cols, rows).astype(np.float64).sum(0).astype(np.float32))


def test_reduce_middle_axis(orc):
    a = orc.normal(3 * 50 * 7, 21).reshape(3, 50, 7)
    out = orc.reduce_outer(a, 21, 7, 350, 7, 50)
    np.testing.assert_allclose(out, a.astype(np.float64).sum(1).reshape(-1), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("causal", [False, True])
def test_attention_vs_torch_sdpa(orc, causal):
    B, H, T, D = 1, 2, 48, 64
    q, k, v, do = (orc.rand_uniform(B * H * T * D, s).reshape(B, H, T, D) for s in (101, 102, 103, 104))
    scale = 1.0 / np.sqrt(D)
    o, lse = orc.attn_forward(q, k, v, scale, causal)
    qt, kt, vt = (torch.from_numpy(a).double().requires_grad_() for a in (q, k, v))
    ot = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, scale=float(scale))
    s = (qt @ kt.transpose(-1, -2)) * float(scale)
    if causal:
        s = s.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf"))
    assert max_rel(o, ot.detach().numpy()) < 1e-5
    assert max_rel(lse, torch.logsumexp(s, -1).detach().numpy()) < 1e-5
    if causal:  # row 0 attends to key 0 only
        np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], rtol=1e-6)
    ot.backward(torch.from_numpy(do).double())
    D_, dq, dk, dv = orc.attn_backward(q, k, v, o, do, lse, scale, causal)
    np.testing.assert_allclose(D_, (do.astype(np.float64) * o).sum(-1), rtol=1e-5, atol=1e-6)
    # precompute-D forms fp32 products (kernels_test.cu:465), the backward double ones (:117)
    np.testing.assert_allclose(orc.attn_precompute_D(do, o), D_, rtol=1e-5, atol=1e-6)
    for got, ref in ((dq, qt.grad), (dk, kt.grad), (dv, vt.grad)):
        assert max_rel(got, ref.numpy()) < 1e-4


@pytest.mark.parametrize("causal", [False, True])
def test_attention_dropout_mask_vs_torch_sdpa(orc, causal):
    # The reference's dropout path multiplies each exp term by mask[(bh*T + i)*T + j] and
    # normalises by the post-dropout sum (fused_attn...:316-334). For a positive mask that is
    # softmax attention with the additive bias log(mask); for a 0/c mask it is attention over
    # the kept keys only, with LSE shifted by log(c). Both are checked against torch float64
    # SDPA with an attn_mask, on a mask that is not symmetric (a transposed index fails).
    B, H, T, D = 1, 2, 40, 64
    q, k, v = (orc.rand_uniform(B * H * T * D, s).reshape(B, H, T, D) for s in (111, 112, 113))
    scale = 1.0 / np.sqrt(D)
    qt, kt, vt = (torch.from_numpy(a).double() for a in (q, k, v))
    causal_inf = torch.zeros(T, T, dtype=torch.float64)
    if causal:
        causal_inf = causal_inf.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), -np.inf)
    s = (qt @ kt.transpose(-1, -2)) * float(scale) + causal_inf
    # positive mask: additive log bias
    pos = orc.rand_uniform(B * H * T * T, 114, 0.25, 2.0).reshape(B, H, T, T)
    o, lse = orc.attn_forward(q, k, v, scale, causal, mask=pos)
    bias = torch.from_numpy(np.log(pos.astype(np.float64))) + causal_inf
    ot = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=bias, scale=float(scale))
    assert max_rel(o, ot.numpy()) < 1e-5
    assert max_rel(lse, torch.logsumexp(s + torch.from_numpy(np.log(pos.astype(np.float64))),
                                        -1).numpy()) < 1e-5
    # 0 / c mask (c = 1 / (1 - p), p = 0.3): attention over the kept keys, LSE + log c
    c = 1.0 / 0.7
    keep = orc.rand_uniform(B * H * T * T, 115, 0.0, 1.0).reshape(B, H, T, T) >= 0.3
    keep[..., 0] = True  # every row keeps key 0, so no row is empty here
    mask = (keep * c).astype(np.float32)
    o, lse = orc.attn_forward(q, k, v, scale, causal, mask=mask)
    drop_inf = torch.from_numpy(np.where(keep, 0.0, -np.inf)) + causal_inf
    ot = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=drop_inf, scale=float(scale))
    assert max_rel(o, ot.numpy()) < 1e-5
    ref_lse = torch.logsumexp(s + drop_inf, -1).numpy() + np.log(np.float32(c))
    assert max_rel(lse, ref_lse) < 1e-5
    # an all-ones mask is no dropout at all
    o1, l1 = orc.attn_forward(q, k, v, scale, causal, mask=np.ones((B, H, T, T), np.float32))
    o0, l0 = orc.attn_forward(q, k, v, scale, causal)
    np.testing.assert_array_equal(o1, o0)
    np.testing.assert_array_equal(l1, l0)
    # a row with nothing kept: O = 0 and LSE = -inf (fused_attn...:333, 345)
    mask[0, 1, 5, :] = 0.0
    o, lse = orc.attn_forward(q, k, v, scale, causal, mask=mask)
    assert (o[0, 1, 5] == 0).all() and lse[0, 1, 5] == -np.inf


# ---------------------------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------------------------


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_vs_numpy(orc, ta, tb):
    M, N, K = 17, 9, 33
    A = orc.splitmix_uniform(M * K, 1).reshape((K, M) if ta else (M, K))
    B = orc.splitmix_uniform(K * N, 2).reshape((N, K) if tb else (K, N))
    C0 = orc.splitmix_uniform(M * N, 3).reshape(M, N)
    bias = orc.splitmix_uniform(N, 4)
    got = orc.sgemm(ta, tb, A, B, alpha=1.5, beta=0.5, C0=C0, bias=bias)
    a = A.T if ta else A
    b = B.T if tb else B
    ref = 1.5 * (a.astype(np.float64) @ b) + 0.5 * C0 + bias
    assert max_rel(got, ref) < 1e-5


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_vs_numpy(orc, ta, tb):
    M, N, K = 24, 40, 56
    A = orc.f32_to_bf16(orc.splitmix_uniform(M * K, 5)).reshape((K, M) if ta else (M, K))
    B = orc.f32_to_bf16(orc.splitmix_uniform(K * N, 6)).reshape((N, K) if tb else (K, N))
    C0 = orc.f32_to_bf16(orc.splitmix_uniform(M * N, 7)).reshape(M, N)
    got = orc.bgemm(ta, tb, A, B, alpha=1.0, beta=0.5, C0=C0)
    a = orc.bf16_to_f32(A).astype(np.float64)
    b = orc.bf16_to_f32(B).astype(np.float64)
    ref = (a.T if ta else a) @ (b.T if tb else b) + 0.5 * orc.bf16_to_f32(C0)
    assert max_rel(got, ref) < 1e-5


@pytest.mark.parametrize("numel", ["N", "M", "1", "MN"])
def test_bgemm_bias_forms_vs_numpy(orc, numel):
    # addmm / split-K bias init forms (bgemm_addmm…:246-300, bgemm_core_template.cu:277-283)
    M, N, K = 24, 40, 56
    A = orc.f32_to_bf16(orc.splitmix_uniform(M * K, 15)).reshape(M, K)
    B = orc.f32_to_bf16(orc.splitmix_uniform(K * N, 16)).reshape(K, N)
    size = {"N": N, "M": M, "1": 1, "MN": M * N}[numel]
    bias = orc.f32_to_bf16(orc.splitmix_uniform(size, 17))
    got = orc.bgemm(0, 0, A, B, alpha=1.5, beta=0.5, bias=bias)
    b64 = orc.bf16_to_f32(bias).astype(np.float64)
    bfull = {"N": lambda: b64[None, :], "M": lambda: b64[:, None],
             "1": lambda: b64.reshape(1, 1), "MN": lambda: b64.reshape(M, N)}[numel]()
    ref = 1.5 * (orc.bf16_to_f32(A).astype(np.float64) @ orc.bf16_to_f32(B)) + 0.5 * bfull
    assert max_rel(got, np.broadcast_to(ref, (M, N))) < 1e-5
