"""Seeded random-shape GPU parity sweep: BF16 BGEMM (every layout, batches, alpha / beta, and NT
products on whole 256 x 160 tiles), FP32 SGEMM (every layout, split-K, bias forms) and attention
forward + backward (ragged T, causal and not, strided [B, T, nh, d] views), each against the
oracle at the same tolerances as the fixed-shape tests (1e-2 for bf16 outputs, 2e-3 for fp32
ones, max|err| / max|ref|).

The shapes are drawn once, from a fixed seed, when the module is collected, so every run sees
the same cases and a failing case is named by its parameters. The draws mix 8-aligned extents
(the MFMA tile paths, with partial tiles) and ragged ones (the fallback kernels)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_rel
from test_gpu_gemm import SG_LAYOUT, _check, _operands, _sg_call, _sg_operands, bits, say, \
    to_dev_bf16, to_host_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _extent(rng, lo, hi, aligned):
    x = int(rng.integers(lo, hi + 1))
    return max(aligned, x - x % aligned) if aligned > 1 else x


def _bgemm_cases(n=24, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        al = 8 if i % 4 else 1  # one case in four takes ragged extents
        M, N, K = (_extent(rng, 1, 700, al), _extent(rng, 1, 700, al), _extent(rng, 1, 600, al))
        ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        batch = int(rng.integers(1, 3))
        alpha = float(rng.choice([1.0, 0.5, -1.25, 2.0]))
        beta = float(rng.choice([0.0, 0.5, 1.0, -0.75]))
        cases.append((M, N, K, ta, tb, batch, alpha, beta, 3000 + 10 * i))
    return cases


@pytest.mark.parametrize("M,N,K,ta,tb,batch,alpha,beta,seed", _bgemm_cases())
def test_bgemm_random_shapes(hk, orc, M, N, K, ta, tb, batch, alpha, beta, seed):
    say("bgemm random", M, N, K, ta, tb, batch, alpha, beta)
    ops = [_operands(orc, M, N, K, ta, tb, seed + b) for b in range(batch)]
    dA = to_dev_bf16(np.stack([o[0] for o in ops]))
    dB = to_dev_bf16(np.stack([o[1] for o in ops]))
    dC = to_dev_bf16(np.stack([o[2] for o in ops]))
    lda, ldb = ops[0][0].shape[1], ops[0][1].shape[1]
    st = hk.lib().hk_bgemm(ta, tb, M, N, K, bits(alpha), dA.data_ptr(), lda, M * K,
                           dB.data_ptr(), ldb, K * N, bits(beta), dC.data_ptr(), N, M * N, batch,
                           torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    for b, (A, B, C0) in enumerate(ops):
        _check(orc, out[b], A, B, C0, ta, tb, alpha, beta)


def _w160_cases(n=10, seed=20261205):
    # NT products of whole 256 x 160 tiles that fit one round (the 16 x 16 x 32 MFMA kernel)
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        M, N = 256 * int(rng.integers(1, 9)), 160 * int(rng.integers(1, 9))
        K, batch = 64 * int(rng.integers(1, 12)), int(rng.integers(1, 4))
        if (M // 256) * (N // 160) * batch > 256 or -(-M // 256) * -(-N // 256) * batch >= 256:
            continue
        alpha = float(rng.choice([1.0, 0.5, -1.25, 2.0]))
        beta = float(rng.choice([0.0, 0.5, 1.0, -0.75]))
        cases.append((M, N, K, batch, alpha, beta, 3500 + 10 * len(cases)))
    return cases


@pytest.mark.parametrize("M,N,K,batch,alpha,beta,seed", _w160_cases())
def test_bgemm_random_256x160_tiles(hk, orc, M, N, K, batch, alpha, beta, seed):
    lib = hk.lib()
    assert lib.hk_bgemm_tile_cols(0, 1, M, N, K, batch, 0) == 160
    say("bgemm random 256x160", M, N, K, batch, alpha, beta)
    ops = [_operands(orc, M, N, K, 0, 1, seed + b) for b in range(batch)]
    dA = to_dev_bf16(np.stack([o[0] for o in ops]))
    dB = to_dev_bf16(np.stack([o[1] for o in ops]))
    dC = to_dev_bf16(np.stack([o[2] for o in ops]))
    st = lib.hk_bgemm(0, 1, M, N, K, bits(alpha), dA.data_ptr(), K, M * K, dB.data_ptr(), K,
                      N * K, bits(beta), dC.data_ptr(), N, M * N, batch,
                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    for b, (A, B, C0) in enumerate(ops):
        _check(orc, out[b], A, B, C0, 0, 1, alpha, beta)


def _sgemm_cases(n=18, seed=20261203):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        al = (8, 4, 1)[i % 3]  # bf16x3 tiles, fp32 MFMA tiles, k-order fallback
        M, N, K = (_extent(rng, 1, 600, al), _extent(rng, 1, 600, al), _extent(rng, 1, 520, al))
        lay = str(rng.choice(list(SG_LAYOUT)))
        split_k = int(rng.choice([0, 1, 2, 3, 5]))
        bias = str(rng.choice(["none", "col", "scalar"]))
        cases.append((M, N, K, lay, split_k, bias, 4000 + 10 * i))
    return cases


@pytest.mark.parametrize("M,N,K,lay,split_k,bias,seed", _sgemm_cases())
def test_sgemm_random_shapes(hk, orc, M, N, K, lay, split_k, bias, seed):
    enum, ta, tb = SG_LAYOUT[lay]
    say("sgemm random", M, N, K, lay, split_k, bias)
    A, B, C0, bvec = _sg_operands(orc, M, N, K, ta, tb, seed)
    if bias == "scalar":
        bvec, stride = bvec[:1].copy(), 1
    else:
        stride = N
    dbias = None if bias == "none" else torch.from_numpy(bvec).to(DEV)
    out = _sg_call(hk, "hk_sgemm", enum, torch.from_numpy(A).to(DEV),
                   torch.from_numpy(B).to(DEV), torch.from_numpy(C0).to(DEV), M, N, K, -0.75,
                   0.5, bias=dbias, bias_stride=0 if bias == "none" else stride, split_k=split_k)
    ref = orc.sgemm(ta, tb, A, B, alpha=-0.75, beta=0.5, C0=C0,
                    bias=None if bias == "none" else (np.full(N, bvec[0], np.float32)
                                                      if bias == "scalar" else bvec))
    assert max_rel(out, ref) <= 2e-3


def _attn_cases(n=10, seed=20261204):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
        T = int(rng.integers(1, 400))
        causal = bool(i % 2)
        bthd = bool(rng.integers(0, 2))  # [B, T, nh, d] storage viewed as [B, nh, T, d]
        scale = float(rng.choice([0.125, 0.1, 0.2]))
        cases.append((B, H, T, causal, bthd, scale, 5000 + 10 * i))
    return cases


def _dev_view(a, bthd):
    if not bthd:
        return torch.from_numpy(a).to(DEV)
    return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(DEV).transpose(1, 2)


@pytest.mark.parametrize("B,H,T,causal,bthd,scale,seed", _attn_cases())
def test_attention_random_shapes(hk, orc, B, H, T, causal, bthd, scale, seed):
    # The GPU chain forward -> precompute D -> backward, each output against the oracle
    D = 64
    say("attention random", B, H, T, causal, bthd, scale)
    q, k, v, do = (orc.normal(B * H * T * D, seed + j).reshape(B, H, T, D) for j in range(4))
    Q, K, V, dO = (_dev_view(a, bthd) for a in (q, k, v, do))
    o = torch.empty(B, T, H, D, device=DEV).transpose(1, 2) if bthd else None
    O, L = hk.fused_attn_forward(Q, K, V, causal, scale, o=o)
    Dt = hk.attn_bwd_precompute_D(dO, O)
    if bthd:
        dq = torch.zeros(B, T, H, D, device=DEV).transpose(1, 2)
        dk = torch.empty(B, T, H, D, device=DEV).transpose(1, 2)
        dv = torch.empty(B, T, H, D, device=DEV).transpose(1, 2)
    else:
        dq = dk = dv = None
    dq, dk, dv = hk.attn_backward(Q, K, V, dO, L, Dt, causal, scale, dq=dq, dk=dk, dv=dv)
    torch.cuda.synchronize()
    ro, rl = orc.attn_forward(q, k, v, scale, causal)
    rD, rdq, rdk, rdv = orc.attn_backward(q, k, v, ro, do, rl, scale, causal)
    assert max_rel(O.cpu().numpy(), ro) <= 2e-3
    assert max_rel(L.cpu().numpy(), rl) <= 2e-3
    assert max_rel(Dt.cpu().numpy(), rD) <= 2e-3
    # With one key (T = 1) dS = P (dP - D) cancels exactly: there dQ and dK are fp32 rounding
    # residue, bounded relative to the size of the cancelling terms |dO| |V|
    term = float(np.abs(do).max() * np.abs(v).max())
    rels = [max_rel(g.cpu().numpy(), r) if np.abs(r).max() > 0
            else float(np.abs(g.cpu().numpy()).max()) / term
            for g, r in ((dq, rdq), (dk, rdk), (dv, rdv))]
    print(f"dQ {rels[0]:.2e} dK {rels[1]:.2e} dV {rels[2]:.2e}")
    assert max(rels) <= 2e-3, rels
