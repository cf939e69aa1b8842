"""GPU parity of fused attention (forward, precompute-D and backward) against the oracle's
restatement of the harness's CPU FlashAttention reference (kernels_test.cu:68-139).
Tolerance: BASELINE.json's max-rel 2e-3 (max|err| / max|ref|) for O, LSE, dQ, dK, dV."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def _qkv(orc, B, H, T, D, seeds, normal=False):
    n = B * H * T * D
    if normal:  # Q, K, V ~ N(0, 1)
        return [orc.normal(n, s).reshape(B, H, T, D) for s in seeds]
    return [orc.rand_uniform(n, s).reshape(B, H, T, D) for s in seeds]  # kernels_test.cu:499


@pytest.mark.parametrize("causal", [False, True])
def test_attn_forward_harness_shape(hk, orc, causal):
    # kernels_test.cu:491-538: B=2, H=6, T=256, d=64, seeds 101..103, scale 1/sqrt(d)
    B, H, T, D = 2, 6, 256, 64
    say("attn fwd harness", causal)
    q, k, v = _qkv(orc, B, H, T, D, (101, 102, 103))
    scale = 1.0 / np.sqrt(np.float32(D))
    o, lse = hk.fused_attn_forward(*(torch.from_numpy(a).to(DEV) for a in (q, k, v)), causal,
                                   float(scale))
    torch.cuda.synchronize()
    ro, rl = orc.attn_forward(q, k, v, scale, causal)
    assert max_rel(o.cpu().numpy(), ro) <= 2e-3
    assert max_rel(lse.cpu().numpy(), rl) <= 2e-3
    print(f"O rel {max_rel(o.cpu().numpy(), ro):.2e} LSE rel {max_rel(lse.cpu().numpy(), rl):.2e}")


@pytest.mark.parametrize("T", [1, 33, 64, 100, 129, 300])
@pytest.mark.parametrize("causal", [False, True])
def test_attn_forward_ragged_T(hk, orc, T, causal):
    B, H, D = 1, 3, 64
    say("attn fwd ragged", T, causal)
    q, k, v = _qkv(orc, B, H, T, D, (11, 12, 13), normal=True)
    o, lse = hk.fused_attn_forward(*(torch.from_numpy(a).to(DEV) for a in (q, k, v)), causal)
    torch.cuda.synchronize()
    ro, rl = orc.attn_forward(q, k, v, 0.125, causal)
    assert max_rel(o.cpu().numpy(), ro) <= 2e-3
    assert max_rel(lse.cpu().numpy(), rl) <= 2e-3


def test_attn_forward_strided_bthd_layout(hk, orc):
    # [B, T, H, d] storage viewed as [B, H, T, d] (non-contiguous head/row strides)
    B, H, T, D = 2, 4, 192, 64
    say("attn fwd strided")
    q, k, v = _qkv(orc, B, H, T, D, (21, 22, 23), normal=True)
    dev = [torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(DEV).transpose(1, 2)
           for a in (q, k, v)]
    o = torch.empty(B, T, H, D, device=DEV).transpose(1, 2)
    o, lse = hk.fused_attn_forward(*dev, True, o=o)
    torch.cuda.synchronize()
    ro, rl = orc.attn_forward(q, k, v, 0.125, True)
    assert max_rel(o.cpu().numpy(), ro) <= 2e-3 and max_rel(lse.cpu().numpy(), rl) <= 2e-3


@pytest.mark.parametrize("causal", [True, False])
def test_attn_forward_baseline_shape_all_heads(hk, orc, causal):
    # B=8, H=12, T=1024, d=64, Q, K, V ~ N(0, 1). Every one of the 96
    # (batch, head) pairs is checked in full against the oracle, and each head on its own (a
    # head-wise bound, so one wrong head cannot hide under the others' magnitude).
    B, H, T, D = 8, 12, 1024, 64
    say("attn fwd baseline all heads", causal)
    q, k, v = _qkv(orc, B, H, T, D, (31, 32, 33), normal=True)
    o, lse = hk.fused_attn_forward(*(torch.from_numpy(a).to(DEV) for a in (q, k, v)), causal)
    torch.cuda.synchronize()
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    ro, rl = orc.attn_forward(q, k, v, 0.125, causal)
    worst = max((max_rel(o[b, h], ro[b, h]), max_rel(lse[b, h], rl[b, h]), (b, h))
                for b in range(B) for h in range(H))
    print(f"worst head {worst[2]}: O rel {worst[0]:.2e} LSE rel {worst[1]:.2e}")
    for b in range(B):
        for h in range(H):
            assert max_rel(o[b, h], ro[b, h]) <= 2e-3, (b, h)
            assert max_rel(lse[b, h], rl[b, h]) <= 2e-3, (b, h)
    if causal:  # invariant: row 0 attends to key 0 only -> O[.,.,0] = V[.,.,0]
        np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], rtol=1e-5, atol=1e-6)


def _bwd_check(hk, orc, q, k, v, do, causal, scale, from_gpu_forward=False):
    ro, rl = orc.attn_forward(q, k, v, scale, causal)
    rD, rdq, rdk, rdv = orc.attn_backward(q, k, v, ro, do, rl, scale, causal)
    Q, K, V, dO = (torch.from_numpy(a).to(DEV) for a in (q, k, v, do))
    if from_gpu_forward:  # the whole GPU chain: forward -> precompute D -> backward
        O, L = hk.fused_attn_forward(Q, K, V, causal, scale)
        Dt = hk.attn_bwd_precompute_D(dO, O)
    else:  # the harness feeds the CPU reference's O, LSE and D (kernels_test.cu:559-561)
        L, Dt = torch.from_numpy(rl).to(DEV), torch.from_numpy(rD).to(DEV)
    dq, dk, dv = hk.attn_backward(Q, K, V, dO, L, Dt, causal, scale)
    torch.cuda.synchronize()
    # With a single key (T = 1) dS = P (dP - D) is an exact cancellation: the reference's dQ and
    # dK are exactly zero and the GPU's are fp32 rounding residue; there the bound is taken
    # relative to the size of the cancelling terms, |dO| |V|.
    term = float(np.abs(do).max() * np.abs(v).max())
    rels = [max_rel(g.cpu().numpy(), r) if np.abs(r).max() > 0
            else float(np.abs(g.cpu().numpy()).max()) / term
            for g, r in ((dq, rdq), (dk, rdk), (dv, rdv))]
    print(f"dQ {rels[0]:.2e} dK {rels[1]:.2e} dV {rels[2]:.2e}")
    assert max(rels) <= 2e-3, rels
    return dq, rdq


@pytest.mark.parametrize("causal", [False, True])
def test_attn_backward_harness_shape(hk, orc, causal):
    # kernels_test.cu:540-594: B=2, H=6, T=256, d=64, dO seed 104
    B, H, T, D = 2, 6, 256, 64
    say("attn bwd harness", causal)
    q, k, v = _qkv(orc, B, H, T, D, (101, 102, 103))
    do = orc.rand_uniform(B * H * T * D, 104).reshape(B, H, T, D)
    _bwd_check(hk, orc, q, k, v, do, causal, float(1.0 / np.sqrt(np.float32(D))))


@pytest.mark.parametrize("causal", [False, True])
def test_attn_backward_gpu_chain(hk, orc, causal):
    B, H, T, D = 1, 4, 384, 64
    say("attn bwd chain", causal)
    q, k, v, do = _qkv(orc, B, H, T, D, (41, 42, 43, 44), normal=True)
    _bwd_check(hk, orc, q, k, v, do, causal, 0.125, from_gpu_forward=True)


# 63 / 65 / 127 / 191 / 257: query tiles that end inside a 16-query dQ block or a 4-row group
# of it (rows past T add 0 to row T - 1)
@pytest.mark.parametrize("T", [1, 33, 63, 65, 100, 127, 129, 191, 257, 300])
@pytest.mark.parametrize("causal", [False, True])
def test_attn_backward_ragged_T(hk, orc, T, causal):
    say("attn bwd ragged", T, causal)
    q, k, v, do = _qkv(orc, 1, 2, T, 64, (51, 52, 53, 54), normal=True)
    _bwd_check(hk, orc, q, k, v, do, causal, 0.125)


def test_attn_backward_dq_accumulates(hk, orc):
    # dQ is added into (the reference zeroes it before the launch and adds atomically)
    say("attn bwd dq accumulate")
    q, k, v, do = _qkv(orc, 1, 2, 128, 64, (61, 62, 63, 64), normal=True)
    ro, rl = orc.attn_forward(q, k, v, 0.125, True)
    rD = orc.attn_precompute_D(do, ro)
    Q, K, V, dO = (torch.from_numpy(a).to(DEV) for a in (q, k, v, do))
    L, Dt = torch.from_numpy(rl).to(DEV), torch.from_numpy(rD).to(DEV)
    dq1, _, _ = hk.attn_backward(Q, K, V, dO, L, Dt, True, 0.125)
    first = dq1.clone()
    hk.attn_backward(Q, K, V, dO, L, Dt, True, 0.125, dq=dq1)
    torch.cuda.synchronize()
    assert max_rel(dq1.cpu().numpy(), 2 * first.cpu().numpy().astype(np.float64)) <= 1e-6


@pytest.mark.parametrize("causal", [True, False])
def test_attn_backward_baseline_shape_all_heads(hk, orc, causal):
    # B=8, H=12, T=1024, d=64, dO ~ N(0, 1), forward's O / LSE reused (the
    # GPU chain forward -> precompute D -> backward). Every one of the 96 (batch, head) pairs
    # is checked in full against the oracle, head by head.
    B, H, T, D = 8, 12, 1024, 64
    say("attn bwd baseline all heads", causal)
    q, k, v, do = _qkv(orc, B, H, T, D, (71, 72, 73, 74), normal=True)
    Q, K, V, dO = (torch.from_numpy(a).to(DEV) for a in (q, k, v, do))
    O, L = hk.fused_attn_forward(Q, K, V, causal)
    Dt = hk.attn_bwd_precompute_D(dO, O)
    dq, dk, dv = hk.attn_backward(Q, K, V, dO, L, Dt, causal)
    torch.cuda.synchronize()
    dq, dk, dv = dq.cpu().numpy(), dk.cpu().numpy(), dv.cpu().numpy()
    ro, rl = orc.attn_forward(q, k, v, 0.125, causal)
    _, rdq, rdk, rdv = orc.attn_backward(q, k, v, ro, do, rl, 0.125, causal)
    worst = [0.0, 0.0, 0.0]
    for b in range(B):
        for h in range(H):
            rels = [max_rel(g[b, h], r[b, h]) for g, r in ((dq, rdq), (dk, rdk), (dv, rdv))]
            worst = [max(w, x) for w, x in zip(worst, rels)]
            assert max(rels) <= 2e-3, ((b, h), rels)
    print(f"worst over 96 heads: dQ {worst[0]:.2e} dK {worst[1]:.2e} dV {worst[2]:.2e}")


def test_attn_precompute_D(hk, orc):
    # kernels_test.cu:459-481 at the GPT shape: B=16, heads=12, T=1024, d=64, seeds 17/18
    B, H, T, D = 16, 12, 1024, 64
    say("precompute D")
    do = orc.rand_uniform(B * H * T * D, 17).reshape(B, H, T, D)
    o = orc.rand_uniform(B * H * T * D, 18).reshape(B, H, T, D)
    Dt = hk.attn_bwd_precompute_D(torch.from_numpy(do).to(DEV), torch.from_numpy(o).to(DEV))
    torch.cuda.synchronize()
    ref = orc.attn_precompute_D(do, o)
    assert max_rel(Dt.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("hd", [16, 32, 48, 64, 80, 96, 128, 160, 192, 256, 20, 7])
def test_attn_precompute_D_head_dims(hk, orc, hd):
    # Every HeadDim the reference instantiates (precompute_D...:93-102), plus two it does not
    # (20: vector path with a partial last 64-float span; 7: scalar path), at a ragged T.
    B, H, T = 2, 3, 77
    say("precompute D head_dim", hd)
    do = orc.rand_uniform(B * H * T * hd, 19).reshape(B, H, T, hd)
    o = orc.rand_uniform(B * H * T * hd, 20).reshape(B, H, T, hd)
    Dt = hk.attn_bwd_precompute_D(torch.from_numpy(do).to(DEV), torch.from_numpy(o).to(DEV))
    torch.cuda.synchronize()
    assert max_rel(Dt.cpu().numpy(), orc.attn_precompute_D(do, o)) <= 1e-5


def test_attn_precompute_D_strided_rows(hk, orc):
    # Rows padded to 65 floats (a stride that is not a multiple of 4) and the heads of a packed
    # [B, T, H, d] tensor: the reference takes any strides, so must this entry point.
    B, H, T, hd = 2, 4, 50, 64
    say("precompute D strided")
    do = orc.rand_uniform(B * H * T * hd, 21).reshape(B, H, T, hd)
    o = orc.rand_uniform(B * H * T * hd, 22).reshape(B, H, T, hd)
    ref = orc.attn_precompute_D(do, o)
    pad = torch.zeros(B, H, T, hd + 1, device=DEV)
    pad[..., :hd] = torch.from_numpy(do).to(DEV)
    packed = torch.from_numpy(np.ascontiguousarray(o.transpose(0, 2, 1, 3))).to(DEV)
    Dt = hk.attn_bwd_precompute_D(pad[..., :hd], packed.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    assert max_rel(Dt.cpu().numpy(), ref) <= 1e-5



def _mask(orc, B, H, T, seed, p=0.3):
    """A 0 / (1 / (1 - p)) dropout mask, fp32 [B, H, T, T], every row keeping key 0."""
    keep = orc.rand_uniform(B * H * T * T, seed, 0.0, 1.0).reshape(B, H, T, T) >= p
    keep[..., 0] = True
    return (keep / np.float32(1.0 - p)).astype(np.float32)


@pytest.mark.parametrize("T", [64, 200, 201])  # 201: rows not 16-byte aligned (scalar loads)
@pytest.mark.parametrize("causal", [False, True])
def test_attn_forward_dropout_mask(hk, orc, T, causal):
    # the reference's dropout path (fused_attn...:316-334): masked exp terms, post-dropout sum
    B, H, D = 2, 3, 64
    say("attn fwd dropout", T, causal)
    q, k, v = _qkv(orc, B, H, T, D, (31, 32, 33), normal=True)
    mask = _mask(orc, B, H, T, 34)
    o, lse = hk.fused_attn_forward(*(torch.from_numpy(a).to(DEV) for a in (q, k, v)), causal,
                                   dropout_p=0.3, dropout_mask=torch.from_numpy(mask).to(DEV))
    torch.cuda.synchronize()
    ro, rl = orc.attn_forward(q, k, v, 0.125, causal, mask=mask)
    assert max_rel(o.cpu().numpy(), ro) <= 2e-3
    assert max_rel(lse.cpu().numpy(), rl) <= 2e-3
    # not the pre-dropout normalisation: that result differs from the reference's here
    r0, _ = orc.attn_forward(q, k, v, 0.125, causal)
    assert max_rel(o.cpu().numpy(), r0) > 2e-2


def test_attn_forward_dropout_off_cases(hk, orc):
    # dropout_p > 0 without a mask, or a mask with dropout_p == 0: no dropout (fused_attn...:321)
    B, H, T, D = 1, 2, 96, 64
    say("attn fwd dropout off")
    q, k, v = (torch.from_numpy(a).to(DEV) for a in _qkv(orc, B, H, T, D, (41, 42, 43)))
    mask = torch.from_numpy(_mask(orc, B, H, T, 44)).to(DEV)
    ref_o, ref_l = hk.fused_attn_forward(q, k, v, True)
    for kw in ({"dropout_p": 0.5}, {"dropout_p": 0.0, "dropout_mask": mask}):
        o, lse = hk.fused_attn_forward(q, k, v, True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(o, ref_o) and torch.equal(lse, ref_l)


def test_attn_forward_dropout_row_with_nothing_kept(hk, orc):
    B, H, T, D = 1, 1, 70, 64
    say("attn fwd dropout empty row")
    q, k, v = _qkv(orc, B, H, T, D, (51, 52, 53))
    mask = _mask(orc, B, H, T, 54)
    mask[0, 0, 9, :] = 0.0
    o, lse = hk.fused_attn_forward(*(torch.from_numpy(a).to(DEV) for a in (q, k, v)), False,
                                   dropout_p=0.3, dropout_mask=torch.from_numpy(mask).to(DEV))
    torch.cuda.synchronize()
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    assert (o[0, 0, 9] == 0).all() and lse[0, 0, 9] == -np.inf
    ro, rl = orc.attn_forward(q, k, v, 0.125, False, mask=mask)
    keep = np.ones(T, bool)
    keep[9] = False
    assert max_rel(o[0, 0, keep], ro[0, 0, keep]) <= 2e-3
    assert max_rel(lse[0, 0, keep], rl[0, 0, keep]) <= 2e-3


@pytest.mark.parametrize("causal", [False, True])
def test_attn_forward_dropout_baseline_shape_sampled_heads(hk, orc, causal):
    # BASELINE configs[2] shape with a p = 0.1 mask; two (batch, head) pairs checked in full
    B, H, T, D = 8, 12, 1024, 64
    say("attn fwd dropout baseline", causal)
    g = torch.Generator(device=DEV)
    g.manual_seed(7)
    q, k, v = (torch.randn(B, H, T, D, generator=g, device=DEV) for _ in range(3))
    mask = (torch.rand(B, H, T, T, generator=g, device=DEV) >= 0.1).float() / 0.9
    o, lse = hk.fused_attn_forward(q, k, v, causal, dropout_p=0.1, dropout_mask=mask)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (7, 11)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ro, rl = orc.attn_forward(*(t[sl].cpu().numpy() for t in (q, k, v)), 0.125, causal,
                                  mask=mask[sl].cpu().numpy())
        assert max_rel(o[sl].cpu().numpy(), ro) <= 2e-3
        assert max_rel(lse[sl].cpu().numpy(), rl) <= 2e-3


@pytest.mark.parametrize("T", [100, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_attn_backward_strided_bthd_layout(hk, orc, T, causal):
    # [B, T, H, d] storage viewed as [B, H, T, d] for Q, K, V, dO and the dQ / dK / dV outputs,
    # and LSE / D inside NaN-padded [B, H + 1, T + 5] buffers: every batch, head and row stride
    # that the Q / dO pre-pass and the kernel read differs from the contiguous one.
    B, H, D = 2, 3, 64
    say("attn bwd strided", T, causal)
    q, k, v, do = _qkv(orc, B, H, T, D, (81, 82, 83, 84), normal=True)
    ro, rl = orc.attn_forward(q, k, v, 0.125, causal)
    rD, rdq, rdk, rdv = orc.attn_backward(q, k, v, ro, do, rl, 0.125, causal)

    def bthd(a):
        return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(DEV).transpose(
            1, 2)

    def padded(a):
        buf = torch.full((B, H + 1, T + 5), float("nan"), device=DEV)
        buf[:, 1:, 2:2 + T] = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
        return buf[:, 1:, 2:2 + T]

    Q, K, V, dO = (bthd(a) for a in (q, k, v, do))
    L, Dt = padded(rl), padded(rD)
    assert not Q.is_contiguous() and not L.is_contiguous()
    dq, dk, dv = (torch.zeros(B, T, H, D, device=DEV).transpose(1, 2) for _ in range(3))
    hk.attn_backward(Q, K, V, dO, L, Dt, causal, 0.125, dq=dq, dk=dk, dv=dv)
    torch.cuda.synchronize()
    rels = [max_rel(g.cpu().numpy(), r) for g, r in ((dq, rdq), (dk, rdk), (dv, rdv))]
    print(f"dQ {rels[0]:.2e} dK {rels[1]:.2e} dV {rels[2]:.2e}")
    assert max(rels) <= 2e-3, rels
