"""GPU parity of the batched BF16 GEMV entry points (blas/bf16/bgemv_sm89_kernel.cu) and of
hk_bgemm's M == 1 / N == 1 products, against the oracle's fp32-accumulated GEMM on the same
bf16 operands. Tolerance: BASELINE.json's bf16 GEMM bar, 1e-2 relative to max|ref|.

Operands live in NaN-filled device buffers with padded rows, batch gaps and element offsets,
so a read outside the operands or a write outside C shows up as NaN or as a changed pad."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAN_BITS = 0x7FC0
TOL = 1e-2


def say(*a):
    print("[case]", *a, flush=True)


def bits(x: float) -> int:
    return int(torch.tensor([x], dtype=torch.bfloat16).view(torch.int16).item()) & 0xFFFF


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV)


def _host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


# kind -> (matrix is [K, R] (rows along the outputs) or [R, K], the x stride is lda)
KINDS = {"nn_row": "KR", "nt_row": "RK", "tn_row": "KR", "nn_col": "RK"}


def _reference(orc, kind, x, m, c0, alpha, beta):
    K = x.size
    if kind == "nn_row":
        r = orc.bgemm(0, 0, x.reshape(1, K), m, alpha, beta, c0.reshape(1, -1))
    elif kind == "nt_row":
        r = orc.bgemm(0, 1, x.reshape(1, K), m, alpha, beta, c0.reshape(1, -1))
    elif kind == "tn_row":
        r = orc.bgemm(1, 0, x.reshape(K, 1), m, alpha, beta, c0.reshape(1, -1))
    else:
        r = orc.bgemm(0, 0, m, x.reshape(K, 1), alpha, beta, c0.reshape(-1, 1))
    return r.reshape(-1)


def _gemv_case(hk, orc, kind, R, K, ld=None, inc=1, batch=1, alpha=1.0, beta=0.5, off=0,
               seed=1, c_nan=False):
    say("bgemv", kind, f"R={R} K={K} ld={ld} inc={inc} batch={batch} off={off} beta={beta}")
    lib = hk.lib()
    rows, cols = (K, R) if KINDS[kind] == "KR" else (R, K)
    ld = cols if ld is None else ld
    sm, sx, sc = rows * ld + 8, K * inc + 8, R + 8
    mflat = np.full(off + batch * sm, NAN_BITS, np.uint16)
    xflat = np.full(off + batch * sx, NAN_BITS, np.uint16)
    cflat = np.full(off + batch * sc, NAN_BITS, np.uint16)
    refs = []
    for b in range(batch):
        x = orc.f32_to_bf16(orc.splitmix_uniform(K, seed + 10 * b + 1))
        m = orc.f32_to_bf16(orc.splitmix_uniform(rows * cols, seed + 10 * b + 2)).reshape(rows,
                                                                                           cols)
        c0 = orc.f32_to_bf16(orc.splitmix_uniform(R, seed + 10 * b + 3))
        mv = mflat[off + b * sm: off + b * sm + rows * ld].reshape(rows, ld)
        mv[:, :cols] = m
        xflat[off + b * sx: off + b * sx + K * inc: inc] = x
        if not c_nan:
            cflat[off + b * sc: off + b * sc + R] = c0
        refs.append(_reference(orc, kind, x, m, c0, alpha, 0.0 if c_nan else beta))
    dm, dx, dc = _dev(mflat), _dev(xflat), _dev(cflat)
    pm = dm.data_ptr() + 2 * off
    px = dx.data_ptr() + 2 * off
    pc = dc.data_ptr() + 2 * off
    s = torch.cuda.current_stream().cuda_stream
    a, bt = bits(alpha), bits(beta)
    if kind == "nn_row":
        st = lib.hk_bgemv_nn_row(R, K, a, px, pm, ld, bt, pc, batch, sx, sm, sc, s)
    elif kind == "nt_row":
        st = lib.hk_bgemv_nt_row(R, K, a, px, pm, ld, bt, pc, batch, sx, sm, sc, s)
    elif kind == "tn_row":
        st = lib.hk_bgemv_tn_row(R, K, a, px, inc, pm, ld, bt, pc, batch, sx, sm, sc, s)
    else:
        st = lib.hk_bgemv_nn_col(R, K, a, pm, ld, px, bt, pc, batch, sm, sx, sc, s)
    assert st == 0
    out = _host(dc)
    rels = []
    for b in range(batch):
        got = orc.bf16_to_f32(out[off + b * sc: off + b * sc + R])
        assert np.isfinite(got).all(), "a NaN pad or a NaN C was read"
        rels.append(max_rel(got, refs[b]))
    # nothing outside the outputs was written
    mask = np.ones(out.size, bool)
    for b in range(batch):
        mask[off + b * sc: off + b * sc + R] = False
    assert (out[mask] == cflat[mask]).all()
    print(f"{kind} R={R} K={K}: max rel {max(rels):.2e}")
    assert max(rels) <= TOL, rels


def test_bgemv_harness_cases(hk, orc):
    # bgemm_test.cu:404-447: K = 512; nn_row N = 2048 (seed 700), nt_row N = 384 (710),
    # tn_row N = 2048 with lda = 1 (720), nn_col M = 320 (730); alpha 1, beta 0.5.
    for kind, R, seed in (("nn_row", 2048, 700), ("nt_row", 384, 710), ("tn_row", 2048, 720),
                          ("nn_col", 320, 730)):
        _gemv_case(hk, orc, kind, R, 512, seed=seed)


@pytest.mark.parametrize("kind,R,K,ld,inc", [
    ("nn_row", 1001, 77, 1001, 1),     # element loads (ld not a multiple of 8)
    ("nn_row", 1000, 300, 1008, 1),    # vector loads
    ("nn_row", 1001, 300, 1008, 1),    # vector loads, last lane's outputs cross R
    ("nt_row", 77, 1001, 1001, 1),     # element loads
    ("nt_row", 77, 1001, 1008, 1),     # vector loads with a k tail
    ("nt_row", 5, 3, 3, 1),
    ("tn_row", 333, 129, 336, 3),      # strided x
    ("tn_row", 1, 1, 1, 1),
    ("nn_col", 100, 999, 1000, 1),
    ("nn_col", 1, 8, 8, 1),
])
@pytest.mark.parametrize("batch,off", [(1, 0), (3, 1)])
def test_bgemv_ragged_strided_batched(hk, orc, kind, R, K, ld, inc, batch, off):
    _gemv_case(hk, orc, kind, R, K, ld=ld, inc=inc, batch=batch, off=off, seed=R + K,
               alpha=1.5, beta=-0.75)


@pytest.mark.parametrize("kind,R,K,ld,inc,batch", [
    ("nt_row", 64, 32768, 32768, 1, 1),   # few rows, long k: split over workgroups
    ("nn_row", 512, 16384, 512, 1, 1),
    ("nn_col", 8, 20000, 20000, 1, 2),
    ("tn_row", 300, 9000, 304, 2, 1),
])
def test_bgemv_k_split(hk, orc, kind, R, K, ld, inc, batch):
    _gemv_case(hk, orc, kind, R, K, ld=ld, inc=inc, batch=batch, seed=3, alpha=0.5, beta=0.25)


@pytest.mark.parametrize("kind", list(KINDS))
def test_bgemv_beta_zero_does_not_read_c(hk, orc, kind):
    # the reference's Beta0 instantiations: C is NaN here and must not reach the output
    _gemv_case(hk, orc, kind, 1000, 640, beta=0.0, c_nan=True, seed=11)
    _gemv_case(hk, orc, kind, 40, 20000, beta=0.0, c_nan=True, seed=12)  # split path


def test_bgemv_k_zero_scales_c(hk, orc):
    for kind in KINDS:
        _gemv_case(hk, orc, kind, 300, 0, beta=0.5, seed=13)


@pytest.mark.parametrize("M,N,K", [(1, 1000, 333), (700, 1, 257), (1, 1, 100), (1, 4096, 8192)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_routes_vector_products(hk, orc, M, N, K, ta, tb):
    # hk_bgemm with M == 1 or N == 1 takes the GEMV kernels; results as for any other shape
    from test_gpu_gemm import _check, _operands, _run

    say("bgemm M/N == 1", M, N, K, ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 50 + M + N)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.25, 0.5)
    _check(orc, out, A, B, C0, ta, tb, 1.25, 0.5)
