"""GPU parity of the BF16 batched GEMM (all layouts, core template with split-K, backward dA/dB)
against the CPU oracle's fp32-accumulated reference (the BLAS harnesses' naive reference,
bgemm_test.cu:186-197, restated on the CPU). Tolerance: BASELINE.json's 1e-2 relative to an
fp32-accumulated reference (max|err| / max|ref|); the tests also report the tighter figure."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
HARNESS_SIZES = [(256, 256, 256), (512, 384, 128), (136, 72, 200)]  # bgemm_test.cu:257-258


def say(*a):
    print("[case]", *a, flush=True)


def to_dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV).view(torch.bfloat16)


def to_host_bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def bits(x: float) -> int:
    return int(torch.tensor([x], dtype=torch.bfloat16).view(torch.int16).item()) & 0xFFFF


def _operands(orc, M, N, K, ta, tb, seed, normal=False):
    if normal:  # A, B ~ N(0, 1/sqrt(K))
        a = orc.normal(M * K, seed, 0.0, K ** -0.5)
        b = orc.normal(K * N, seed + 1, 0.0, K ** -0.5)
    else:  # bgemm_test.cu:161-172 fill: splitmix64 U(-1, 1)
        a = orc.splitmix_uniform(M * K, seed + 1, -1.0, 1.0)
        b = orc.splitmix_uniform(K * N, seed + 2, -1.0, 1.0)
    A = orc.f32_to_bf16(a).reshape((K, M) if ta else (M, K))
    B = orc.f32_to_bf16(b).reshape((N, K) if tb else (K, N))
    C0 = orc.f32_to_bf16(orc.splitmix_uniform(M * N, seed + 3, -1.0, 1.0)).reshape(M, N)
    return A, B, C0


def _run(hk, fn, A, B, C0, M, N, K, ta, tb, alpha, beta, **kw):
    lib = hk.lib()
    dA, dB = to_dev_bf16(A), to_dev_bf16(B)
    dC = to_dev_bf16(C0)
    stream = torch.cuda.current_stream().cuda_stream
    lda, ldb = A.shape[1], B.shape[1]
    if fn == "hk_bgemm":
        st = lib.hk_bgemm(ta, tb, M, N, K, bits(alpha), dA.data_ptr(), lda, 0, dB.data_ptr(), ldb,
                          0, bits(beta), dC.data_ptr(), N, 0, 1, stream)
    elif fn == "hk_bgemm_core":
        layout = {(0, 1): 0, (1, 0): 1, (0, 0): 2}[(ta, tb)]
        st = lib.hk_bgemm_core(layout, kw.get("split_k", 1), M, N, K, bits(alpha), dA.data_ptr(),
                               lda, 0, dB.data_ptr(), ldb, 0, bits(beta), dC.data_ptr(), N, 0, 1,
                               stream)
    else:
        st = getattr(lib, fn)(M, N, K, bits(alpha), dA.data_ptr(), lda, 0, dB.data_ptr(), ldb, 0,
                              bits(beta), dC.data_ptr(), N, 0, 1, stream)
    assert st == 0
    return to_host_bits(dC)


def _check(orc, out_bits, A, B, C0, ta, tb, alpha, beta, tol=1e-2):
    ref = orc.bgemm(ta, tb, A, B, alpha=alpha, beta=beta, C0=C0)
    rel = max_rel(orc.bf16_to_f32(out_bits), ref)
    # Output rounding alone allows 2^-9 of the element; the accumulation order differs from the
    # naive k-order loop by fp32 rounding only.
    assert rel <= tol, rel
    return rel


@pytest.mark.parametrize("M,N,K", HARNESS_SIZES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_all_layouts_harness_sizes(hk, orc, M, N, K, ta, tb):
    say("bgemm", M, N, K, ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 100 + M)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    rel = _check(orc, out, A, B, C0, ta, tb, 1.0, 0.5)
    print(f"rel {rel:.2e}")


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (0, 0)])
@pytest.mark.parametrize("split_k", [1, 4])
def test_bgemm_core_template_split_k(hk, orc, ta, tb, split_k):
    M, N, K = 512, 384, 1000 - 1000 % 8
    say("bgemm core", ta, tb, split_k)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 300)
    out = _run(hk, "hk_bgemm_core", A, B, C0, M, N, K, ta, tb, 1.0, 0.5, split_k=split_k)
    _check(orc, out, A, B, C0, ta, tb, 1.0, 0.5)


def test_bgemm_backward_entry_points(hk, orc):
    M, N, K = 256, 128, 320
    say("bgemm nt/tn backward")
    A, B, C0 = _operands(orc, M, N, K, 0, 1, 400)
    _check(orc, _run(hk, "hk_bgemm_nt_backward", A, B, C0, M, N, K, 0, 1, 1.0, 0.0), A, B, C0,
           0, 1, 1.0, 0.0)
    A, B, C0 = _operands(orc, M, N, K, 1, 0, 401)
    _check(orc, _run(hk, "hk_bgemm_tn_backward", A, B, C0, M, N, K, 1, 0, 2.0, 1.0), A, B, C0,
           1, 0, 2.0, 1.0)


@pytest.mark.parametrize("M,N,K,ta,tb", [(17, 9, 33, 0, 0), (33, 65, 7, 1, 1), (64, 64, 8, 1, 0),
                                         (300, 260, 72, 0, 1)])
def test_bgemm_ragged_and_partial_tiles(hk, orc, M, N, K, ta, tb):
    say("bgemm ragged", M, N, K, ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 500)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    _check(orc, out, A, B, C0, ta, tb, 1.0, 0.5)


def test_bgemm_batched_strided(hk, orc):
    M, N, K, batch = 128, 256, 64, 3
    say("bgemm batched")
    As, Bs = [], []
    for b in range(batch):
        A, B, _ = _operands(orc, M, N, K, 0, 0, 600 + 10 * b)
        As.append(A)
        Bs.append(B)
    dA, dB = to_dev_bf16(np.stack(As)), to_dev_bf16(np.stack(Bs))
    dC = torch.zeros(batch, M, N, device=DEV, dtype=torch.bfloat16)
    lib = hk.lib()
    st = lib.hk_bgemm(0, 0, M, N, K, bits(1.0), dA.data_ptr(), K, M * K, dB.data_ptr(), N, K * N,
                      bits(0.0), dC.data_ptr(), N, M * N, batch,
                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    for b in range(batch):
        ref = orc.bgemm(0, 0, As[b], Bs[b])
        assert max_rel(orc.bf16_to_f32(out[b]), ref) <= 1e-2


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_baseline_shape_sampled_rows(hk, orc, ta, tb):
    # M=8192, K=1280, N=5120, A,B ~ N(0, 1/sqrt(K)), beta = 0. The whole
    # product runs on the GPU; the oracle checks 96 rows spread over M (every tile row) in full.
    M, N, K = 8192, 5120, 1280
    say("bgemm baseline", ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 700, normal=True)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.0)
    rows = np.unique(np.concatenate([np.arange(0, M, 97), [M - 1]]))
    Asub = A[:, rows] if ta else A[rows, :]
    ref = orc.bgemm(ta, tb, np.ascontiguousarray(Asub), B)
    rel = max_rel(orc.bf16_to_f32(out[rows]), ref)
    print(f"baseline rel {rel:.2e}")
    assert rel <= 1e-2
