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


def _tile_rows(M):
    """About 96 rows spread over M, at least one in every 256-row output tile, plus the last."""
    rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 96)), [M - 1]]))
    assert len(np.unique(rows // 256)) == -(-M // 256)
    return rows


@pytest.mark.parametrize("which", ["dA_NT", "dB_TN"])
def test_bgemm_backward_baseline_shapes_library_split(hk, orc, which):
    # BASELINE configs[4] backward of Y[8192, 5120] = X[8192, 1280] W[1280, 5120]:
    #   dA = dY W^T: hk_bgemm_nt_backward, M=8192, N=1280, K=5120 (bgemm_backward_nt…:23-32);
    #   dB = X^T dY: hk_bgemm_tn_backward, M=1280, N=5120, K=8192 (bgemm_backward_tn…:25-34).
    # Both have too few 256 x 256 output tiles to fill the device. The library's cost model
    # runs dA (160 tiles of 80 k-tiles) as one split and splits dB's K (100 tiles of 128
    # k-tiles) into fp32 partials summed in split order by the finalize: the paths the bench
    # times. A, B ~ N(0, 1/sqrt(K)); rows in every 256-row tile are checked in full against the
    # oracle, with alpha / beta both active; two runs must give the same bits.
    lib = hk.lib()
    if which == "dA_NT":
        fn, (M, N, K), (ta, tb) = "hk_bgemm_nt_backward", (8192, 1280, 5120), (0, 1)
    else:
        fn, (M, N, K), (ta, tb) = "hk_bgemm_tn_backward", (1280, 5120, 8192), (1, 0)
    splits = lib.hk_bgemm_split_count(ta, tb, M, N, K, 1, 0)
    rows = lib.hk_bgemm_tile_rows(ta, tb, M, N, K, 1, 0)
    cols = lib.hk_bgemm_tile_cols(ta, tb, M, N, K, 1, 0)
    say("bgemm backward baseline", which, "splits", splits, "tile", rows, "x", cols)
    assert splits == (1 if which == "dA_NT" else 2)
    # dA's 160 tiles of 256 x 256 leave 96 CUs idle: it runs on 256 tiles of 256 x 160
    assert (rows, cols) == ((256, 160) if which == "dA_NT" else (256, 256))
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 1000 + M, normal=True)
    first = _run(hk, fn, A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    second = _run(hk, fn, A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    assert np.array_equal(first, second)
    rows = _tile_rows(M)
    Asub = np.ascontiguousarray(A[:, rows] if ta else A[rows, :])
    ref = orc.bgemm(ta, tb, Asub, B, alpha=1.0, beta=0.5, C0=np.ascontiguousarray(C0[rows]))
    rel = max_rel(orc.bf16_to_f32(first[rows]), ref)
    print(f"{which} rel {rel:.2e} over {len(rows)} rows")
    assert rel <= 1e-2


@pytest.mark.parametrize("M,N,K", [(192, 256, 64), (200, 264, 136), (400, 512, 72),
                                   (1000, 136, 520)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1)])
def test_bgemm_192_row_tiles(hk, orc, M, N, K, ta, tb):
    # Products with few 256-row tiles and a k-major A run on 192-row tiles: whole and partial
    # last row tiles, partial column tiles and a K tail, alpha and beta both active
    lib = hk.lib()
    assert lib.hk_bgemm_tile_rows(ta, tb, M, N, K, 1, 0) == 192
    say("bgemm 192-row tiles", M, N, K, ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 1200 + M)
    _check(orc, _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.5, 0.5), A, B, C0, ta, tb, 1.5,
           0.5)


def test_bgemm_tile_rows_query(hk):
    lib = hk.lib()
    # 256 x 160 tiles: NT, one split, whole tiles, 256 x 256 tiles under one round, 256 x 160
    # tiles within one
    assert (lib.hk_bgemm_tile_rows(0, 1, 8192, 1280, 5120, 1, 0),
            lib.hk_bgemm_tile_cols(0, 1, 8192, 1280, 5120, 1, 0)) == (256, 160)
    assert lib.hk_bgemm_tile_cols(0, 0, 8192, 1280, 5120, 1, 0) == 256  # B not k-major
    assert lib.hk_bgemm_tile_cols(0, 1, 8192, 1280, 5112, 1, 0) == 256  # K % 64 != 0
    assert lib.hk_bgemm_tile_cols(0, 1, 8192, 1440, 5120, 1, 0) == 256  # 288 tiles of 160
    assert lib.hk_bgemm_tile_cols(0, 1, 8192, 5120, 1280, 1, 0) == 256  # 256-wide fill
    assert lib.hk_bgemm_tile_cols(0, 1, 8192, 1280, 5120, 1, 2) == 256  # explicit split
    assert lib.hk_bgemm_tile_cols(0, 1, 1, 512, 512, 1, 0) == 0  # GEMV
    assert lib.hk_bgemm_tile_cols(0, 1, -1, 512, 512, 1, 0) == -1
    assert lib.hk_bgemm_tile_rows(0, 0, 8192, 5120, 1280, 1, 0) == 256  # 640 tiles: 2.5 rounds
    assert lib.hk_bgemm_tile_rows(1, 0, 512, 512, 512, 1, 0) == 256  # M-major A
    assert lib.hk_bgemm_tile_rows(0, 0, 512, 512, 512, 1, 4) == 256  # split K
    assert lib.hk_bgemm_tile_rows(0, 0, 1, 512, 512, 1, 0) == 0  # GEMV
    assert lib.hk_bgemm_tile_rows(0, 0, 0, 512, 512, 1, 0) == 0
    assert lib.hk_bgemm_tile_rows(0, 0, -1, 512, 512, 1, 0) == -1


@pytest.mark.parametrize("M,N,K,batch", [(256, 160, 64, 1), (512, 320, 128, 1),
                                         (1024, 800, 320, 1), (2048, 1280, 192, 1),
                                         (512, 480, 256, 2)])
def test_bgemm_256x160_tiles(hk, orc, M, N, K, batch):
    # NT products (both operands k-major) that run on 256 x 160 tiles of 16 x 16 x 32 MFMAs:
    # one tile up to 64, batched, alpha and beta active; each batch against its own product
    lib = hk.lib()
    assert lib.hk_bgemm_tile_rows(0, 1, M, N, K, batch, 0) == 256
    assert lib.hk_bgemm_tile_cols(0, 1, M, N, K, batch, 0) == 160
    say("bgemm 256x160 tiles", M, N, K, batch)
    ops = [_operands(orc, M, N, K, 0, 1, 1300 + 10 * b) for b in range(batch)]
    dA = to_dev_bf16(np.stack([o[0] for o in ops]))
    dB = to_dev_bf16(np.stack([o[1] for o in ops]))
    dC = to_dev_bf16(np.stack([o[2] for o in ops]))
    st = lib.hk_bgemm(0, 1, M, N, K, bits(1.5), dA.data_ptr(), K, M * K, dB.data_ptr(), K, N * K,
                      bits(0.5), dC.data_ptr(), N, M * N, batch,
                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    for b, (A, B, C0) in enumerate(ops):
        _check(orc, out[b], A, B, C0, 0, 1, 1.5, 0.5)


@pytest.mark.parametrize("bias_numel", ["M", "N"])
def test_bgemm_256x160_tiles_bias_and_backward_entry(hk, orc, bias_numel):
    # the bias form (C written, not read) and the dA entry point on 256 x 160 tiles
    M, N, K = 1024, 640, 256
    lib = hk.lib()
    assert lib.hk_bgemm_tile_cols(0, 1, M, N, K, 1, 1) == 160
    say("bgemm 256x160 bias", bias_numel)
    A, B, C0 = _operands(orc, M, N, K, 0, 1, 1400)
    n = M if bias_numel == "M" else N
    bias = orc.f32_to_bf16(orc.splitmix_uniform(n, 1401))
    dA, dB, dC, dbias = to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(C0), to_dev_bf16(bias)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.hk_bgemm_core_bias(0, 1, M, N, K, bits(1.0), dA.data_ptr(), K, 0, dB.data_ptr(),
                                  K, 0, bits(2.0), dbias.data_ptr(), n, dC.data_ptr(), N, 0, 1,
                                  stream) == 0
    ref = orc.bgemm(0, 1, A, B, alpha=1.0, beta=2.0, bias=bias)
    assert max_rel(orc.bf16_to_f32(to_host_bits(dC)), ref) <= 1e-2
    _check(orc, _run(hk, "hk_bgemm_nt_backward", A, B, C0, M, N, K, 0, 1, 1.0, 0.5), A, B, C0,
           0, 1, 1.0, 0.5)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bgemm_long_k_library_split_deterministic(hk, orc, ta, tb):
    # One output tile and 128 k-tiles: the library's split-K choice is >= 2 splits; the fp32
    # partials are summed in split order, so two runs are bit-identical and match the oracle.
    M, N, K = 256, 256, 8192
    lib = hk.lib()
    splits = lib.hk_bgemm_split_count(ta, tb, M, N, K, 1, 0)
    say("bgemm long K", ta, tb, "splits", splits)
    assert splits >= 2
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 1100)
    first = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    second = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    assert np.array_equal(first, second)
    _check(orc, first, A, B, C0, ta, tb, 1.0, 0.5)


@pytest.mark.parametrize("M,N,K,ta,tb", [(17, 9, 33, 0, 0), (33, 65, 7, 1, 1), (64, 64, 8, 1, 0),
                                         (300, 260, 72, 0, 1),
                                         # MFMA path with partial M / N tiles and a K tail
                                         (300, 264, 136, 0, 0), (264, 136, 100, 1, 0),
                                         (520, 392, 200, 1, 1), (264, 520, 328, 0, 1)])
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


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_half_width_tail_tiles(hk, orc, ta, tb):
    # 32 x 20 = 640 output tiles of 256 x 256 would leave half of a third round empty: the
    # library runs the last 4 tile columns (from column 4096) as 256 x 128 tiles, the last of
    # them 120 wide (N = 5112), with a partial last k-tile (K = 136). Rows over every tile row
    # in full, so both column regions and their boundary are checked.
    M, N, K = 8192, 5112, 136
    say("bgemm half-width tail", ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 900)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    rows = _tile_rows(M)
    Asub = np.ascontiguousarray(A[:, rows] if ta else A[rows, :])
    ref = orc.bgemm(ta, tb, Asub, B, alpha=1.0, beta=0.5, C0=np.ascontiguousarray(C0[rows]))
    rel = max_rel(orc.bf16_to_f32(out[rows]), ref)
    print(f"half-width tail rel {rel:.2e}")
    assert rel <= 1e-2


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bgemm_one_launch_ragged_rows(hk, orc, ta, tb):
    # M = 8000: the last tile row of both tile widths is partial (rows 7936..7999) in the launch
    # that runs the 256-wide and the 128-wide tiles together (N = 5112, K = 136 as above).
    M, N, K = 8000, 5112, 136
    say("bgemm one launch ragged rows", ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 950)
    out = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    rows = np.unique(np.concatenate([_tile_rows(M), np.arange(M - 64, M)]))
    Asub = np.ascontiguousarray(A[:, rows] if ta else A[rows, :])
    ref = orc.bgemm(ta, tb, Asub, B, alpha=1.0, beta=0.5, C0=np.ascontiguousarray(C0[rows]))
    rel = max_rel(orc.bf16_to_f32(out[rows]), ref)
    print(f"one launch ragged rows rel {rel:.2e}")
    assert rel <= 1e-2


def test_bgemm_one_launch_batched(hk, orc):
    # Two batches of 4096 x 5120 (2 x 320 tiles of 256 x 256, so the last 4 tile columns of each
    # batch run 128 wide in the same launch, grid.z = 2): each batch against its own product.
    M, N, K, batch = 4096, 5120, 136, 2
    say("bgemm one launch batched")
    As, Bs, Cs = [], [], []
    for b in range(batch):
        A, B, C0 = _operands(orc, M, N, K, 0, 0, 960 + 10 * b)
        As.append(A)
        Bs.append(B)
        Cs.append(C0)
    dA, dB, dC = to_dev_bf16(np.stack(As)), to_dev_bf16(np.stack(Bs)), to_dev_bf16(np.stack(Cs))
    lib = hk.lib()
    assert lib.hk_bgemm_split_count(0, 0, M, N, K, batch, 0) == 1
    st = lib.hk_bgemm(0, 0, M, N, K, bits(1.0), dA.data_ptr(), K, M * K, dB.data_ptr(), N, K * N,
                      bits(0.5), dC.data_ptr(), N, M * N, batch,
                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    rows = _tile_rows(M)
    for b in range(batch):
        ref = orc.bgemm(0, 0, np.ascontiguousarray(As[b][rows, :]), Bs[b], alpha=1.0, beta=0.5,
                        C0=np.ascontiguousarray(Cs[b][rows]))
        assert max_rel(orc.bf16_to_f32(out[b][rows]), ref) <= 1e-2


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_bgemm_partial_last_round_deterministic(hk, orc, ta, tb):
    # 17 x 17 = 289 output tiles (a last round of 33 on 256 CUs), 17 k-tiles, the last partial.
    # Rows sampled over every tile row; the same call twice must give the same bits, and the
    # bias form runs at the same shape.
    M, N, K = 4352, 4352, 1032
    say("bgemm partial last round", ta, tb)
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 800)
    rows = np.unique(np.concatenate([np.arange(0, M, 37), [M - 1]]))
    Asub = np.ascontiguousarray(A[:, rows] if ta else A[rows, :])
    ref = orc.bgemm(ta, tb, Asub, B, alpha=1.0, beta=0.5, C0=np.ascontiguousarray(C0[rows]))
    first = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    second = _run(hk, "hk_bgemm", A, B, C0, M, N, K, ta, tb, 1.0, 0.5)
    assert np.array_equal(first, second)
    rel = max_rel(orc.bf16_to_f32(first[rows]), ref)
    print(f"rel {rel:.2e}")
    assert rel <= 1e-2
    if (ta, tb) == (0, 0):
        lib = hk.lib()
        bias = orc.f32_to_bf16(orc.splitmix_uniform(N, 801, -1.0, 1.0))
        dA, dB, dbias = to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(bias)
        dC = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        stream = torch.cuda.current_stream().cuda_stream
        assert lib.hk_bgemm_addmm(M, N, K, bits(1.0), dA.data_ptr(), K, 0, dB.data_ptr(), N, 0,
                                  bits(0.5), dbias.data_ptr(), N, dC.data_ptr(), N, 0, 1,
                                  stream) == 0
        out = to_host_bits(dC)
        refb = orc.bgemm(0, 0, Asub, B, alpha=1.0, beta=0.5, bias=bias)  # bias per column
        assert max_rel(orc.bf16_to_f32(out[rows]), refb) <= 1e-2


# ---------------------------------------------------------------------------------------------
# FP32 SGEMM (blas/fp32): C = alpha op(A) op(B) + beta C + bias, bias added once; bf16x3 products
# on the BF16 GEMM tiles for 8-aligned shapes, fp32 MFMA tiles for other 4-aligned ones.
# Tolerance: BASELINE.json's 2e-3 relative (max|err| / max|ref|) against the oracle's fp32
# k-order reference (sgemm_test.cu:176-185 restated on the CPU).
# ---------------------------------------------------------------------------------------------
SG_LAYOUT = {"NT": (0, 0, 1), "TN": (1, 1, 0), "NN": (2, 0, 0)}  # name -> (enum, ta, tb)
SG_HARNESS = [(256, 256, 256), (512, 384, 128), (256, 128, 96)]  # sgemm_test.cu:245


def _sg_operands(orc, M, N, K, ta, tb, seed, normal=False):
    if normal:  # A, B ~ N(0, 1/sqrt(K)), bias ~ N(0, 0.02), C0 ~ N(0, 1)
        a = orc.normal(M * K, seed, 0.0, K ** -0.5)
        b = orc.normal(K * N, seed + 1, 0.0, K ** -0.5)
        c0 = orc.normal(M * N, seed + 2)
        bias = orc.normal(N, seed + 3, 0.0, 0.02)
    else:  # sgemm_test.cu:253-270: splitmix U(-1, 1), seeds +1..+4
        a = orc.splitmix_uniform(M * K, seed + 1)
        b = orc.splitmix_uniform(K * N, seed + 2)
        c0 = orc.splitmix_uniform(M * N, seed + 3)
        bias = orc.splitmix_uniform(N, seed + 4)
    return (a.reshape((K, M) if ta else (M, K)), b.reshape((N, K) if tb else (K, N)),
            c0.reshape(M, N), bias)


def _sg_call(hk, fn, layout, A, B, C, M, N, K, alpha, beta, bias=None, bias_stride=0,
             split_k=1, batch=1, sA=0, sB=0, sC=0):
    lib = hk.lib()
    stream = torch.cuda.current_stream().cuda_stream
    lda, ldb = A.shape[-1], B.shape[-1]
    bptr = 0 if bias is None else bias.data_ptr()
    if fn == "hk_sgemm":
        st = lib.hk_sgemm(layout, M, N, K, alpha, A.data_ptr(), lda, sA, B.data_ptr(), ldb, sB,
                          beta, C.data_ptr(), N, sC, bptr, bias_stride, batch, split_k, stream)
    elif fn == "hk_sgemm_addmm":
        st = lib.hk_sgemm_addmm(M, N, K, alpha, A.data_ptr(), lda, sA, B.data_ptr(), ldb, sB,
                                beta, bptr, bias_stride, C.data_ptr(), N, sC, batch, stream)
    else:
        st = lib.hk_sgemm_layout(layout, M, N, K, alpha, A.data_ptr(), lda, sA, B.data_ptr(),
                                 ldb, sB, beta, C.data_ptr(), N, sC, batch, split_k, stream)
    assert st == 0
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("M,N,K", SG_HARNESS)
@pytest.mark.parametrize("lay", ["NN", "NT", "TN"])
@pytest.mark.parametrize("split_k", [0, 1, 4])
def test_sgemm_harness_sizes_bias_split_k(hk, orc, M, N, K, lay, split_k):
    # split_k >= 1 cuts the k loop into split_k ranges of whole 64-deep k-tiles (the bf16x3
    # path's k axis is 3 K long), as the reference's k_chunk rounds to its 16-deep tiles
    # (sgemm_sm89_core_template.cu:126): the non-empty ranges run. 0 is the library's choice.
    enum, ta, tb = SG_LAYOUT[lay]
    if split_k:
        ktiles = -(-3 * K // 64)
        per = -(-ktiles // split_k)
        assert hk.lib().hk_sgemm_split_count(enum, M, N, K, 1, split_k) == -(-ktiles // per)
    say("sgemm", lay, M, N, K, split_k)
    A, B, C0, bias = _sg_operands(orc, M, N, K, ta, tb, 7 + M)
    out = _sg_call(hk, "hk_sgemm", enum, torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV),
                   torch.from_numpy(C0).to(DEV), M, N, K, 1.5, 0.5,
                   bias=torch.from_numpy(bias).to(DEV), bias_stride=N, split_k=split_k)
    ref = orc.sgemm(ta, tb, A, B, alpha=1.5, beta=0.5, C0=C0, bias=bias)
    assert max_rel(out, ref) <= 2e-3


def test_sgemm_bias_strides_and_batches(hk, orc):
    M, N, K, batch = 64, 96, 40, 3
    say("sgemm bias strides")
    As = [_sg_operands(orc, M, N, K, 0, 0, 50 + b) for b in range(batch)]
    A = torch.from_numpy(np.stack([x[0] for x in As])).to(DEV)
    B = torch.from_numpy(np.stack([x[1] for x in As])).to(DEV)
    C0 = np.stack([x[2] for x in As])
    full_bias = orc.splitmix_uniform(M * N, 77).reshape(M, N)
    for stride, bias_np in ((N, As[0][3]), (M * N, full_bias.reshape(-1)), (1, full_bias[0, :1])):
        for split_k in (1, 3):
            C = torch.from_numpy(C0.copy()).to(DEV)
            out = _sg_call(hk, "hk_sgemm", 2, A, B, C, M, N, K, 1.0, -0.5,
                           bias=torch.from_numpy(np.ascontiguousarray(bias_np)).to(DEV),
                           bias_stride=stride, split_k=split_k, batch=batch, sA=M * K, sB=K * N,
                           sC=M * N)
            for b in range(batch):
                ref = orc.sgemm(0, 0, As[b][0], As[b][1], alpha=1.0, beta=-0.5, C0=C0[b])
                if stride == N:
                    ref = ref + bias_np
                elif stride == M * N:  # the reference's (batch % M) * N row (core_template:310)
                    ref = ref + full_bias[b % M]
                else:
                    ref = ref + bias_np[0]
                assert max_rel(out[b], ref) <= 2e-3, (stride, split_k, b)


@pytest.mark.parametrize("lay", ["NN", "TN"])
@pytest.mark.parametrize("split_k", [1, 3])
def test_sgemm_tiles_write_c_one_split_or_serial_ranges(hk, orc, lay, split_k):
    # 4 batches of 2048 x 2048 fill the device with 256 output tiles, so the GEMM tiles apply
    # alpha, beta and the bias to C themselves: with one k split, or with 3 (3 K = 768, 12
    # k-tiles, 3 ranges of 4) added into C one after the other, beta and the bias in the first
    # only. A bias added per range would be off by 2 bias, beta applied per range by a power.
    M, N, K, batch = 2048, 2048, 256, 4
    enum, ta, tb = SG_LAYOUT[lay]
    say("sgemm tiles write C", lay, "split_k", split_k)
    assert hk.lib().hk_sgemm_split_count(enum, M, N, K, batch, split_k) == split_k
    As = [_sg_operands(orc, M, N, K, ta, tb, 300 + 10 * b) for b in range(batch)]
    A = torch.from_numpy(np.stack([x[0] for x in As])).to(DEV)
    B = torch.from_numpy(np.stack([x[1] for x in As])).to(DEV)
    C0 = np.stack([x[2] for x in As])
    full_bias = orc.splitmix_uniform(M * N, 377).reshape(M, N)
    for stride, bias_np in ((N, As[0][3]), (M * N, full_bias.reshape(-1)), (1, full_bias[0, :1])):
        C = torch.from_numpy(C0.copy()).to(DEV)
        out = _sg_call(hk, "hk_sgemm", enum, A, B, C, M, N, K, 1.5, -0.5,
                       bias=torch.from_numpy(np.ascontiguousarray(bias_np)).to(DEV),
                       bias_stride=stride, batch=batch, sA=M * K, sB=K * N, sC=M * N,
                       split_k=split_k)
        for b in range(batch):
            ref = orc.sgemm(ta, tb, As[b][0], As[b][1], alpha=1.5, beta=-0.5, C0=C0[b])
            if stride == N:
                ref = ref + bias_np
            elif stride == M * N:  # the reference's (batch % M) * N row (core_template:310)
                ref = ref + full_bias[b % M]
            else:
                ref = ref + bias_np[0]
            assert max_rel(out[b], ref) <= 2e-3, (stride, b)


def test_sgemm_addmm_beta_scaled_bias(hk, orc):
    M, N, K = 256, 256, 256
    say("sgemm addmm")
    A, B, C0, bias = _sg_operands(orc, M, N, K, 0, 0, 90)
    out = _sg_call(hk, "hk_sgemm_addmm", 2, torch.from_numpy(A).to(DEV),
                   torch.from_numpy(B).to(DEV), torch.from_numpy(C0).to(DEV), M, N, K, 1.0, 0.5,
                   bias=torch.from_numpy(bias).to(DEV), bias_stride=N)
    ref = orc.sgemm(0, 0, A, B, alpha=1.0, beta=0.5, C0=C0) + 0.5 * bias
    assert max_rel(out, ref) <= 2e-3


@pytest.mark.parametrize("lay", ["NN", "NT", "TN"])
def test_sgemm_tile_kernel_entry_point(hk, orc, lay):
    enum, ta, tb = SG_LAYOUT[lay]
    M, N, K = 512, 384, 128
    say("sgemm layout entry", lay)
    A, B, C0, _ = _sg_operands(orc, M, N, K, ta, tb, 120)
    out = _sg_call(hk, "hk_sgemm_layout", enum, torch.from_numpy(A).to(DEV),
                   torch.from_numpy(B).to(DEV), torch.from_numpy(C0).to(DEV), M, N, K, 1.0, 0.5,
                   split_k=2)
    assert max_rel(out, orc.sgemm(ta, tb, A, B, alpha=1.0, beta=0.5, C0=C0)) <= 2e-3


@pytest.mark.parametrize("M,N,K,lay", [(260, 264, 100, "NN"), (260, 264, 100, "NT"),
                                       (260, 264, 100, "TN"), (300, 256, 64, "TN"),
                                       # whole 256 x 256 tiles, 16 k-tiles with a K tail
                                       (768, 512, 516, "NN"), (768, 512, 516, "NT"),
                                       (516, 512, 768, "TN")])
@pytest.mark.parametrize("split_k", [1, 2])
def test_sgemm_fp32_tile_path(hk, orc, M, N, K, lay, split_k):
    # K (or M for TN) a multiple of 4 but not of 8: the fp32 MFMA tiles, not the bf16x3 path
    enum, ta, tb = SG_LAYOUT[lay]
    say("sgemm fp32 tiles", M, N, K, lay, split_k)
    A, B, C0, bias = _sg_operands(orc, M, N, K, ta, tb, 900 + K)
    out = _sg_call(hk, "hk_sgemm", enum, torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV),
                   torch.from_numpy(C0).to(DEV), M, N, K, 1.5, 0.5,
                   bias=torch.from_numpy(bias).to(DEV), bias_stride=N, split_k=split_k)
    ref = orc.sgemm(ta, tb, A, B, alpha=1.5, beta=0.5, C0=C0, bias=bias)
    assert max_rel(out, ref) <= 2e-3


@pytest.mark.parametrize("M,N,K,lay", [(17, 9, 33, "NN"), (33, 65, 7, "TN"), (5, 300, 41, "NT")])
def test_sgemm_ragged(hk, orc, M, N, K, lay):
    enum, ta, tb = SG_LAYOUT[lay]
    say("sgemm ragged", M, N, K, lay)
    A, B, C0, bias = _sg_operands(orc, M, N, K, ta, tb, 130)
    out = _sg_call(hk, "hk_sgemm", enum, torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV),
                   torch.from_numpy(C0).to(DEV), M, N, K, 1.0, 1.0,
                   bias=torch.from_numpy(bias).to(DEV), bias_stride=N)
    assert max_rel(out, orc.sgemm(ta, tb, A, B, alpha=1.0, beta=1.0, C0=C0, bias=bias)) <= 2e-3


@pytest.mark.parametrize("lay", ["NN", "NT", "TN"])
@pytest.mark.parametrize("split_k", [4, 0])
def test_sgemm_baseline_shape_split_k4_sampled_rows(hk, orc, lay, split_k):
    # 4096^3 with split-K 4 (4 k ranges really run: the 256 output tiles
    # fill the device, so the ranges are added into C in split order) and the fused bias;
    # split_k 0 is the library's own plan.
    # beta = 1 with C0 ~ N(0, 1) and the bias ~ N(0, 0.02) against a product of std 1/64: a
    # bias added once per split (the reference's split-K epilogue) would be off by 3 * bias,
    # ~8x the 2e-3 bound, and beta * C applied per split by 3 * C0. 64 rows checked in full.
    enum, ta, tb = SG_LAYOUT[lay]
    M = N = K = 4096
    splits = hk.lib().hk_sgemm_split_count(enum, M, N, K, 1, split_k)
    say("sgemm baseline", lay, "split_k", split_k, "splits", splits)
    if split_k:
        assert splits == split_k
    A, B, C0, bias = _sg_operands(orc, M, N, K, ta, tb, 140, normal=True)
    out = _sg_call(hk, "hk_sgemm", enum, torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV),
                   torch.from_numpy(C0).to(DEV), M, N, K, 1.0, 1.0,
                   bias=torch.from_numpy(bias).to(DEV), bias_stride=N, split_k=split_k)
    rows = np.unique(np.concatenate([np.arange(0, M, 67), [M - 1]]))
    Asub = np.ascontiguousarray(A[:, rows] if ta else A[rows, :])
    ref = orc.sgemm(ta, tb, Asub, B, alpha=1.0, beta=1.0, C0=np.ascontiguousarray(C0[rows]),
                    bias=bias)
    rel = max_rel(out[rows], ref)
    print(f"sgemm baseline rel {rel:.2e}")
    assert rel <= 2e-3


@pytest.mark.parametrize("split_k", [1, 3])
def test_sgemm_infinite_operand(hk, orc, split_k):
    # An inf in A reaches the outputs of its row as +-inf, as it does through the reference's
    # TF32 products and the oracle's fp32 loop. The bf16x3 split keeps the inf in the high part
    # and zeroes its low part and its copy in the cross term; without that, inf * b_lo (NaN for
    # b_lo = 0 or of the other sign) and bf16(inf - inf) would turn the row into NaN.
    M, N, K = 64, 128, 96
    say("sgemm inf operand", split_k)
    A, B, C0, _ = _sg_operands(orc, M, N, K, 0, 0, 150)
    A = A.copy()
    A[3, 5] = np.inf
    A[7, 9] = -np.inf
    A[11, 2] = np.float32(3.4e38)  # finite, rounds past bf16's largest value, not to inf
    assert hk.lib().hk_sgemm_split_count(2, M, N, K, 1, split_k) == split_k
    out = _sg_call(hk, "hk_sgemm", 2, torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV),
                   torch.from_numpy(C0).to(DEV), M, N, K, 1.0, 0.5, split_k=split_k)
    ref = orc.sgemm(0, 0, A, B, alpha=1.0, beta=0.5, C0=C0)
    for r in (3, 7):
        assert np.isinf(ref[r]).all()
        np.testing.assert_array_equal(out[r], ref[r])
    # the 3.4e38 row stays finite (hi = bf16's largest value, lo = the rest), as in TF32, and
    # matches the oracle's fp32 products (|b| < 1, so no product overflows)
    assert np.abs(B[2]).max() < 1 and np.isfinite(ref[11]).all()
    assert np.isfinite(out[11]).all()
    assert max_rel(out[11], ref[11]) <= 2e-3
    finite = np.setdiff1d(np.arange(M), [3, 7, 11])
    assert max_rel(out[finite], ref[finite]) <= 2e-3


def test_bgemm_split_k_on_concurrent_streams(hk, orc):
    # Split-K partials live in a library workspace; two streams running split-K GEMMs at the
    # same time must each get their own (a shared one would mix the partials).
    lib = hk.lib()
    say("bgemm split-K on two streams")
    M, N, K = 512, 512, 2048
    cases = []
    for seed in (900, 910):
        A, B, C0 = _operands(orc, M, N, K, 0, 0, seed)
        cases.append((A, B, C0, to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(C0)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for rep in range(3):
        for (A, B, C0, dA, dB, dC), s in zip(cases, streams):
            with torch.cuda.stream(s):
                st = lib.hk_bgemm_core(2, 4, M, N, K, bits(1.0), dA.data_ptr(), K, 0,
                                       dB.data_ptr(), N, 0, bits(0.0), dC.data_ptr(), N, 0, 1,
                                       s.cuda_stream)
                assert st == 0
        torch.cuda.synchronize()
        for (A, B, C0, dA, dB, dC) in cases:
            _check(orc, to_host_bits(dC), A, B, C0, 0, 0, 1.0, 0.0)


@pytest.mark.parametrize("numel", ["N", "M", "1", "MN", "none"])
@pytest.mark.parametrize("M,N,K", [(256, 512, 128), (300, 264, 136), (17, 9, 33)])
def test_bgemm_addmm_bias_forms(hk, orc, numel, M, N, K):
    # bgemm_addmm_kernel: C = alpha A B + beta bias, C not read (test_bgemm_addmm_sm89.cu:91-94)
    say("bgemm addmm", numel, M, N, K)
    lib = hk.lib()
    A, B, C0 = _operands(orc, M, N, K, 0, 0, 700)
    size = {"N": N, "M": M, "1": 1, "MN": M * N, "none": 0}[numel]
    bias = orc.f32_to_bf16(orc.splitmix_uniform(max(size, 1), 701)) if size else None
    dA, dB, dC = to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(C0)
    dbias = to_dev_bf16(bias) if size else None
    st = lib.hk_bgemm_addmm(M, N, K, bits(1.5), dA.data_ptr(), K, 0, dB.data_ptr(), N, 0,
                            bits(0.5), dbias.data_ptr() if size else None, size, dC.data_ptr(),
                            N, 0, 1, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    out = to_host_bits(dC)
    # C is only written: the previous contents (C0) must not contribute
    ref = (orc.bgemm(0, 0, A, B, alpha=1.5, beta=0.5, bias=bias) if size
           else orc.bgemm(0, 0, A, B, alpha=1.5))
    assert max_rel(orc.bf16_to_f32(out), ref) <= 1e-2


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("split_k", [1, 3])
def test_bgemm_core_bias_split_k(hk, orc, ta, tb, split_k):
    # core template with the split-K bias initialisation (bgemm_core_template.cu:270-289)
    M, N, K = 264, 520, 328
    say("bgemm core bias", ta, tb, split_k)
    lib = hk.lib()
    A, B, C0 = _operands(orc, M, N, K, ta, tb, 720)
    bias = orc.f32_to_bf16(orc.splitmix_uniform(M, 721))  # per-row form
    dA, dB, dC = to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(C0)
    dbias = to_dev_bf16(bias)
    layout = {(0, 1): 0, (1, 0): 1, (0, 0): 2}[(ta, tb)]
    st = lib.hk_bgemm_core_bias(layout, split_k, M, N, K, bits(1.0), dA.data_ptr(), A.shape[1], 0,
                                dB.data_ptr(), B.shape[1], 0, bits(2.0), dbias.data_ptr(), M,
                                dC.data_ptr(), N, 0, 1, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    ref = orc.bgemm(ta, tb, A, B, alpha=1.0, beta=2.0, bias=bias)
    assert max_rel(orc.bf16_to_f32(to_host_bits(dC)), ref) <= 1e-2


def test_bgemm_addmm_rejects_unknown_bias_size(hk, orc):
    lib = hk.lib()
    M, N, K = 64, 64, 64
    A, B, C0 = _operands(orc, M, N, K, 0, 0, 730)
    dA, dB, dC = to_dev_bf16(A), to_dev_bf16(B), to_dev_bf16(C0)
    dbias = to_dev_bf16(orc.f32_to_bf16(orc.splitmix_uniform(7, 731)))
    st = lib.hk_bgemm_addmm(M, N, K, bits(1.0), dA.data_ptr(), K, 0, dB.data_ptr(), N, 0,
                            bits(1.0), dbias.data_ptr(), 7, dC.data_ptr(), N, 0, 1,
                            torch.cuda.current_stream().cuda_stream)
    assert st == 1  # hipErrorInvalidValue
