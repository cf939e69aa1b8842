"""GPU parity of hk_unified_reduce_sum_f32_noalloc (the reduce whose split partials live in a
fixed device array instead of an allocated workspace) against hk_unified_reduce_sum_f32 on the
same inputs: the same plan, so the same bits. Two calls in a row, the second smaller, on the
split inner and outer paths, plus the paths that need no partials."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def _layout(hk, path, rows, cols):
    L = hk.ReductionLayout()
    L.num_outputs, L.reduced_count = rows, cols
    if path == "outer":
        L.path, L.inner_count, L.input_row_stride, L.input_outer_stride = (
            hk.REDUCE_OUTER, rows, rows, rows)
    else:
        L.path = hk.REDUCE_INNER if path == "inner" else hk.REDUCE_GENERIC
        L.input_outer_stride, L.inner_count, L.input_row_stride = cols, 1, 1
    return L


def _both(hk, L, src):
    lib = hk.lib()
    stream = torch.cuda.current_stream().cuda_stream
    n = L.num_outputs
    ref = torch.full((n,), float("nan"), device=DEV)
    got = torch.full((n,), float("nan"), device=DEV)
    assert lib.hk_unified_reduce_sum_f32(ctypes.byref(L), src.data_ptr(), ref.data_ptr(),
                                         stream) == 0
    assert lib.hk_unified_reduce_sum_f32_noalloc(ctypes.byref(L), src.data_ptr(), got.data_ptr(),
                                                 stream) == 0
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


# (path, rows, cols) of the first call, then a smaller second one. The inner cases split each
# row over many workgroups (few long rows); the outer ones split the reduced axis (2304 x 16384
# is the reference self-test's bias-gradient shape and the largest partial set at 256 CUs).
CASES = [
    ("inner", (3, 1000003), (2, 300001)),
    ("outer", (2304, 16384), (768, 4099)),
    ("inner", (4096, 777), (64, 100)),      # one workgroup per row or a wave per row
    ("generic", (256, 3000), (64, 100)),    # no partials
]


@pytest.mark.parametrize("path,first,second", CASES)
def test_noalloc_reduce_matches_allocating_entry_point(hk, orc, path, first, second):
    for seed, (rows, cols) in ((11, first), (12, second)):
        say("noalloc reduce", path, rows, cols)
        a = orc.normal(rows * cols, seed)
        src = torch.from_numpy(a).to(DEV)
        ref, got = _both(hk, _layout(hk, path, rows, cols), src)
        np.testing.assert_array_equal(got, ref)
        exact = (a.reshape(cols, rows).astype(np.float64).sum(0) if path == "outer"
                 else a.reshape(rows, cols).astype(np.float64).sum(1))
        assert max_rel(got, exact) <= 1e-5


def test_noalloc_reduce_selftest_input_exact(hk, orc):
    # the reference self-test's exactly summable input ((i % 17) - 8) / 4: bit-exact sums
    for rows, cols in ((3, 1000003), (2304, 16384)):
        path = "inner" if rows == 3 else "outer"
        say("noalloc reduce selftest input", path, rows, cols)
        src = orc.reduce_selftest_input(rows * cols)
        ref, got = _both(hk, _layout(hk, path, rows, cols), torch.from_numpy(src).to(DEV))
        want = (orc.reduce_outer(src, rows, rows, rows, rows, cols) if path == "outer"
                else orc.reduce_inner(src, rows, cols))
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(ref, want)
