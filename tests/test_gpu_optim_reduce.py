"""GPU parity of multi-tensor AdamW (bit-exact, BASELINE asks <= 1 ulp) and the unified
reduce against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_rel
from hyperkernels_amd import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> int:
    """Max distance in units in the last place between two fp32 arrays (sign-magnitude aware)."""
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.max(np.abs(ia - ib))) if a.size else 0


def _adam_inputs(orc, sizes, seed0, harness=False):
    out = []
    for t, n in enumerate(sizes):
        if harness:  # kernels_test.cu:433-434
            p = orc.rand_uniform(n, 13 + 4 * t)
            g = orc.rand_uniform(n, 14 + 4 * t)
            m = orc.rand_uniform(n, 15 + 4 * t, 0.0, 0.1)
            v = orc.rand_uniform(n, 16 + 4 * t, 0.0, 0.1)
        else:  # p~N(0,.02), g~N(0,1e-2), m~U(0,.1), v~U(0,.1)
            p = orc.normal(n, seed0 + 4 * t, 0.0, 0.02)
            g = orc.normal(n, seed0 + 4 * t + 1, 0.0, 1e-2)
            m = orc.splitmix_uniform(n, seed0 + 4 * t + 2, 0.0, 0.1)
            v = orc.splitmix_uniform(n, seed0 + 4 * t + 3, 0.0, 0.1)
        out.append((p, g, m, v))
    return out


def _check_adam(orc, host_inputs, dev_tensors, hyper):
    lr, b1, b2, eps, wd, bc1, bc2 = hyper
    torch.cuda.synchronize()
    worst = 0
    for (p, g, m, v), (P, G, M, V) in zip(host_inputs, dev_tensors):
        pr, mr, vr = orc.adamw(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2)
        for got, ref in ((P, pr), (M, mr), (V, vr)):
            worst = max(worst, ulp_distance(got.cpu().numpy(), ref))
    return worst


def test_adam_reference_metadata_launch(hk, orc):
    # kernels_test.cu:407-457: one launch over a cycle of GPT shapes up to 48 tensors/320 chunks
    shapes = [768, 768, 3072, 768, 768, 3072]
    sizes = [shapes[t % 6] for t in range(48)]
    say("adam metadata 48 tensors")
    hin = _adam_inputs(orc, sizes, 0, harness=True)
    T = [[torch.from_numpy(a).to(DEV) for a in quad] for quad in hin]
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    hyper = (lr, b1, b2, eps, wd, 1 - b1, 1 - b2)
    hk.multi_tensor_adam([t[0] for t in T], [t[1] for t in T], [t[2] for t in T],
                         [t[3] for t in T], *hyper)
    assert _check_adam(orc, hin, T, hyper) == 0


def test_adam_plan_gpt2_small_148_tensors(hk, orc):
    # 148 tensors, 124,439,808 params, lr 3e-4, b1 .9, b2 .95, wd .1,
    # eps 1e-8, step 1 (bc = 1 - beta).
    sizes = [workloads.numel(s) for s in workloads.gpt2_param_shapes()]
    say("adam plan gpt2 148 tensors", sum(sizes))
    hin = _adam_inputs(orc, sizes, 1000)
    T = [[torch.from_numpy(a).to(DEV) for a in quad] for quad in hin]
    c = workloads.ADAMW
    hyper = (c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"], 1 - c["beta1"],
             1 - c["beta2"])
    plan = hk.AdamPlan([t[0] for t in T], [t[1] for t in T], [t[2] for t in T], [t[3] for t in T])
    assert plan.num_chunks >= 3892  # at least the reference's 32768-element chunking
    plan.step(*hyper)
    assert _check_adam(orc, hin, T, hyper) == 0
    plan.close()


def test_adam_plan_unaligned_and_ragged(hk, orc):
    # tensors that start off a 16-byte boundary (views at odd offsets), sizes not multiple of 4,
    # an empty tensor, a tensor whose four arrays have different 16-byte phases
    sizes = [1, 5, 32769, 0, 70001]
    say("adam plan ragged", sizes)
    hin = _adam_inputs(orc, sizes, 2000)
    T = []
    for k, quad in enumerate(hin):
        ts = []
        for j, a in enumerate(quad):
            off = (k + (j if k == 4 else 0)) % 4
            buf = torch.empty(a.size + off, device=DEV)
            t = buf[off:]
            t.copy_(torch.from_numpy(a))
            ts.append(t)
        T.append(ts)
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.01, 0.1, 0.001)
    plan = hk.AdamPlan([t[0] for t in T], [t[1] for t in T], [t[2] for t in T], [t[3] for t in T])
    plan.step(*hyper)
    assert _check_adam(orc, hin, T, hyper) == 0


# ---------------------------------------------------------------------------------------------
# Unified reduce
# ---------------------------------------------------------------------------------------------
SELFTEST = [  # unified_reduce_standalone.cu:936-951
    ("inner", 64, 100), ("inner", 1024, 4096), ("outer", 64, 100), ("outer", 512, 2048),
    ("generic", 64, 100), ("generic", 256, 3000), ("outer", 2304, 16384), ("outer", 768, 16384),
]


def _layout(hk, path, rows, cols):
    L = hk.ReductionLayout()
    L.num_outputs = rows
    L.reduced_count = cols
    if path == "outer":
        L.path = hk.REDUCE_OUTER
        L.inner_count = rows
        L.input_row_stride = rows
        L.input_outer_stride = rows
    else:
        L.path = hk.REDUCE_INNER if path == "inner" else hk.REDUCE_GENERIC
        L.input_outer_stride = cols
        L.inner_count = 1
        L.input_row_stride = 1
    return L


@pytest.mark.parametrize("path,rows,cols", SELFTEST)
def test_reduce_selftest_cases_exact(hk, orc, path, rows, cols):
    # The self-test input ((i % 17) - 8) * 0.25 sums exactly in fp32: results must be bit-exact.
    say("reduce selftest", path, rows, cols)
    src = orc.reduce_selftest_input(rows * cols)
    out = hk.unified_reduce_sum(torch.from_numpy(src).to(DEV), _layout(hk, path, rows, cols))
    torch.cuda.synchronize()
    if path == "outer":
        ref = orc.reduce_outer(src, rows, rows, rows, rows, cols)
    else:
        ref = orc.reduce_inner(src, rows, cols)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("path,rows,cols", [("inner", 2048, 50304), ("inner", 3, 1000003),
                                            ("inner", 4096, 7), ("outer", 2304, 16384),
                                            ("outer", 5, 300001), ("outer", 100003, 3)])
def test_reduce_random_inputs(hk, orc, path, rows, cols):
    say("reduce random", path, rows, cols)
    src = orc.normal(rows * cols, 91)
    out = hk.unified_reduce_sum(torch.from_numpy(src).to(DEV), _layout(hk, path, rows, cols))
    torch.cuda.synchronize()
    if path == "outer":
        ref = orc.reduce_outer(src, rows, rows, rows, rows, cols)
    else:
        ref = orc.reduce_inner(src, rows, cols)
    # fp32 sums of N(0,1) terms vs a double-accumulated reference: error grows like
    # sqrt(len) * eps * |terms|, i.e. relative to the largest output below 1e-5 here
    assert max_rel(out.cpu().numpy(), ref) <= 1e-5


def test_reduce_middle_axis_and_generic_strides(hk, orc):
    say("reduce middle axis + generic")
    a = orc.normal(6 * 999 * 33, 92).reshape(6, 999, 33)
    A = torch.from_numpy(a).to(DEV)
    L = hk.ReductionLayout()
    L.path, L.num_outputs, L.reduced_count = hk.REDUCE_OUTER, 6 * 33, 999
    L.inner_count, L.input_row_stride, L.input_outer_stride = 33, 33, 999 * 33
    out = hk.unified_reduce_sum(A, L)
    torch.cuda.synchronize()
    assert max_rel(out.cpu().numpy(), a.astype(np.float64).sum(1).reshape(-1)) <= 1e-5
    # generic: sum over axes (0, 2) of [6, 999, 33] -> 999 outputs
    out2 = hk.reduce_generic(A, [999], [33], [6, 33], [999 * 33, 1])
    torch.cuda.synchronize()
    assert max_rel(out2.cpu().numpy(), a.astype(np.float64).sum((0, 2))) <= 1e-5
    # empty reduction writes zeros
    L0 = _layout(hk, "inner", 5, 0)
    z = hk.unified_reduce_sum(A, L0, dst=torch.full((5,), 7.0, device=DEV))
    torch.cuda.synchronize()
    assert (z.cpu().numpy() == 0).all()
