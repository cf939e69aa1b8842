"""Shared pytest configuration: the `gpu` marker, import paths and tolerance helpers."""
from __future__ import annotations

import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on first use."""
    import oracle

    oracle.lib()
    oracle.set_threads(min(16, os.cpu_count() or 1))
    return oracle


@pytest.fixture(scope="session")
def hk():
    """The HIP kernel library through its torch front end; requires a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test without a visible GPU")
    from hyperkernels_amd import kernels

    kernels.lib()
    return kernels


def max_rel(out, ref) -> float:
    """The reference harnesses' metric: max |out - ref| / max |ref| (sgemm_test.cu:204)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    return float(np.max(np.abs(out - ref))) / denom if ref.size else 0.0


def bf16_ulp_check(out_bits: np.ndarray, ref_f32: np.ndarray, rel_tol: float = 1e-5):
    """bf16 outputs vs an fp32 reference: the output must equal RNE(ref) except on elements
    whose reference sits within rel_tol * max|ref| of a rounding midpoint, where one bf16 ulp
    either way is accepted. Returns (number of boundary elements, max rel vs rounded ref)."""
    import oracle

    ref_bits = oracle.f32_to_bf16(ref_f32)
    out_f = oracle.bf16_to_f32(out_bits).astype(np.float64)
    ref_r = oracle.bf16_to_f32(ref_bits).astype(np.float64)
    mism = out_bits != ref_bits
    n_mis = int(mism.sum())
    scale = max(float(np.max(np.abs(ref_f32))), 1e-30)
    if n_mis:
        r = ref_f32.astype(np.float64)[mism]
        o = out_f[mism]
        rr = ref_r[mism]
        # o and rr must be adjacent bf16 values with r near their midpoint
        mid = 0.5 * (o + rr)
        ulp = np.abs(o - rr)
        ok = (np.abs(r - mid) <= rel_tol * scale) & (ulp <= np.maximum(np.abs(rr), np.abs(o)) * 2.0**-7 + 1e-45)
        assert ok.all(), (
            f"{int((~ok).sum())} bf16 outputs differ from RNE(reference) away from a rounding "
            f"boundary; first at {np.flatnonzero(mism)[np.flatnonzero(~ok)[0]]}")
    return n_mis, max_rel(out_f, ref_r)
