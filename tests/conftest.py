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


def half_ulp_check(out_bits: np.ndarray, ref_f32: np.ndarray, fmt: str = "bf16",
                   rel_tol: float = 1e-5):
    """16-bit outputs (raw bits, fmt "bf16" or "f16") vs an fp32 reference: every output must
    be the rounding of a value within rel_tol * max|ref| of the reference, i.e.
    |out - ref| <= rel_tol * max|ref| + half an ulp of the format. Returns (number of outputs
    that differ from RNE(ref): the rounding-boundary elements, max rel of the outputs against
    RNE(ref)). RNE(ref) is the oracle's bf16 rounding or numpy's IEEE fp16 conversion."""
    import oracle

    ref_f32 = np.asarray(ref_f32, np.float32)
    out_bits = np.asarray(out_bits, np.uint16)
    if fmt == "bf16":
        ref_bits = oracle.f32_to_bf16(ref_f32)
        to_f = oracle.bf16_to_f32
        mant, min_half_ulp = 7, 0.0
    elif fmt == "f16":
        ref_bits = ref_f32.astype(np.float16).view(np.uint16)
        to_f = lambda b: b.view(np.float16).astype(np.float32)  # noqa: E731
        mant, min_half_ulp = 10, 2.0 ** -25  # subnormal spacing 2^-24
    else:
        raise ValueError(fmt)
    out_f = to_f(out_bits).astype(np.float64)
    ref = ref_f32.astype(np.float64)
    scale = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    _, ex = np.frexp(np.maximum(np.abs(out_f), np.abs(ref)))
    half_ulp = np.maximum(np.ldexp(1.0, ex - mant - 2), min_half_ulp)
    bad = np.abs(out_f - ref) > rel_tol * scale + half_ulp
    assert not bad.any(), (
        f"{int(bad.sum())} {fmt} outputs are not the rounding of a value within {rel_tol:g} "
        f"(relative to max|ref|) of the reference; first at {int(np.flatnonzero(bad)[0])}: "
        f"out {out_f[bad][0]!r} ref {ref[bad][0]!r}")
    n_mis = int((out_bits != ref_bits).sum())
    return n_mis, max_rel(out_f, to_f(ref_bits))


def bf16_ulp_check(out_bits: np.ndarray, ref_f32: np.ndarray, rel_tol: float = 1e-5):
    """half_ulp_check for bf16 outputs."""
    return half_ulp_check(out_bits, ref_f32, "bf16", rel_tol)
