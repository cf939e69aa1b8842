"""hyperkernels_amd - MI355X (gfx950) HIP implementation of the HyperKernels training-kernel surface.

The product is the C-ABI shared library ``libhk_amd.so`` (declared in ``include/hk.h``); this
package builds it (``hyperkernels_amd.build``), loads it (``hyperkernels_amd._lib``) and mirrors
the reference kernel surface over torch device tensors (``hyperkernels_amd.kernels``).
"""
from __future__ import annotations

__all__ = ["lib"]


def lib():
    """The loaded C-ABI library (raises if it has not been built)."""
    from ._lib import lib as _load

    return _load()
