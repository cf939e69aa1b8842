"""The HBM stream measurement kernel (hk_hbm_stream) computes what its header states, so the
ceilings bench.py reports come from a kernel that really reads and writes every byte."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("nin,nout", [(1, 0), (0, 1), (1, 1), (2, 1), (4, 3), (3, 2)])
@pytest.mark.parametrize("unroll", [1, 2, 4])
def test_hbm_stream_values(nin, nout, unroll):
    from hyperkernels_amd import _lib

    L = _lib.lib()
    n = 1024 * 37 + 4  # a partial last span
    print("[case]", nin, nout, unroll, n, flush=True)
    ins = [torch.randn(n, device=DEV) for _ in range(nin)]
    outs = [torch.full((n,), float("nan"), device=DEV) for _ in range(nout)]
    sink = torch.zeros(-(-n // 1024), device=DEV)
    pin = (ctypes.c_void_p * 4)(*[t.data_ptr() for t in ins])
    pout = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in outs])
    assert L.hk_hbm_stream(pin, nin, pout, nout, n, unroll, sink.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    ref = sum(ins) if nin else torch.zeros(n, device=DEV)
    for j, o in enumerate(outs):
        # same summation order as the kernel (inputs in order), so the sums agree exactly
        acc = torch.zeros(n, device=DEV)
        for t in ins:
            acc = acc + t
        assert torch.equal(o, acc + float(j)), (j, (o - ref - j).abs().max())
    if nout == 0:
        assert torch.count_nonzero(sink) == 0


def test_hbm_stream_rejects_bad_arguments():
    from hyperkernels_amd import _lib

    L = _lib.lib()
    x = torch.zeros(8, device=DEV)
    p = (ctypes.c_void_p * 4)(x.data_ptr(), 0, 0, 0)
    assert L.hk_hbm_stream(p, 5, p, 1, 8, 1, None, _stream()) != 0      # too many inputs
    assert L.hk_hbm_stream(p, 1, p, 1, 6, 1, None, _stream()) != 0      # n not a multiple of 4
    assert L.hk_hbm_stream(p, 1, p, 1, 8, 3, None, _stream()) != 0      # unroll not 1, 2, 4
    assert L.hk_hbm_stream(p, 1, None, 0, 8, 1, None, _stream()) != 0   # read-only needs a sink
