"""The C-ABI boundary, checked without a GPU: the library loads, exports every symbol that
include/hk.h declares, its structs have the reference's byte layout, and argument validation
rejects bad calls before any device work is issued."""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HIP_ERROR_INVALID_VALUE = 1


@pytest.fixture(scope="module")
def L():
    from hyperkernels_amd import _lib

    return _lib.lib()


def test_package_front_end_imports():
    import hyperkernels_amd
    from hyperkernels_amd import kernels, workloads

    assert callable(kernels.gelu_forward) and callable(kernels.AdamPlan)
    assert workloads.GPT2_NUM_PARAMS == 124_439_808
    assert hyperkernels_amd.lib() is not None


def test_every_header_symbol_is_exported(L):
    from hyperkernels_amd import _lib

    decls = _lib.parse_header()
    assert len(decls) >= 18
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    missing = sorted(set(decls) - exported)
    assert not missing, f"declared in hk.h but not exported: {missing}"
    extra = sorted(s for s in exported if s.startswith("hk_") and s not in decls)
    assert not extra, f"exported hk_ symbols missing from hk.h: {extra}"
    assert L.hk_abi_version() == 1


_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "hk.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu\n", sizeof(hk_adam_launch_metadata),
         offsetof(hk_adam_launch_metadata, sizes), offsetof(hk_adam_launch_metadata, block_to_tensor),
         offsetof(hk_adam_launch_metadata, block_to_chunk), sizeof(hk_reduction_layout));
  return 0;
}
"""


def test_struct_layouts_match_reference(tmp_path):
    # AdamLaunchMetadata (multi_tensor_adam_sm89_kernel.cu:13-21): 4 x 48 pointers, 48 int64
    # sizes, 320 uchar, 320 int -> 3520 bytes on LP64.
    from hyperkernels_amd.kernels import AdamLaunchMetadata, ReductionLayout

    src = tmp_path / "probe.c"
    src.write_text(_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True)
    size, off_sizes, off_b2t, off_b2c, red = map(int, subprocess.run(
        [str(exe)], capture_output=True, text=True, check=True).stdout.split())
    assert (size, off_sizes, off_b2t, off_b2c) == (3520, 1536, 1920, 2240)
    assert ctypes.sizeof(AdamLaunchMetadata) == size
    assert AdamLaunchMetadata.block_to_chunk.offset == off_b2c
    assert ctypes.sizeof(ReductionLayout) == red == 48


def test_validation_rejects_bad_arguments_without_device_work(L):
    null = ctypes.c_void_p(0)
    assert L.hk_gelu_forward_f32(null, null, -1, null) == HIP_ERROR_INVALID_VALUE
    assert L.hk_gelu_backward_bf16(null, null, null, 16, null) == HIP_ERROR_INVALID_VALUE
    assert L.hk_layer_norm_forward_f32(null, null, null, null, null, null, -1, 768,
                                       ctypes.c_float(1e-5), null) == HIP_ERROR_INVALID_VALUE
    assert L.hk_layer_norm_forward_f32(null, null, null, null, null, null, 4, 768,
                                       ctypes.c_float(1e-5), null) == HIP_ERROR_INVALID_VALUE
    assert L.hk_sparse_ce_forward_f32_i32(null, null, null, null, null, 4, 0,
                                          null) == HIP_ERROR_INVALID_VALUE
    assert L.hk_multi_tensor_adam(null, 1, *([ctypes.c_float(0)] * 7), null) == HIP_ERROR_INVALID_VALUE
    plan = ctypes.c_void_p()
    assert L.hk_adam_plan_create(-1, null, null, null, null, null,
                                 ctypes.byref(plan)) == HIP_ERROR_INVALID_VALUE
    assert L.hk_unified_reduce_sum_f32(null, null, null, null) == HIP_ERROR_INVALID_VALUE
    # empty problems are valid no-ops
    assert L.hk_gelu_forward_f32(null, null, 0, null) == 0
    assert L.hk_sparse_ce_forward_f32_i32(null, null, null, null, null, 0, 7, null) == 0
