// hk_host.h - host-side helpers shared by the launchers (validation, device facts, workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hk.h"

#define HK_CHECK_ARG(cond)                 \
  do {                                     \
    if (!(cond)) return hipErrorInvalidValue; \
  } while (0)

#define HK_RETURN_IF_ERROR(expr)           \
  do {                                     \
    hipError_t hk_e_ = (expr);             \
    if (hk_e_ != hipSuccess) return hk_e_; \
  } while (0)

namespace hk {

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Scratch device memory for the launchers' multi-workgroup partials (split-K, reduce, the
// LayerNorm gamma/beta partials): one grow-only buffer per (device, stream), held until the
// process ends. Work on one stream runs in order, so consecutive calls on that stream reuse
// the buffer safely; calls on different streams get different buffers. The pointer is valid
// until the next call on the same (device, stream) asks for more bytes, so a launcher fetches
// it once per call; growing it first waits for the work queued on that stream.
hipError_t device_workspace(size_t bytes, hipStream_t stream, void** out);

// Batched BF16 matrix-vector product (bgemv.hip), shared by the hk_bgemv_* entry points and
// hk_bgemm's M == 1 / N == 1 products. Per batch b (element strides sm, sx, sy):
//   dot_form:  y[r*incy] = alpha sum_k mtx[r*ld + k] x[k*incx] + beta y[r*incy]
//   otherwise: y[r*incy] = alpha sum_k x[k*incx] mtx[k*ld + r] + beta y[r*incy]
// for r < R; y is not read when beta == 0.
hipError_t bgemv_run(bool dot_form, int R, int K, hk_bf16 alpha, hk_bf16 beta,
                     const hk_bf16* mtx, int64_t ld, int64_t sm, const hk_bf16* x, int64_t incx,
                     int64_t sx, hk_bf16* y, int64_t incy, int64_t sy, int batch,
                     hipStream_t stream);

// fp32 output written straight from the BF16 GEMM tiles when the product has one split:
// C[b][row][col] = alpha * acc + beta * C (C not read when beta == 0) + bias_scale * bias, the
// bias selected by bias_stride as hk_sgemm does (N: bias[col]; M*N: bias[(b % M) * N + col];
// 1: bias[0]; bias NULL: none).
struct F32Out {
  float* C;
  int64_t ldc, sC;
  float alpha, beta;
  const float* bias;
  int64_t bias_stride;
  float bias_scale;
};

// fp32 product of bf16 operands on the BF16 GEMM tiles (bgemm.hip), written as split-K partials
// part[s][batch][M][N] (s < used) of op(A) op(B) over k-range [s kps, (s + 1) kps); their sum
// in split order is the product. With used == 1 and out != NULL the tiles write out->C through
// its epilogue instead (part is not touched). Needs the tiled path's alignment: 8-element
// multiples and 16-byte aligned bases. bgemm_split_plan picks (used, kps) for a shape: split_k
// ranges of kps k each (split_k == 0: the library's choice), `used` of them non-empty.
void bgemm_split_plan(int M, int N, int K, int batch, int split_k, int* used, int* kps);
hipError_t bgemm_partials(bool ta, bool tb, int M, int N, int K, const hk_bf16* A, int64_t lda,
                          int64_t sA, const hk_bf16* B, int64_t ldb, int64_t sB, int batch,
                          int used, int kps, float* part, const F32Out* out,
                          hipStream_t stream);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Status of the launch just issued on this thread.
inline hipError_t launch_status() { return hipGetLastError(); }

}  // namespace hk
