// bgemv.hip - batched BF16 matrix-vector products (the M == 1 / N == 1 GEMMs), fp32 accumulate.
//
// Reference behaviour (blas/bf16/bgemv_sm89_kernel.cu:11-208), per batch b:
//   nn_row  M == 1: C[n] = alpha sum_k A[k]       B[k*ldb + n]  (+ beta C[n])
//   nt_row  M == 1: C[n] = alpha sum_k A[k]       B[n*ldb + k]
//   tn_row  M == 1: C[n] = alpha sum_k A[k*lda]   B[k*ldb + n]
//   nn_col  N == 1: C[m] = alpha sum_k A[m*lda+k] B[k]
// with batch strides sA, sB, sC; the reference's Beta0 instantiations are beta == 0 here, where
// C is not read. Results are rounded to bf16 once, to nearest even.
//
// Two shapes of work cover all four (and every M == 1 / N == 1 product of hk_bgemm):
//   dot form   y[r] = sum_k Mtx[r*ld + k] x[k*incx]  - matrix rows run along k (nt_row, nn_col)
//   bcast form y[n] = sum_k x[k*incx] Mtx[k*ld + n]  - matrix rows run along n (nn_row, tn_row)
// Both stream the matrix from HBM exactly once with 16-byte loads (8 bf16), so the bound is HBM
// bandwidth: 2 K R bytes per batch. The vector (x) is small and is re-read from L2.
//
// Design (gfx950):
//   dot form: 16 lanes per matrix row (256 B of the row per step), 16 rows per 256-lane
//     workgroup, eight steps of loads in flight per lane; the 16 partial sums of a row are
//     combined with lane shuffles.
//   bcast form: each lane owns 8 consecutive outputs, so a 64-lane wave covers 512 outputs;
//     the 16 waves of a workgroup take interleaved k and are summed through LDS (measured on
//     MI355X at K 4096 x N 16384: 6.9 TB/s with 16 waves against 5.6 with 4). A round's eight
//     x values are loaded once per wave and broadcast with readlane.
//   When rows (dot) or 512-column strips (bcast) alone give too few workgroups to keep every
//   CU streaming, k is split across workgroups: each writes fp32 partials to the per-stream
//   workspace and a finalize pass sums them in split order, so results do not depend on
//   timing.
#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kDotLanes = 16;                   // lanes per row, dot form
constexpr int kDotRows = kThreads / kDotLanes;  // rows per workgroup, dot form
constexpr int kDotStep = kDotLanes * 8;         // k per step of a 16-lane group
constexpr int kColsPerWave = HK_WAVE * 8;       // outputs per workgroup, bcast form
constexpr int kWaves = 16;                      // waves per workgroup, bcast form
constexpr int kBcastThreads = kWaves * HK_WAVE;
constexpr int kUnroll = 8;                      // 16-byte matrix loads in flight per lane
// workgroups per launch that keep every CU streaming (about 32 waves per CU)
constexpr int kDotTargetGroups = 2048;
constexpr int kBcastTargetGroups = 512;

struct Out {
  float alpha, beta;
  uint16_t* y;
  int64_t incy, sy;
  float* part;  // NULL: write y; else partials [batch][nsplit][R]
  int nsplit;
};

__device__ __forceinline__ void emit(const Out& o, int b, int s, int R, int r, float sum) {
  if (o.part) {
    o.part[(static_cast<int64_t>(b) * o.nsplit + s) * R + r] = sum;
    return;
  }
  uint16_t* yp = o.y + b * o.sy + r * o.incy;
  float v = o.alpha * sum;
  if (o.beta != 0.0f) v += o.beta * hk::bf16_to_f32(*yp);
  *yp = hk::f32_to_bf16(v);
}

__device__ __forceinline__ float dot8(const uint4& a, const uint4& b) {
  float fa[8], fb[8];
  hk::BF16::unpack(a, fa);
  hk::BF16::unpack(b, fb);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += fa[i] * fb[i];
  return s;
}

// ---- dot form --------------------------------------------------------------------------------
// grid: (ceil(R / 16), nsplit, batch). VEC: matrix rows and x start 16-byte aligned (ld, sM,
// sx multiples of 8, incx == 1); otherwise element loads.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_dot(int R, int K, int kchunk,
                                                     const uint16_t* __restrict__ mtx,
                                                     int64_t ld, int64_t sm,
                                                     const uint16_t* __restrict__ x,
                                                     int64_t incx, int64_t sx, Out out) {
  const int b = blockIdx.z, s = blockIdx.y;
  const int j = threadIdx.x & (kDotLanes - 1);
  const int r = blockIdx.x * kDotRows + (threadIdx.x >> 4);
  const int kbeg = s * kchunk;
  const int kend = min(K, kbeg + kchunk);
  float acc = 0.f;
  if (r < R) {
    const uint16_t* row = mtx + b * sm + static_cast<int64_t>(r) * ld;
    const uint16_t* xb = x + b * sx;
    if (VEC) {
      const int kvec = kbeg + ((kend - kbeg) & ~7);  // end of the whole 8-element vectors
      // kUnroll vectors in flight per lane, the last round predicated
      for (int k = kbeg + 8 * j; k < kvec; k += kUnroll * kDotStep) {
        uint4 m[kUnroll], v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          if (k + u * kDotStep < kvec) {
            m[u] = hk::ld_nt(reinterpret_cast<const uint4*>(row + k + u * kDotStep));
            v[u] = *reinterpret_cast<const uint4*>(xb + k + u * kDotStep);
          }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
          if (k + u * kDotStep < kvec) acc += dot8(m[u], v[u]);
      }
      if (kvec + j < kend) acc += hk::bf16_to_f32(row[kvec + j]) * hk::bf16_to_f32(xb[kvec + j]);
    } else {
      for (int k = kbeg + j; k < kend; k += kDotLanes)
        acc += hk::bf16_to_f32(row[k]) * hk::bf16_to_f32(xb[k * incx]);
    }
  }
  static_assert(kDotLanes == 16, "the dot form sums each row over one 16-lane DPP row");
  acc = hk::row16_sum(acc);
  if (r < R && j == 0) emit(out, b, s, R, r, acc);
}

// ---- bcast form ------------------------------------------------------------------------------
// grid: (ceil(R / 512), nsplit, batch). VEC: matrix rows start 16-byte aligned (ld, sM
// multiples of 8); the workgroup whose 512 outputs cross R loads element by element.
template <bool VEC>
__global__ __launch_bounds__(kBcastThreads) void gemv_bcast(int R, int K, int kchunk,
                                                       const uint16_t* __restrict__ mtx,
                                                       int64_t ld, int64_t sm,
                                                       const uint16_t* __restrict__ x,
                                                       int64_t incx, int64_t sx, Out out) {
  __shared__ float4 red[kWaves - 1][HK_WAVE][2];
  const int b = blockIdx.z, s = blockIdx.y;
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * kColsPerWave + 8 * lane;
  const int kbeg = s * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const uint16_t* base = mtx + b * sm + n0;
  const uint16_t* xb = x + b * sx;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int k = kbeg + wave;
  if (VEC && static_cast<int>(blockIdx.x + 1) * kColsPerWave <= R) {
    // Every lane of the workgroup owns 8 outputs (uniform branch). Whole rounds: kUnroll rows
    // of 16 bytes in flight per lane with no condition between them; the round's kUnroll x
    // values come from one load spread over the first lanes, broadcast with readlane, so no
    // matrix load waits on an x load.
    for (; k + (kUnroll - 1) * kWaves < kend; k += kUnroll * kWaves) {
      const int xr = xb[(k + (lane & (kUnroll - 1)) * kWaves) * incx];
      uint4 m[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        m[u] = hk::ld_nt(reinterpret_cast<const uint4*>(base + (k + u * kWaves) * ld));
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float xv =
            __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(xr, u)) << 16);
        float f[8];
        hk::BF16::unpack(m[u], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += xv * f[i];
      }
    }
    for (; k < kend; k += kWaves) {  // fewer than kUnroll rows left
      float f[8];
      hk::BF16::unpack(hk::ld_nt(reinterpret_cast<const uint4*>(base + k * ld)), f);
      const float xv = hk::bf16_to_f32(xb[k * incx]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += xv * f[i];
    }
  } else if (n0 < R) {
    // the strip that straddles R, or rows that are not 16-byte aligned: element loads
    for (; k < kend; k += kWaves) {
      const float xv = hk::bf16_to_f32(xb[k * incx]);
      const uint16_t* rowp = base + k * ld;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (n0 + i < R) acc[i] += xv * hk::bf16_to_f32(rowp[i]);
    }
  }
  // the other waves hand their sums to wave 0, which adds them in wave order
  if (wave > 0) {
    red[wave - 1][lane][0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    red[wave - 1][lane][1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  __syncthreads();
  if (wave == 0 && n0 < R) {
#pragma unroll 3  // bounded: a full unroll hoists all 30 LDS reads and spills
    for (int w = 0; w < kWaves - 1; ++w) {
      const float4 lo = red[w][lane][0], hi = red[w][lane][1];
      acc[0] += lo.x; acc[1] += lo.y; acc[2] += lo.z; acc[3] += lo.w;
      acc[4] += hi.x; acc[5] += hi.y; acc[6] += hi.z; acc[7] += hi.w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (n0 + i < R) emit(out, b, s, R, n0 + i, acc[i]);
  }
}

// y = alpha * (sum of the nsplit partials, in split order) + beta * y
__global__ __launch_bounds__(kThreads) void gemv_finalize(int R, int batch, Out out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= static_cast<int64_t>(R) * batch) return;
  const int b = static_cast<int>(i / R), r = static_cast<int>(i - static_cast<int64_t>(b) * R);
  const float* p = out.part + static_cast<int64_t>(b) * out.nsplit * R + r;
  float s = 0.f;
  // sixteen partial loads in flight (one round at the usual split counts), added in split order
  for (int k = 0; k < out.nsplit; k += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = k + u < out.nsplit ? p[static_cast<int64_t>(k + u) * R] : 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u) s += v[u];
  }
  Out o = out;
  o.part = nullptr;
  emit(o, b, 0, R, r, s);
}

float bf16_bits_to_float(hk_bf16 h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// k split so that (groups per split) x nsplit reaches `target`, keeping at least
// min_k k per split; the chunk is a multiple of `align`.
void pick_split(int64_t groups, int64_t target, int K, int min_k, int align, int* nsplit,
                int* kchunk) {
  int64_t s = 1;
  if (groups < target && K > min_k) {
    s = hk::ceil_div(target, groups);
    const int64_t cap = K / min_k;
    if (s > cap) s = cap;
    if (s < 1) s = 1;
  }
  int64_t chunk = hk::ceil_div(hk::ceil_div(K, s), align) * align;
  if (chunk < 1) chunk = 1;
  *kchunk = static_cast<int>(chunk);
  *nsplit = static_cast<int>(K == 0 ? 1 : hk::ceil_div(K, chunk));
}

}  // namespace

namespace hk {

hipError_t bgemv_run(bool dot_form, int R, int K, hk_bf16 alpha, hk_bf16 beta,
                     const hk_bf16* mtx, int64_t ld, int64_t sm, const hk_bf16* x, int64_t incx,
                     int64_t sx, hk_bf16* y, int64_t incy, int64_t sy, int batch,
                     hipStream_t stream) {
  HK_CHECK_ARG(R >= 0 && K >= 0 && batch >= 0);
  if (R == 0 || batch == 0) return hipSuccess;
  HK_CHECK_ARG(y != nullptr && (K == 0 || (mtx != nullptr && x != nullptr)));
  HK_CHECK_ARG(batch <= 65535);
  Out out{bf16_bits_to_float(alpha), bf16_bits_to_float(beta), y, incy, sy, nullptr, 1};
  const int64_t strips = dot_form ? hk::ceil_div(R, kDotRows) : hk::ceil_div(R, kColsPerWave);
  HK_CHECK_ARG(strips <= INT32_MAX);
  int nsplit = 1, kchunk = K;
  if (dot_form)
    pick_split(strips * batch, kDotTargetGroups, K, 4 * kDotStep, kDotStep, &nsplit, &kchunk);
  else
    pick_split(strips * batch, kBcastTargetGroups, K, kUnroll * kWaves, kWaves, &nsplit,
               &kchunk);
  HK_CHECK_ARG(nsplit <= 65535);
  if (nsplit > 1) {
    void* ws = nullptr;
    HK_RETURN_IF_ERROR(hk::device_workspace(
        static_cast<size_t>(batch) * nsplit * R * sizeof(float), stream, &ws));
    out.part = static_cast<float*>(ws);
    out.nsplit = nsplit;
  }
  const dim3 grid(static_cast<unsigned>(strips), static_cast<unsigned>(nsplit),
                  static_cast<unsigned>(batch));
  if (dot_form) {
    const bool vec = ld % 8 == 0 && sm % 8 == 0 && incx == 1 && sx % 8 == 0 &&
                     hk::aligned16(mtx) && hk::aligned16(x);
    hipLaunchKernelGGL(vec ? gemv_dot<true> : gemv_dot<false>, grid, dim3(kThreads), 0, stream, R,
                       K, kchunk, mtx, ld, sm, x, incx, sx, out);
  } else {
    const bool vec = ld % 8 == 0 && sm % 8 == 0 && hk::aligned16(mtx);
    hipLaunchKernelGGL(vec ? gemv_bcast<true> : gemv_bcast<false>, grid, dim3(kBcastThreads), 0,
                       stream, R, K, kchunk, mtx, ld, sm, x, incx, sx, out);
  }
  HK_RETURN_IF_ERROR(hk::launch_status());
  if (nsplit > 1) {
    const int64_t total = static_cast<int64_t>(R) * batch;
    hipLaunchKernelGGL(gemv_finalize, dim3(static_cast<unsigned>(hk::ceil_div(total, kThreads))),
                       dim3(kThreads), 0, stream, R, batch, out);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  return hipSuccess;
}

}  // namespace hk

extern "C" hipError_t hk_bgemv_nn_row(int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                      const hk_bf16* B, int ldb, hk_bf16 beta, hk_bf16* C,
                                      int batchCount, long long sA, long long sB, long long sC,
                                      hipStream_t stream) {
  HK_CHECK_ARG(ldb >= N);
  return hk::bgemv_run(false, N, K, alpha, beta, B, ldb, sB, A, 1, sA, C, 1, sC, batchCount,
                       stream);
}

extern "C" hipError_t hk_bgemv_nt_row(int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                      const hk_bf16* B, int ldb, hk_bf16 beta, hk_bf16* C,
                                      int batchCount, long long sA, long long sB, long long sC,
                                      hipStream_t stream) {
  HK_CHECK_ARG(ldb >= K);
  return hk::bgemv_run(true, N, K, alpha, beta, B, ldb, sB, A, 1, sA, C, 1, sC, batchCount,
                       stream);
}

extern "C" hipError_t hk_bgemv_tn_row(int N, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                      const hk_bf16* B, int ldb, hk_bf16 beta, hk_bf16* C,
                                      int batchCount, long long sA, long long sB, long long sC,
                                      hipStream_t stream) {
  HK_CHECK_ARG(lda >= 1 && ldb >= N);
  return hk::bgemv_run(false, N, K, alpha, beta, B, ldb, sB, A, lda, sA, C, 1, sC, batchCount,
                       stream);
}

extern "C" hipError_t hk_bgemv_nn_col(int M, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                      const hk_bf16* B, hk_bf16 beta, hk_bf16* C,
                                      int batchCount, long long sA, long long sB, long long sC,
                                      hipStream_t stream) {
  HK_CHECK_ARG(lda >= K);
  return hk::bgemv_run(true, M, K, alpha, beta, A, lda, sA, B, 1, sB, C, 1, sC, batchCount,
                       stream);
}
