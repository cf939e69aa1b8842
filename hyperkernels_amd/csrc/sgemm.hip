// sgemm.hip - batched FP32 GEMM on gfx950 fp32 MFMA with split-K and a fused bias epilogue.
//
// Reference behaviour:
//   sgemm_sm89_kernel<Cfg, Aligned, SplitK, Layout>   blas/fp32/sgemm_sm89_core_template.cu:85-327
//       C = alpha * op(A) op(B) + bias + beta * C; layouts SgemmLayout {NT, TN, NN} (:9);
//       bias indexed by bias_stride: N -> bias[col], M*N -> bias[(batch % M) * N + col],
//       1 -> bias[0] (:303-315); split-K adds atomically into C pre-scaled by beta
//       (sgemm_sm89_scale_kernel, :329-333) and re-adds the bias in every split.
//   sgemm_addmm_sm89_kernel                            blas/fp32/sgemm_addmm_sm89_kernel.cu:66-335
//       C = alpha * A B + beta * C + beta * bias, bias selected by bias_numel (1, N, M*N).
//   tile-specialised kernels (sgemm_nn_256x128_..., sgemm_nt_..., sgemm_tn_...): the same
//       product without bias for one layout each; splitK where the reference has it.
// The reference multiplies with single-pass TF32 MMA; gfx950 has no TF32 matrix instruction, so
// this file uses the full-precision fp32 MFMA (v_mfma_f32_32x32x2_f32): products are exact fp32
// and only the summation order differs from a naive fp32 loop. The roofline for this path is
// MI355X's fp32 matrix peak (157.3 TFLOP/s).
//
// Design (gfx950): the same tiling as the BF16 GEMM of this library - 256 x 256 workgroup
// tile, 4 waves of 128 x 128 (4 x 4 MFMA tiles, 256 fp32 accumulators per lane), k-tiles of
// 32 fp32 (128-byte LDS rows, chunks XOR-permuted so fragment reads and stores are free of
// bank conflicts), two LDS stages with the next k-tile's loads in flight. An operand
// that is M/N-contiguous in HBM is read as 8 k-rows x 4 values and transposed in registers.
// Lane (r, h) of a wave feeds k = 16h + s of each 32-deep k-tile at step s, so a lane reads 16
// consecutive k values of its row per tile as four 16-byte LDS loads.
// Split-K: every split writes fp32 partials; a second kernel sums them in split order and
// applies alpha, beta and the bias exactly once (deterministic, and the bias is not repeated
// per split as in the reference's atomics).
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int kThreads = 256;
constexpr int kWave = 128;
constexpr int kTileElems = 256 * BK;                  // one operand stage, floats
constexpr int kStagePitch = 128 + 4;
constexpr size_t kLdsMain = 2 * 2 * kTileElems * sizeof(float);                    // 131072
constexpr size_t kLdsEpi = static_cast<size_t>(BM) * kStagePitch * sizeof(float);   // 135168
constexpr size_t kLdsBytes = kLdsMain > kLdsEpi ? kLdsMain : kLdsEpi;

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Same placement as the BF16 GEMM: 128-byte rows, 16-byte chunk c of row r at c ^ f(r),
// f(r) = (r ^ (r >> 3)) & 7, conflict-free for 8 consecutive rows at one chunk, for one row at
// 8 chunks and for the transposed stores (rows 4l + c, l = 0..7). Returns the offset in floats.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 32 + ((chunk ^ ((row ^ (row >> 3)) & 7)) * 4);
}

// One operand's share of a k-tile (256 rows x 32 k fp32), 8 16-byte loads per thread.
// KMAJOR: element (row, k) at base[row * ld + k]; thread tt loads chunk tt % 8 of rows
//   tt / 8 + 32 j.
// otherwise: element at base[k * ld + row]; thread tt owns rows 4 (tt % 64) .. +4 and k-rows
//   8 (tt / 64) .. +8 (64 lanes read 1 KB contiguous per k-row), transposed in registers into
//   4 rows x 2 chunks.
template <bool KMAJOR>
struct TileLoader {
  const float* base;
  int64_t ld;
  int rows, K, rbase, tt;

  __device__ void init(const float* b, int64_t l, int nrows, int k, int tile_row0, int t) {
    base = b;
    ld = l;
    rows = nrows;
    K = k;
    rbase = tile_row0;
    tt = t;
  }

  __device__ void load(int k0, float4 (&reg)[8]) const {
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    if (KMAJOR) {
      const int k = k0 + (tt & 7) * 4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = rbase + (tt >> 3) + 32 * j;
        reg[j] = (r < rows && k < K)
                     ? *reinterpret_cast<const float4*>(base + static_cast<int64_t>(r) * ld + k)
                     : zero;
      }
    } else {
      const int r = rbase + (tt & 63) * 4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = k0 + (tt >> 6) * 8 + j;
        reg[j] = (r < rows && k < K)
                     ? *reinterpret_cast<const float4*>(base + static_cast<int64_t>(k) * ld + r)
                     : zero;
      }
    }
  }

  __device__ void store(float* stage, const float4 (&reg)[8]) const {
    if (KMAJOR) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<float4*>(stage + lds_off((tt >> 3) + 32 * j, tt & 7)) = reg[j];
    } else {
      const int row0 = (tt & 63) * 4;
      const int ch0 = (tt >> 6) * 2;
      const float* v = reinterpret_cast<const float*>(reg);  // v[k * 4 + c]
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        *reinterpret_cast<float4*>(stage + lds_off(row0 + c, ch0)) =
            make_float4(v[0 * 4 + c], v[1 * 4 + c], v[2 * 4 + c], v[3 * 4 + c]);
        *reinterpret_cast<float4*>(stage + lds_off(row0 + c, ch0 + 1)) =
            make_float4(v[4 * 4 + c], v[5 * 4 + c], v[6 * 4 + c], v[7 * 4 + c]);
      }
    }
  }
};

__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
  constexpr int G = 8;
  const int per_group = G * tiles_n;
  const int group = t / per_group;
  const int first_m = group * G;
  const int gsz = min(tiles_m - first_m, G);
  const int in_group = t - group * per_group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

__device__ __forceinline__ void mma_stage(const float* a_st, const float* b_st, int wm, int wn,
                                          int lane, f32x16_t (&acc)[4][4]) {
  const int frow = lane & 31;
  const int half = lane >> 5;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float4 af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *reinterpret_cast<const float4*>(a_st + lds_off(wm * kWave + i * 32 + frow,
                                                              half * 4 + q));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bfr[j] = *reinterpret_cast<const float4*>(b_st + lds_off(wn * kWave + j * 32 + frow,
                                                               half * 4 + q));
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = e == 0 ? af[i].x : e == 1 ? af[i].y : e == 2 ? af[i].z : af[i].w;
          const float b = e == 0 ? bfr[j].x : e == 1 ? bfr[j].y : e == 2 ? bfr[j].z : bfr[j].w;
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[i][j], 0, 0, 0);
        }
  }
}

struct Epilogue {
  float alpha, beta;
  const float* bias;
  int64_t bias_stride;  // N, M*N (per-batch row vector at (batch % M) * N), 1, or 0 = none
  float bias_scale;     // 1 (bias added once) or beta (addmm)
};

__device__ __forceinline__ float bias_at(const Epilogue& ep, int M, int N, int batch, int col) {
  if (!ep.bias) return 0.f;
  if (ep.bias_stride == N) return ep.bias[col];
  if (ep.bias_stride == static_cast<int64_t>(M) * N)
    return ep.bias[static_cast<int64_t>(batch % M) * N + col];
  if (ep.bias_stride == 1) return ep.bias[0];
  return 0.f;
}

template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL>
__global__ __launch_bounds__(kThreads, 1) void sgemm_tiled(
    int M, int N, int K, const float* __restrict__ A, int64_t lda, int64_t sA,
    const float* __restrict__ B, int64_t ldb, int64_t sB, float* __restrict__ C, int64_t ldc,
    int64_t sC, Epilogue ep, int split_k, int k_per_split, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  float* sA_st = reinterpret_cast<float*>(lds_raw);
  float* sB_st = sA_st + 2 * kTileElems;

  const int batch = blockIdx.z / split_k;
  const int split = blockIdx.z - batch * split_k;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * k_per_split;
  const int kend = min(K, kbeg + k_per_split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  TileLoader<A_KMAJOR> la;
  TileLoader<B_KMAJOR> lb;
  la.init(A + static_cast<int64_t>(batch) * sA, lda, M, kend, m0, tid);
  lb.init(B + static_cast<int64_t>(batch) * sB, ldb, N, kend, n0, tid);

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  float4 ra[8], rb[8];
  const int ktiles = (kend - kbeg + BK - 1) / BK;
  if (ktiles > 0) {
    la.load(kbeg, ra);
    lb.load(kbeg, rb);
    la.store(sA_st, ra);
    lb.store(sB_st, rb);
  }
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      la.load(kbeg + (kt + 1) * BK, ra);
      lb.load(kbeg + (kt + 1) * BK, rb);
    }
    mma_stage(sA_st + cur * kTileElems, sB_st + cur * kTileElems, wm, wn, lane, acc);
    if (more) {
      la.store(sA_st + (cur ^ 1) * kTileElems, ra);
      lb.store(sB_st + (cur ^ 1) * kTileElems, rb);
    }
    __syncthreads();
  }

  const int lrow = 4 * (lane >> 5);
  const int lcol = lane & 31;
  if (PARTIAL) {
    float* out = part + (static_cast<int64_t>(split) * (gridDim.z / split_k) + batch) *
                            static_cast<int64_t>(M) * N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * kWave + i * 32 + 8 * (r >> 2) + lrow + (r & 3);
          const int col = n0 + wn * kWave + j * 32 + lcol;
          if (row < M && col < N) out[static_cast<int64_t>(row) * N + col] = acc[i][j][r];
        }
    return;
  }

  float* stage = reinterpret_cast<float*>(lds_raw);
  float* Cb = C + static_cast<int64_t>(batch) * sC;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (wn == half) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * kWave + i * 32 + 8 * (r >> 2) + lrow + (r & 3);
            stage[row * kStagePitch + j * 32 + lcol] = acc[i][j][r];
          }
    }
    __syncthreads();
#pragma unroll 4
    for (int it = 0; it < 32; ++it) {
      const int q = tid + it * kThreads;
      const int row = q >> 5;
      const int c4 = (q & 31) * 4;
      const int grow = m0 + row;
      const int gcol = n0 + half * 128 + c4;
      if (grow < M && gcol < N) {
        const float4 v = *reinterpret_cast<const float4*>(stage + row * kStagePitch + c4);
        float4* dst = reinterpret_cast<float4*>(Cb + static_cast<int64_t>(grow) * ldc + gcol);
        float f[4] = {v.x, v.y, v.z, v.w};
        float old[4] = {0.f, 0.f, 0.f, 0.f};
        if (ep.beta != 0.0f) {
          const float4 o = *dst;
          old[0] = o.x; old[1] = o.y; old[2] = o.z; old[3] = o.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[e] = ep.alpha * f[e];
          if (ep.beta != 0.0f) f[e] += ep.beta * old[e];
          if (ep.bias) f[e] += ep.bias_scale * bias_at(ep, M, N, batch, gcol + e);
        }
        *dst = make_float4(f[0], f[1], f[2], f[3]);
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void sgemm_splitk_finalize(const float* __restrict__ part,
                                                             int split_k, int batch, int M, int N,
                                                             float* __restrict__ C, int64_t ldc,
                                                             int64_t sC, Epilogue ep) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t mn = static_cast<int64_t>(M) * N;
  if (idx >= mn * batch) return;
  const int b = static_cast<int>(idx / mn);
  const int64_t e = idx - b * mn;
  const int row = static_cast<int>(e / N), col = static_cast<int>(e - static_cast<int64_t>(row) * N);
  float s = 0.f;
  for (int k = 0; k < split_k; ++k) s += part[(static_cast<int64_t>(k) * batch + b) * mn + e];
  float* dst = C + b * sC + static_cast<int64_t>(row) * ldc + col;
  float f = ep.alpha * s;
  if (ep.beta != 0.0f) f += ep.beta * *dst;
  if (ep.bias) f += ep.bias_scale * bias_at(ep, M, N, b, col);
  *dst = f;
}

// Fallback for shapes the tiled kernel does not take: one thread per output, k-order fp32 sum.
__global__ __launch_bounds__(256) void sgemm_simple(int ta, int tb, int M, int N, int K,
                                                    const float* __restrict__ A, int64_t lda,
                                                    int64_t sA, const float* __restrict__ B,
                                                    int64_t ldb, int64_t sB,
                                                    float* __restrict__ C, int64_t ldc,
                                                    int64_t sC, Epilogue ep) {
  const int col = blockIdx.x * 16 + (threadIdx.x & 15);
  const int row = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int b = blockIdx.z;
  if (row >= M || col >= N) return;
  const float* Ab = A + b * sA;
  const float* Bb = B + b * sB;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const float a = ta ? Ab[static_cast<int64_t>(k) * lda + row] : Ab[static_cast<int64_t>(row) * lda + k];
    const float v = tb ? Bb[static_cast<int64_t>(col) * ldb + k] : Bb[static_cast<int64_t>(k) * ldb + col];
    acc += a * v;
  }
  float* dst = C + b * sC + static_cast<int64_t>(row) * ldc + col;
  float f = ep.alpha * acc;
  if (ep.beta != 0.0f) f += ep.beta * *dst;
  if (ep.bias) f += ep.bias_scale * bias_at(ep, M, N, b, col);
  *dst = f;
}

template <bool AK, bool BKM, bool P>
hipError_t launch_tiled(dim3 grid, hipStream_t stream, int M, int N, int K, const float* A,
                        int64_t lda, int64_t sA, const float* B, int64_t ldb, int64_t sB,
                        float* C, int64_t ldc, int64_t sC, const Epilogue& ep, int split_k,
                        int kps, float* part) {
  static std::once_flag once;
  static hipError_t attr_status = hipSuccess;
  std::call_once(once, [] {
    attr_status = hipFuncSetAttribute(reinterpret_cast<const void*>(&sgemm_tiled<AK, BKM, P>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLdsBytes));
  });
  HK_RETURN_IF_ERROR(attr_status);
  hipLaunchKernelGGL((sgemm_tiled<AK, BKM, P>), grid, dim3(kThreads), kLdsBytes, stream, M, N, K,
                     A, lda, sA, B, ldb, sB, C, ldc, sC, ep, split_k, kps, part);
  return hk::launch_status();
}

template <bool P>
hipError_t dispatch_layout(bool ta, bool tb, dim3 grid, hipStream_t stream, int M, int N, int K,
                           const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb,
                           int64_t sB, float* C, int64_t ldc, int64_t sC, const Epilogue& ep,
                           int split_k, int kps, float* part) {
  if (!ta && !tb)
    return launch_tiled<true, false, P>(grid, stream, M, N, K, A, lda, sA, B, ldb, sB, C, ldc,
                                        sC, ep, split_k, kps, part);
  if (!ta && tb)
    return launch_tiled<true, true, P>(grid, stream, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                       ep, split_k, kps, part);
  if (ta && !tb)
    return launch_tiled<false, false, P>(grid, stream, M, N, K, A, lda, sA, B, ldb, sB, C, ldc,
                                         sC, ep, split_k, kps, part);
  return launch_tiled<false, true, P>(grid, stream, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                      ep, split_k, kps, part);
}

hipError_t sgemm_run(bool ta, bool tb, int M, int N, int K, float alpha, const float* A, int lda,
                     long long strideA, const float* B, int ldb, long long strideB, float beta,
                     float* C, int ldc, long long strideC, const float* bias,
                     long long bias_stride, float bias_scale, int batchCount, int splitK,
                     hipStream_t stream) {
  HK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batchCount >= 0 && splitK >= 1);
  if (M == 0 || N == 0 || batchCount == 0) return hipSuccess;
  HK_CHECK_ARG(C != nullptr && ldc >= N);
  HK_CHECK_ARG(K == 0 || (A != nullptr && B != nullptr));
  HK_CHECK_ARG(lda >= (ta ? M : K) && ldb >= (tb ? K : N));
  if (bias) {
    HK_CHECK_ARG(bias_stride == N || bias_stride == static_cast<long long>(M) * N ||
                 bias_stride == 1);
  }
  const Epilogue ep{alpha, beta, bias, bias ? static_cast<int64_t>(bias_stride) : 0, bias_scale};
  const int contig_a = ta ? M : K, contig_b = tb ? K : N;
  const bool tiled_ok = (contig_a % 4 == 0) && (contig_b % 4 == 0) && (N % 4 == 0) &&
                        (lda % 4 == 0) && (ldb % 4 == 0) && (ldc % 4 == 0) &&
                        (strideA % 4 == 0) && (strideB % 4 == 0) && (strideC % 4 == 0) &&
                        hk::aligned16(A) && hk::aligned16(B) && hk::aligned16(C) && K > 0;
  if (!tiled_ok) {
    dim3 grid((N + 15) / 16, (M + 15) / 16, batchCount);
    hipLaunchKernelGGL(sgemm_simple, grid, dim3(256), 0, stream, ta ? 1 : 0, tb ? 1 : 0, M, N, K,
                       A, static_cast<int64_t>(lda), static_cast<int64_t>(strideA), B,
                       static_cast<int64_t>(ldb), static_cast<int64_t>(strideB), C,
                       static_cast<int64_t>(ldc), static_cast<int64_t>(strideC), ep);
    return hk::launch_status();
  }
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  HK_CHECK_ARG(tiles <= INT32_MAX && static_cast<int64_t>(batchCount) * splitK <= 65535);
  if (splitK == 1) {
    dim3 grid(static_cast<unsigned>(tiles), 1, batchCount);
    return dispatch_layout<false>(ta, tb, grid, stream, M, N, K, A, lda, strideA, B, ldb, strideB,
                                  C, ldc, strideC, ep, 1, K, nullptr);
  }
  const int kps = static_cast<int>(hk::ceil_div(hk::ceil_div(K, splitK), BK) * BK);
  const int used = static_cast<int>(hk::ceil_div(K, kps));
  void* ws = nullptr;
  HK_RETURN_IF_ERROR(hk::device_workspace(
      static_cast<size_t>(used) * batchCount * M * N * sizeof(float), &ws));
  float* part = static_cast<float*>(ws);
  dim3 grid(static_cast<unsigned>(tiles), 1, batchCount * used);
  HK_RETURN_IF_ERROR(dispatch_layout<true>(ta, tb, grid, stream, M, N, K, A, lda, strideA, B, ldb,
                                           strideB, C, ldc, strideC, ep, used, kps, part));
  const int64_t total = static_cast<int64_t>(M) * N * batchCount;
  hipLaunchKernelGGL(sgemm_splitk_finalize, dim3(static_cast<unsigned>(hk::ceil_div(total, 256))),
                     dim3(256), 0, stream, part, used, batchCount, M, N, C,
                     static_cast<int64_t>(ldc), static_cast<int64_t>(strideC), ep);
  return hk::launch_status();
}

bool layout_trans(int layout, bool* ta, bool* tb) {
  if (layout < HK_LAYOUT_NT || layout > HK_LAYOUT_NN) return false;
  *ta = layout == HK_LAYOUT_TN;
  *tb = layout == HK_LAYOUT_NT;
  return true;
}

}  // namespace

extern "C" hipError_t hk_sgemm(int layout, int M, int N, int K, float alpha, const float* A,
                               int lda, long long strideA, const float* B, int ldb,
                               long long strideB, float beta, float* C, int ldc,
                               long long strideC, const float* bias, long long bias_stride,
                               int batchCount, int splitK, hipStream_t stream) {
  bool ta, tb;
  HK_CHECK_ARG(layout_trans(layout, &ta, &tb));
  return sgemm_run(ta, tb, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                   bias, bias_stride, 1.0f, batchCount, splitK, stream);
}

extern "C" hipError_t hk_sgemm_addmm(int M, int N, int K, float alpha, const float* A, int lda,
                                     long long strideA, const float* B, int ldb,
                                     long long strideB, float beta, const float* bias,
                                     int64_t bias_numel, float* C, int ldc, long long strideC,
                                     int batchCount, hipStream_t stream) {
  return sgemm_run(false, false, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc,
                   strideC, bias, bias_numel, beta, batchCount, 1, stream);
}

extern "C" hipError_t hk_sgemm_layout(int layout, int M, int N, int K, float alpha,
                                      const float* A, int lda, long long strideA, const float* B,
                                      int ldb, long long strideB, float beta, float* C, int ldc,
                                      long long strideC, int batchCount, int splitK,
                                      hipStream_t stream) {
  bool ta, tb;
  HK_CHECK_ARG(layout_trans(layout, &ta, &tb));
  return sgemm_run(ta, tb, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                   nullptr, 0, 1.0f, batchCount, splitK, stream);
}
