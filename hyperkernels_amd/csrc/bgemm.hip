// bgemm.hip - batched BF16 GEMM on gfx950 MFMA: C = alpha * op(A) op(B) + beta * C,
// bf16 operands, fp32 accumulation, bf16 output, row-major, all four transpose layouts.
//
// Reference behaviour:
//   bgemm_NN_kernel<transA, transB>          blas/bf16/bgemm_nn_128x128_sm89_kernel.cu:23-216
//   bgemm_NN_128x128_64x3_kernel             blas/bf16/bgemm_nn_128x128_64x3_sm89_kernel.cu:23
//   bgemm_backward_template_kernel<...>      blas/bf16/bgemm_core_template.cu:61-268 (NN/NT/TN,
//                                            split-K accumulated with bf16 atomics)
//   bgemm_nt_backward_kernel (dA)            blas/bf16/bgemm_backward_nt_sm89_kernel.cu:23-180
//   bgemm_tn_backward_kernel (dB)            blas/bf16/bgemm_backward_tn_sm89_kernel.cu:25-182
// Layouts (row-major): op(A) = A [M,K] (lda >= K) or A^T with A stored [K,M] (lda >= M);
// op(B) = B [K,N] (ldb >= N) or B^T with B stored [N,K] (ldb >= K).
//
// Design (gfx950, CDNA4):
//   - Workgroup tile 256 x 256, k-step 64, 4 waves (2 x 2, one per SIMD); each wave owns a
//     128 x 128 block of C as 4 x 4 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators
//     per lane). Per 16-deep k step a wave issues 16 MFMAs against 8 LDS fragment reads.
//   - Both operands live in LDS "k-contiguous" ([row][64 k] bf16, 128 B rows; chunk
//     placement XOR-permuted so fragment reads and both store patterns are free of bank
//     conflicts, see lds_off). An operand that is k-contiguous in HBM is copied as
//     16-byte chunks; one that is M- or N-contiguous (A^T, plain B) is read as 8 x 8 bf16
//     blocks along its contiguous axis and transposed in registers before the LDS store, so
//     all four layouts share one compute loop and every HBM access is a 16-byte load.
//   - Two LDS stages and two register stages: tile kt + 2 is being fetched from HBM/L2 while
//     tile kt + 1 waits in registers and tile kt is multiplied; one barrier per k-tile.
//   - Epilogue: accumulators are staged through LDS as fp32 (half a tile at a time) and written
//     as 16-byte bf16 rows, with alpha and beta applied in fp32 and a single rounding (the
//     reference rounds alpha*acc to bf16 and then blends beta*C in bf16 arithmetic).
//   - Workgroup order: consecutive tiles go to one XCD (the hardware deals workgroups to the 8
//     XCDs round-robin) in groups of 8 tile-rows, so each XCD's L2 sees a compact C region.
//   - Split-K (the core-template entry point with splitK > 1): each split writes fp32 partials
//     to the library workspace; a second kernel sums them in split order and applies
//     alpha/beta (deterministic; the reference accumulates with lossy bf16 atomics).
// Shapes the tiled kernel does not take (a contiguous extent or leading dimension that is not
// a multiple of 8, pointers not 16-byte aligned) run on a simple fp32-accumulating kernel.
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 256;                         // 4 waves, 2 x 2 over the tile
constexpr int kWaveM = 128, kWaveN = 128;             // 4 x 4 MFMA tiles of 32 x 32 per wave
constexpr int kTileElems = 256 * BK;                  // one operand stage, bf16 elements
constexpr int kStagePitch = 128 + 4;                  // fp32 epilogue staging row pitch
constexpr size_t kLdsMain = 2 * 2 * kTileElems * sizeof(uint16_t);                 // 131072
constexpr size_t kLdsEpi = static_cast<size_t>(BM) * kStagePitch * sizeof(float);   // 135168
constexpr size_t kLdsBytes = kLdsMain > kLdsEpi ? kLdsMain : kLdsEpi;

typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// LDS layout of one operand stage: 256 rows x 64 k (bf16). A row is 128 bytes, i.e. one pass
// over the 32 LDS banks; its eight 16-byte chunks are placed at chunk ^ f(row),
// f(row) = (row ^ (row >> 3)) & 7. A 16-byte LDS access is served 8 lanes at a time, and with
// this placement each group of 8 lanes touches 8 distinct chunk positions (all 32 banks) in the
// three access patterns below:
//   - MFMA fragment reads: 8 consecutive rows, one chunk (f = row ^ const);
//   - k-major stores: one row, 8 chunks;
//   - transposed stores: rows 8l + j for 8 consecutive l, one chunk (f = j ^ l).
// Returns the offset in bf16 elements.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row ^ (row >> 3)) & 7)) * 8);
}

// Transposes an 8 x 8 block of bf16: in[r] holds 8 values of row r (two per 32-bit word, lower
// index in the low half); out[c] receives column c.
__device__ __forceinline__ void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
  const uint32_t* w[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) w[r] = reinterpret_cast<const uint32_t*>(&in[r]);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    uint32_t o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t a = w[2 * d][c >> 1], b = w[2 * d + 1][c >> 1];
      o[d] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    out[c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One operand's share of a k-tile (256 rows of M or N x 64 k), 8 16-byte loads per thread.
// KMAJOR (element (row, k) at base[row * ld + k]): thread tt loads chunk tt % 8 of rows
//   tt / 8 + 32 j; eight lanes read one contiguous 128-byte row segment.
// otherwise (element at base[k * ld + row]): thread tt owns the 8 x 8 block of rows
//   8 (tt % 32) .. +8 and k chunk tt / 32, read as 8 k-rows of 16 bytes (32 lanes read 512
//   contiguous bytes) and transposed in registers.
template <bool KMAJOR>
struct TileLoader {
  const uint16_t* base;
  int64_t ld;
  int rows, K;
  int rbase;  // first global row of this tile
  int tt;

  __device__ void init(const uint16_t* b, int64_t l, int nrows, int k, int tile_row0, int t) {
    base = b;
    ld = l;
    rows = nrows;
    K = k;
    rbase = tile_row0;
    tt = t;
  }

  __device__ void load(int k0, uint4 (&reg)[8]) const {
    const uint4 zero = make_uint4(0, 0, 0, 0);
    if (KMAJOR) {
      const int k = k0 + (tt & 7) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = rbase + (tt >> 3) + 32 * j;
        reg[j] = (r < rows && k < K)
                     ? *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(r) * ld + k)
                     : zero;
      }
    } else {
      const int r = rbase + (tt & 31) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = k0 + (tt >> 5) * 8 + j;
        reg[j] = (r < rows && k < K)
                     ? *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(k) * ld + r)
                     : zero;
      }
    }
  }

  __device__ void store(uint16_t* stage, const uint4 (&reg)[8]) const {
    if (KMAJOR) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<uint4*>(stage + lds_off((tt >> 3) + 32 * j, tt & 7)) = reg[j];
    } else {
      uint4 t[8];
      transpose8x8(reg, t);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<uint4*>(stage + lds_off((tt & 31) * 8 + j, tt >> 5)) = t[j];
    }
  }
};

// Linear workgroup id -> (tile_m, tile_n): consecutive ids to one XCD, grouped 8 tile-rows.
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

// 16 MFMAs per 16-deep k step against 8 fragment reads.
__device__ __forceinline__ void mma_stage(const uint16_t* a_st, const uint16_t* b_st, int wm,
                                          int wn, int lane, f32x16_t (&acc)[4][4]) {
  const int frow = lane & 31;
  const int fch = lane >> 5;
#pragma unroll
  for (int s = 0; s < BK / 16; ++s) {
    bf16x8_t af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *reinterpret_cast<const bf16x8_t*>(a_st + lds_off(wm * kWaveM + i * 32 + frow,
                                                                s * 2 + fch));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bfr[j] = *reinterpret_cast<const bf16x8_t*>(b_st + lds_off(wn * kWaveN + j * 32 + frow,
                                                                 s * 2 + fch));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  }
}

template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL>
__global__ __launch_bounds__(kThreads, 1) void bgemm_tiled(
    int M, int N, int K, float alpha, const uint16_t* __restrict__ A, int64_t lda, int64_t sA,
    const uint16_t* __restrict__ B, int64_t ldb, int64_t sB, float beta, uint16_t* __restrict__ C,
    int64_t ldc, int64_t sC, int split_k, int k_per_split, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  uint16_t* sA_st = reinterpret_cast<uint16_t*>(lds_raw);           // [2][256*64]
  uint16_t* sB_st = sA_st + 2 * kTileElems;                         // [2][256*64]

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

  // The next k-tile's global loads are in flight while the current one is multiplied.
  uint4 ra[8], rb[8];
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

  // Accumulator (i, j, r) of this lane sits at tile row wm*128 + i*32 + 8*(r/4) + 4*(lane/32)
  // + r%4 and tile column wn*128 + j*32 + lane%32.
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
          const int row = m0 + wm * kWaveM + i * 32 + 8 * (r >> 2) + lrow + (r & 3);
          const int col = n0 + wn * kWaveN + j * 32 + lcol;
          if (row < M && col < N) out[static_cast<int64_t>(row) * N + col] = acc[i][j][r];
        }
    return;
  }

  float* stage = reinterpret_cast<float*>(lds_raw);
  uint16_t* Cb = C + static_cast<int64_t>(batch) * sC;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (wn == half) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wm * kWaveM + i * 32 + 8 * (r >> 2) + lrow + (r & 3);
            stage[row * kStagePitch + j * 32 + lcol] = acc[i][j][r];
          }
    }
    __syncthreads();
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int q = tid + it * kThreads;
      const int row = q >> 4;
      const int c8 = (q & 15) * 8;
      const int grow = m0 + row;
      const int gcol = n0 + half * 128 + c8;
      if (grow < M && gcol < N) {
        const float4 v0 = *reinterpret_cast<const float4*>(stage + row * kStagePitch + c8);
        const float4 v1 = *reinterpret_cast<const float4*>(stage + row * kStagePitch + c8 + 4);
        float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        uint4* dst = reinterpret_cast<uint4*>(Cb + static_cast<int64_t>(grow) * ldc + gcol);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= alpha;
        if (beta != 0.0f) {
          const uint4 old = *dst;
          const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[2 * e] += beta * __uint_as_float(ow[e] << 16);
            f[2 * e + 1] += beta * __uint_as_float(ow[e] & 0xffff0000u);
          }
        }
        *dst = make_uint4(hk::pack_bf16x2(f[0], f[1]), hk::pack_bf16x2(f[2], f[3]),
                          hk::pack_bf16x2(f[4], f[5]), hk::pack_bf16x2(f[6], f[7]));
      }
    }
    __syncthreads();
  }
}

// C = alpha * sum_s part[s] + beta * C (split order), fp32 -> bf16.
__global__ __launch_bounds__(256) void bgemm_splitk_finalize(const float* __restrict__ part,
                                                             int split_k, int batch, int M, int N,
                                                             float alpha, float beta,
                                                             uint16_t* __restrict__ C,
                                                             int64_t ldc, int64_t sC) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t mn = static_cast<int64_t>(M) * N;
  if (idx >= mn * batch) return;
  const int b = static_cast<int>(idx / mn);
  const int64_t e = idx - b * mn;
  const int row = static_cast<int>(e / N), col = static_cast<int>(e - static_cast<int64_t>(row) * N);
  float s = 0.f;
  for (int k = 0; k < split_k; ++k) s += part[(static_cast<int64_t>(k) * batch + b) * mn + e];
  uint16_t* dst = C + b * sC + static_cast<int64_t>(row) * ldc + col;
  float f = alpha * s;
  if (beta != 0.0f) f += beta * hk::bf16_to_f32(*dst);
  *dst = hk::f32_to_bf16(f);
}

// Fallback: one thread per output, fp32 accumulation in k order.
__global__ __launch_bounds__(256) void bgemm_simple(int ta, int tb, int M, int N, int K,
                                                    float alpha, const uint16_t* __restrict__ A,
                                                    int64_t lda, int64_t sA,
                                                    const uint16_t* __restrict__ B, int64_t ldb,
                                                    int64_t sB, float beta,
                                                    uint16_t* __restrict__ C, int64_t ldc,
                                                    int64_t sC) {
  const int col = blockIdx.x * 16 + (threadIdx.x & 15);
  const int row = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int b = blockIdx.z;
  if (row >= M || col >= N) return;
  const uint16_t* Ab = A + b * sA;
  const uint16_t* Bb = B + b * sB;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const float a = hk::bf16_to_f32(ta ? Ab[static_cast<int64_t>(k) * lda + row]
                                       : Ab[static_cast<int64_t>(row) * lda + k]);
    const float v = hk::bf16_to_f32(tb ? Bb[static_cast<int64_t>(col) * ldb + k]
                                       : Bb[static_cast<int64_t>(k) * ldb + col]);
    acc += a * v;
  }
  uint16_t* dst = C + b * sC + static_cast<int64_t>(row) * ldc + col;
  float f = alpha * acc;
  if (beta != 0.0f) f += beta * hk::bf16_to_f32(*dst);
  *dst = hk::f32_to_bf16(f);
}

float bf16_bits_to_float(hk_bf16 h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

template <bool AK, bool BKM, bool P>
hipError_t launch_tiled(dim3 grid, hipStream_t stream, int M, int N, int K, float alpha,
                        const uint16_t* A, int64_t lda, int64_t sA, const uint16_t* B,
                        int64_t ldb, int64_t sB, float beta, uint16_t* C, int64_t ldc,
                        int64_t sC, int split_k, int kps, float* part) {
  static std::once_flag once;
  static hipError_t attr_status = hipSuccess;
  std::call_once(once, [] {
    attr_status = hipFuncSetAttribute(reinterpret_cast<const void*>(&bgemm_tiled<AK, BKM, P>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLdsBytes));
  });
  HK_RETURN_IF_ERROR(attr_status);
  hipLaunchKernelGGL((bgemm_tiled<AK, BKM, P>), grid, dim3(kThreads), kLdsBytes, stream, M, N, K,
                     alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, split_k, kps, part);
  return hk::launch_status();
}

template <bool P>
hipError_t dispatch_layout(bool ta, bool tb, dim3 grid, hipStream_t stream, int M, int N, int K,
                           float alpha, const uint16_t* A, int64_t lda, int64_t sA,
                           const uint16_t* B, int64_t ldb, int64_t sB, float beta, uint16_t* C,
                           int64_t ldc, int64_t sC, int split_k, int kps, float* part) {
  // A is k-major unless transposed; B is k-major only when transposed.
  if (!ta && !tb)
    return launch_tiled<true, false, P>(grid, stream, M, N, K, alpha, A, lda, sA, B, ldb, sB,
                                        beta, C, ldc, sC, split_k, kps, part);
  if (!ta && tb)
    return launch_tiled<true, true, P>(grid, stream, M, N, K, alpha, A, lda, sA, B, ldb, sB,
                                       beta, C, ldc, sC, split_k, kps, part);
  if (ta && !tb)
    return launch_tiled<false, false, P>(grid, stream, M, N, K, alpha, A, lda, sA, B, ldb, sB,
                                         beta, C, ldc, sC, split_k, kps, part);
  return launch_tiled<false, true, P>(grid, stream, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta,
                                      C, ldc, sC, split_k, kps, part);
}

hipError_t bgemm_run(int transA, int transB, int M, int N, int K, hk_bf16 alpha_bits,
                     const hk_bf16* A, int lda, long long strideA, const hk_bf16* B, int ldb,
                     long long strideB, hk_bf16 beta_bits, hk_bf16* C, int ldc, long long strideC,
                     int batchCount, int splitK, hipStream_t stream) {
  HK_CHECK_ARG(transA >= 0 && transA <= 2 && transB >= 0 && transB <= 2);
  HK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batchCount >= 0 && splitK >= 1);
  if (M == 0 || N == 0 || batchCount == 0) return hipSuccess;
  HK_CHECK_ARG(C != nullptr && ldc >= N);
  const bool ta = transA != 0, tb = transB != 0;  // OP_C is OP_T for real bf16
  HK_CHECK_ARG(K == 0 || (A != nullptr && B != nullptr));
  HK_CHECK_ARG(lda >= (ta ? M : K) && ldb >= (tb ? K : N));
  const float alpha = bf16_bits_to_float(alpha_bits);
  const float beta = bf16_bits_to_float(beta_bits);

  const int contig_a = ta ? M : K, contig_b = tb ? K : N;
  const bool tiled_ok = (contig_a % 8 == 0) && (contig_b % 8 == 0) && (N % 8 == 0) &&
                        (lda % 8 == 0) && (ldb % 8 == 0) && (ldc % 8 == 0) &&
                        (strideA % 8 == 0) && (strideB % 8 == 0) && (strideC % 8 == 0) &&
                        hk::aligned16(A) && hk::aligned16(B) && hk::aligned16(C) && K > 0;
  if (!tiled_ok) {
    if (K == 0) splitK = 1;
    dim3 grid((N + 15) / 16, (M + 15) / 16, batchCount);
    hipLaunchKernelGGL(bgemm_simple, grid, dim3(256), 0, stream, ta ? 1 : 0, tb ? 1 : 0, M, N,
                       K, alpha, A, static_cast<int64_t>(lda), static_cast<int64_t>(strideA), B,
                       static_cast<int64_t>(ldb), static_cast<int64_t>(strideB), beta, C,
                       static_cast<int64_t>(ldc), static_cast<int64_t>(strideC));
    return hk::launch_status();
  }
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  HK_CHECK_ARG(tiles <= INT32_MAX && static_cast<int64_t>(batchCount) * splitK <= 65535);
  if (splitK == 1) {
    dim3 grid(static_cast<unsigned>(tiles), 1, batchCount);
    return dispatch_layout<false>(ta, tb, grid, stream, M, N, K, alpha, A, lda, strideA, B, ldb,
                                  strideB, beta, C, ldc, strideC, 1, K, nullptr);
  }
  // k range per split rounded to the k-tile
  const int kps = static_cast<int>(hk::ceil_div(hk::ceil_div(K, splitK), BK) * BK);
  const int used = static_cast<int>(hk::ceil_div(K, kps));
  void* ws = nullptr;
  const size_t part_bytes = static_cast<size_t>(used) * batchCount * M * N * sizeof(float);
  HK_RETURN_IF_ERROR(hk::device_workspace(part_bytes, &ws));
  float* part = static_cast<float*>(ws);
  dim3 grid(static_cast<unsigned>(tiles), 1, batchCount * used);
  HK_RETURN_IF_ERROR(dispatch_layout<true>(ta, tb, grid, stream, M, N, K, alpha, A, lda, strideA,
                                           B, ldb, strideB, beta, C, ldc, strideC, used, kps,
                                           part));
  const int64_t total = static_cast<int64_t>(M) * N * batchCount;
  hipLaunchKernelGGL(bgemm_splitk_finalize, dim3(static_cast<unsigned>(hk::ceil_div(total, 256))),
                     dim3(256), 0, stream, part, used, batchCount, M, N, alpha, beta, C,
                     static_cast<int64_t>(ldc), static_cast<int64_t>(strideC));
  return hk::launch_status();
}

}  // namespace

extern "C" hipError_t hk_bgemm(int transA, int transB, int M, int N, int K, hk_bf16 alpha,
                               const hk_bf16* A, int lda, long long strideA, const hk_bf16* B,
                               int ldb, long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                               long long strideC, int batchCount, hipStream_t stream) {
  return bgemm_run(transA, transB, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc,
                   strideC, batchCount, 1, stream);
}

extern "C" hipError_t hk_bgemm_core(int layout, int splitK, int M, int N, int K, hk_bf16 alpha,
                                    const hk_bf16* A, int lda, long long strideA,
                                    const hk_bf16* B, int ldb, long long strideB, hk_bf16 beta,
                                    hk_bf16* C, int ldc, long long strideC, int batchCount,
                                    hipStream_t stream) {
  // BgemmLayout { NT, TN, NN } (blas/bf16/bgemm_core_template.cu:59)
  HK_CHECK_ARG(layout >= HK_LAYOUT_NT && layout <= HK_LAYOUT_NN);
  const int ta = layout == HK_LAYOUT_TN ? 1 : 0;
  const int tb = layout == HK_LAYOUT_NT ? 1 : 0;
  return bgemm_run(ta, tb, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc,
                   strideC, batchCount, splitK, stream);
}

extern "C" hipError_t hk_bgemm_nt_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                           int lda, long long strideA, const hk_bf16* B, int ldb,
                                           long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                           long long strideC, int batchCount,
                                           hipStream_t stream) {
  return bgemm_run(0, 1, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                   batchCount, 1, stream);
}

extern "C" hipError_t hk_bgemm_tn_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                           int lda, long long strideA, const hk_bf16* B, int ldb,
                                           long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                           long long strideC, int batchCount,
                                           hipStream_t stream) {
  return bgemm_run(1, 0, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                   batchCount, 1, stream);
}
