// sgemm.hip - batched FP32 GEMM on gfx950 (bf16x3 split or fp32 MFMA) with split-K and a fused
// bias epilogue.
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
// The reference multiplies with single-pass TF32 MMA; gfx950 has no TF32 matrix instruction.
// Two paths:
//   bf16x3 (shapes whose dimensions are multiples of 8, the common case): A and B are split into
//     bf16 hi / lo operands over a tripled k axis (split3) so that one bf16 GEMM on the BF16 GEMM
//     tiles of this library (bgemm.hip) sums ah bh + ah bl + al bh in fp32. With one k split
//     the GEMM tiles apply alpha, beta and the bias and write C; with more, the split-K
//     finalize below does. Relative error ~1e-5 (max-rel 3e-6 at 4096^3 against a float64
//     product) at bf16 MFMA rate: 4096^3 + bias in ~0.39 ms against ~1.17 ms on the fp32
//     MFMA. Roofline: the bf16 peak / 3 (three products per fp32 product).
//   fp32 MFMA tiles (other 4-element-aligned shapes): v_mfma_f32_32x32x2_f32, exact fp32
//     products; roofline the fp32 matrix peak (157.3 TFLOP/s).
//
// Design of the fp32 tiles (gfx950): the same tiling as the BF16 GEMM of this library - 256 x 256 workgroup
// tile, 8 waves of 128 x 64 (2 x 4, two per SIMD; 4 x 2 MFMA tiles, 128 fp32 accumulators per
// lane; with 4 waves of 128 x 128 the 256 accumulators spilled), k-tiles of
// 32 fp32 copied HBM/L2 -> LDS without passing through registers (global_load_lds_dwordx4)
// into a 2-stage LDS ring, one barrier per k-tile. K-major operands sit in LDS as [row][k]
// (read 4 k at a time with 16-byte reads), M/N-major ones as [k][row] like in HBM (one float
// per lane and MFMA step, 128 contiguous bytes per half-wave), so no layout is transposed in
// registers. Lane (r, h) of a wave feeds k = 16h + s of each 32-deep k-tile at step s.
// The epilogue writes straight from registers: with the MFMA inputs swapped each lane holds 4
// consecutive columns of one output row per accumulator quad (one 16-byte store).
// Split-K: every split writes fp32 partials; a second kernel sums them in split order and
// applies alpha, beta and the bias exactly once (deterministic, and the bias is not repeated
// per split as in the reference's atomics).
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int kStages = 2;                             // LDS ring depth (k-tiles)
constexpr int kWaves = 8;                              // 2 x 4 over the tile, 2 per SIMD
constexpr int kThreads = kWaves * 64;
constexpr int kWaveM = 128, kWaveN = 64;               // 4 x 2 MFMA tiles of 32 x 32 per wave
constexpr int kBlkM = kWaveM / 32, kBlkN = kWaveN / 32;
constexpr int kStageBytes = 256 * BK * 4;              // one operand, one k-tile (32 KiB)
constexpr int kLoadsPerWave = kStageBytes / 1024 / kWaves;  // 16-byte lane copies per operand per wave
constexpr size_t kLdsBytes = static_cast<size_t>(kStages) * 2 * kStageBytes;  // 128 KiB

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
#define HK_LDS __attribute__((address_space(3)))

// 16-byte global -> LDS copy of one lane (global_load_lds_dwordx4); the wave's 64 lanes write
// 1 KiB at m0 + 16 * lane. Inline asm so that the compiler does not make every later LDS read
// wait for all outstanding copies (the kernel orders them itself with vmcnt + barrier).
// Address = sbase (wave-uniform 64-bit) + voff (per-lane byte offset).
__device__ __forceinline__ void copy16_to_lds(const void* sbase, int voff, unsigned lds_addr) {
  // m0 (the LDS destination) is an input operand, so the compiler knows the asm sets it. Its
  // hazard checks do not see inside the asm, so the asm supplies the wait states itself: an
  // SALU write of m0 needs 1 before an LDS-DMA load, and an SGPR of sbase written by a VALU
  // (v_readlane, when the compiler reloads a spilled SGPR) needs 5 before a VMEM read of it.
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "{m0}"(lds_addr));
}

// One operand of a k-tile in LDS: 256 rows of M (or N) by BK = 32 k, fp32, 32 KiB.
// gfx950's LDS has 64 banks of 4 bytes and serves 256 bytes per cycle: 16 lanes of a 16-byte
// read, 64 lanes of a 4-byte read. Each such lane group must cover the 64 banks once.
//
// K-major operands (element (row, k) at base[row * ld + k]) are stored [row][32 k]: 128-byte
// rows whose 16-byte chunks (4 k each) sit at chunk ^ ((row >> 1) & 7); a copy instruction
// moves 8 rows (lane l: row l / 8, stored chunk l % 8), 8 lanes per 128-byte HBM row segment.
// Lane (r, h) of a wave feeds k = 16 h + s of the tile at MFMA step s, so it reads 16
// consecutive k of its row as four 16-byte LDS reads (chunks 4 h .. 4 h + 3); 16 consecutive
// rows at one chunk: the even rows fill one bank half at 8 distinct positions, the odd rows
// the other.
// M/N-major operands (element at base[k * ld + row]) are stored as in HBM, [32 k][256 rows]
// (1 KiB per k-row, one copy instruction), with the 16-byte chunks of k-rows 16 .. 31 at
// chunk ^ 8; the operand of MFMA step s is one float per lane, row k = 16 h + s, 32
// consecutive rows per half-wave, the two half-waves in opposite bank halves.
template <bool KMAJOR>
struct TileOperand {
  __device__ static void source(int ii, int lane, int& row, int& k) {
    if (KMAJOR) {
      row = ii * 8 + (lane >> 3);
      k = ((lane & 7) ^ ((row >> 1) & 7)) * 4;
    } else {
      k = ii;
      row = (lane ^ (8 * ((k >> 4) & 1))) * 4;
    }
  }
  __device__ static int64_t byte_offset(int row, int k, int64_t ld) {
    return KMAJOR ? 4 * (static_cast<int64_t>(row) * ld + k)
                  : 4 * (static_cast<int64_t>(k) * ld + row);
  }
  __device__ static int64_t ktile_step(int64_t ld) { return KMAJOR ? BK : BK * ld; }
  // Operands of MFMA steps 4 qd .. 4 qd + 3 for MFMA block b (32 rows at wave offset wo).
  __device__ static f32x4_t read(const unsigned char HK_LDS* st, int wo, int b, int qd,
                                 int lane) {
    const int r = wo + b * 32 + (lane & 31), h = lane >> 5;
    if (KMAJOR) {
      const int c = 4 * h + qd;
      return *reinterpret_cast<const f32x4_t HK_LDS*>(st + r * 128 +
                                                      ((c ^ ((r >> 1) & 7)) * 16));
    } else {
      // k-rows 16 h + 4 qd .. +3 all lie in one half (h), so one chunk flip serves the four
      const int rs = r ^ (32 * h);
      const float HK_LDS* col =
          reinterpret_cast<const float HK_LDS*>(st) + (16 * h + 4 * qd) * 256 + rs;
      return f32x4_t{col[0], col[256], col[512], col[768]};
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

__device__ __forceinline__ float f4_get(const f32x4_t& v, int e) { return v[e]; }

// 8 MFMAs (4 x 2 blocks) per k step, 4 k steps; B block as the MFMA "A" input so that each
// lane ends up holding 4 consecutive output columns of one output row per accumulator quad.
__device__ __forceinline__ void mma_quad(const f32x4_t (&af)[kBlkM], const f32x4_t (&bf)[kBlkN],
                                         f32x16_t (&acc)[kBlkM][kBlkN]) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < kBlkM; ++i)
#pragma unroll
      for (int j = 0; j < kBlkN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f4_get(bf[j], e), f4_get(af[i], e),
                                                         acc[i][j], 0, 0, 0);
}

// Main loop per k-tile kt (ring slot kt % 2) in 4 quads of 4 MFMA steps (32 MFMAs each):
// quads 0-2 read the operands of the next quad while multiplying; quad 3 waits for this
// wave's copies of tile kt + 1, takes the barrier, reads quad 0 of tile kt + 1 and issues the
// copies of tile kt + 2 into slot kt % 2 between its MFMAs.
template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL>
__global__ __launch_bounds__(kThreads, 1) void sgemm_tiled(
    int M, int N, int K, const float* __restrict__ A, int64_t lda, int64_t sA,
    const float* __restrict__ B, int64_t ldb, int64_t sB, float* __restrict__ C, int64_t ldc,
    int64_t sC, Epilogue ep, int split_k, int k_per_split, float* __restrict__ part) {
  using OA = TileOperand<A_KMAJOR>;
  using OB = TileOperand<B_KMAJOR>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  unsigned char HK_LDS* ldsA = (unsigned char HK_LDS*)lds_raw;
  unsigned char HK_LDS* ldsB = ldsA + kStages * kStageBytes;

  const int batch = blockIdx.z / split_k;
  const int split = blockIdx.z - batch * split_k;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * k_per_split;
  const int klen = min(K, kbeg + k_per_split) - kbeg;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // Rows past M (N) are read clamped (their outputs are not stored); k past the split's end is
  // zero-filled on the last k-tile.
  const unsigned char* gA = reinterpret_cast<const unsigned char*>(
      A + static_cast<int64_t>(batch) * sA +
      (A_KMAJOR ? static_cast<int64_t>(m0) * lda + kbeg : static_cast<int64_t>(kbeg) * lda + m0));
  const unsigned char* gB = reinterpret_cast<const unsigned char*>(
      B + static_cast<int64_t>(batch) * sB +
      (B_KMAJOR ? static_cast<int64_t>(n0) * ldb + kbeg : static_cast<int64_t>(kbeg) * ldb + n0));
  int offA[kLoadsPerWave], offB[kLoadsPerWave], kA[kLoadsPerWave], kB[kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    int row, k;
    OA::source(wave * kLoadsPerWave + i, lane, row, k);
    row = min(row, (A_KMAJOR ? M - 1 : M - 4) - m0);
    offA[i] = static_cast<int>(OA::byte_offset(row, k, lda));
    kA[i] = k;
    OB::source(wave * kLoadsPerWave + i, lane, row, k);
    row = min(row, (B_KMAJOR ? N - 1 : N - 4) - n0);
    offB[i] = static_cast<int>(OB::byte_offset(row, k, ldb));
    kB[i] = k;
  }
  const int64_t stepA = 4 * OA::ktile_step(lda), stepB = 4 * OB::ktile_step(ldb);
  const unsigned ldsA_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ldsA));
  const unsigned ldsB_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ldsB));
  const int ktiles = (klen + BK - 1) / BK;
  const bool tail = (klen % BK) != 0;

  auto copy = [&](int kt, int slot, int q, bool fill) {
    const bool isA = q < kLoadsPerWave;
    const int i = isA ? q : q - kLoadsPerWave;
    const unsigned char* base = (isA ? gA + kt * stepA : gB + kt * stepB);
    const int off = isA ? offA[i] : offB[i];
    const unsigned lds = (isA ? ldsA_addr : ldsB_addr) + slot * kStageBytes +
                         (wave * kLoadsPerWave + i) * 1024;
    if (!fill) {
      copy16_to_lds(base, off, lds);
    } else if (kt * BK + (isA ? kA[i] : kB[i]) < klen) {
      copy16_to_lds(base, off, lds);
    } else {
      typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
      *reinterpret_cast<u32x4_t HK_LDS*>((unsigned char HK_LDS*)(uintptr_t)lds + 16 * lane) =
          u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  constexpr int kCopies = 2 * kLoadsPerWave;

  f32x16_t acc[kBlkM][kBlkN];
#pragma unroll
  for (int i = 0; i < kBlkM; ++i)
#pragma unroll
    for (int j = 0; j < kBlkN; ++j) acc[i][j] = f32x16_t{};

#pragma unroll
  for (int p = 0; p < kStages; ++p)
    if (p < ktiles) {
      const bool fill = tail && p == ktiles - 1;
#pragma unroll
      for (int q = 0; q < kCopies; ++q) copy(p, p, q, fill);
    }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();

  f32x4_t fa[2][kBlkM], fb[2][kBlkN];
  if (ktiles > 0) {
#pragma unroll
    for (int i = 0; i < kBlkM; ++i) fa[0][i] = OA::read(ldsA, wm * kWaveM, i, 0, lane);
#pragma unroll
    for (int j = 0; j < kBlkN; ++j) fb[0][j] = OB::read(ldsB, wn * kWaveN, j, 0, lane);
  }

  for (int kt = 0; kt < ktiles; ++kt) {
    const int slot = kt & 1;
    const unsigned char HK_LDS* sa = ldsA + slot * kStageBytes;
    const unsigned char HK_LDS* sb = ldsB + slot * kStageBytes;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int cur = qd & 1, nxt = cur ^ 1;
      if (qd + 1 < 4) {
#pragma unroll
        for (int i = 0; i < kBlkM; ++i) fa[nxt][i] = OA::read(sa, wm * kWaveM, i, qd + 1, lane);
#pragma unroll
        for (int j = 0; j < kBlkN; ++j) fb[nxt][j] = OB::read(sb, wn * kWaveN, j, qd + 1, lane);
        mma_quad(fa[cur], fb[cur], acc);
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < ktiles) {
          const unsigned char HK_LDS* na = ldsA + (slot ^ 1) * kStageBytes;
          const unsigned char HK_LDS* nb = ldsB + (slot ^ 1) * kStageBytes;
#pragma unroll
          for (int i = 0; i < kBlkM; ++i) fa[nxt][i] = OA::read(na, wm * kWaveM, i, 0, lane);
#pragma unroll
          for (int j = 0; j < kBlkN; ++j) fb[nxt][j] = OB::read(nb, wn * kWaveN, j, 0, lane);
        }
        const bool more = kt + kStages < ktiles;
        const bool fill = tail && kt + kStages == ktiles - 1;
        // 32 MFMAs with the 8 copies of tile kt + 2 spread between them
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < kBlkM; ++i)
#pragma unroll
            for (int j = 0; j < kBlkN; ++j) {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                  f4_get(fb[cur][j], e), f4_get(fa[cur][i], e), acc[i][j], 0, 0, 0);
              const int q = (e * kBlkM + i) * kBlkN + j;
              if (more && (q & 3) == 0 && (q >> 2) < kCopies) copy(kt + kStages, slot, q >> 2, fill);
            }
      }
    }
  }

  // Epilogue. Lane l holds, for MFMA block (i, j) and quad q, output row
  // wm*128 + 32 i + l % 32 and columns wn*64 + 32 j + 8 q + 4 (l / 32) .. +3.
  const int row0 = m0 + wm * kWaveM + (lane & 31);
  const int col0 = n0 + wn * kWaveN + 4 * (lane >> 5);
  if (PARTIAL) {
    float* out = part + (static_cast<int64_t>(split) * (gridDim.z / split_k) + batch) *
                            static_cast<int64_t>(M) * N;
#pragma unroll
    for (int i = 0; i < kBlkM; ++i) {
      const int row = row0 + 32 * i;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < kBlkN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = col0 + 32 * j + 8 * q;
          if (col < N)
            *reinterpret_cast<float4*>(out + static_cast<int64_t>(row) * N + col) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                            acc[i][j][4 * q + 3]);
        }
    }
    return;
  }
  float* Cb = C + static_cast<int64_t>(batch) * sC;
#pragma unroll
  for (int i = 0; i < kBlkM; ++i) {
    const int row = row0 + 32 * i;
    if (row >= M) continue;
    float* crow = Cb + static_cast<int64_t>(row) * ldc;
#pragma unroll
    for (int j = 0; j < kBlkN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = col0 + 32 * j + 8 * q;
        if (col >= N) continue;
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = ep.alpha * acc[i][j][4 * q + e];
        float4* dst = reinterpret_cast<float4*>(crow + col);
        if (ep.beta != 0.0f) {
          const float4 o = *dst;
          f[0] += ep.beta * o.x;
          f[1] += ep.beta * o.y;
          f[2] += ep.beta * o.z;
          f[3] += ep.beta * o.w;
        }
        if (ep.bias) {
#pragma unroll
          for (int e = 0; e < 4; ++e) f[e] += ep.bias_scale * bias_at(ep, M, N, batch, col + e);
        }
        *dst = make_float4(f[0], f[1], f[2], f[3]);
      }
  }
}

// C = alpha * (sum of the split partials, in split order) + beta * C + bias, four consecutive
// outputs per thread (N % 4 == 0 on the tiled paths). I: the index type, uint32_t when every
// index of the launch fits in 31 bits (a 64-bit division costs several times a 32-bit one).
template <typename I>
__global__ __launch_bounds__(256) void sgemm_splitk_finalize(const float* __restrict__ part,
                                                             int split_k, int batch, int M, int N,
                                                             float* __restrict__ C, int64_t ldc,
                                                             int64_t sC, Epilogue ep) {
  const I idx = (static_cast<I>(blockIdx.x) * 256 + threadIdx.x) * 4;
  const I mn = static_cast<I>(M) * N;
  if (idx >= mn * batch) return;
  const I b = idx / mn;
  const I e = idx - b * mn;
  const I row = e / N, col = e - row * N;
  // The partials are read once: non-temporal loads (4096^3 at split-K 4: 487.5 -> 479.7 us for
  // the whole call). One partial at a time, in split order.
  f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < split_k; ++k)
    s += __builtin_nontemporal_load(
        reinterpret_cast<const f32x4_t*>(part + (static_cast<int64_t>(k) * batch + b) * mn + e));
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(C + b * sC + static_cast<int64_t>(row) * ldc + col);
  f32x4_t f = ep.alpha * s;
  if (ep.beta != 0.0f) f += ep.beta * *dst;
  if (ep.bias) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      f[i] += ep.bias_scale * bias_at(ep, M, N, static_cast<int>(b), static_cast<int>(col) + i);
  }
  *dst = f;
}

hipError_t launch_finalize(hipStream_t stream, const float* part, int used, int batch, int M,
                           int N, float* C, int64_t ldc, int64_t sC, const Epilogue& ep) {
  const int64_t total = static_cast<int64_t>(M) * N * batch / 4;
  const dim3 grid(static_cast<unsigned>(hk::ceil_div(total, 256)));
  if (static_cast<int64_t>(M) * N * batch < (int64_t{1} << 31))
    hipLaunchKernelGGL(sgemm_splitk_finalize<uint32_t>, grid, dim3(256), 0, stream, part, used,
                       batch, M, N, C, ldc, sC, ep);
  else
    hipLaunchKernelGGL(sgemm_splitk_finalize<int64_t>, grid, dim3(256), 0, stream, part, used,
                       batch, M, N, C, ldc, sC, ep);
  return hk::launch_status();
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

// bf16x3 operand of an fp32 matrix X (rows x cols, leading dimension ldx, batch stride sx):
// each x = hi + lo (bf16, round to nearest even, |x - hi - lo| <= 2^-18 |x|) and the k axis is
// tripled into three segments, (hi, hi', lo) for the left operand and (hi, lo, hi') for the
// right, so that a bf16 GEMM over 3K sums ah bh + ah' bl + al bh'. KCOLS: k runs along the
// columns (Y[r][s cols + c]); otherwise along the rows (Y[s rows + r][c]). Four columns per
// thread (cols % 4 == 0, 16-byte aligned rows): one 16-byte load, three 8-byte stores; batch b
// in blockIdx.y and a 32-bit index within one matrix (rows * cols / 4 < 2^31, checked by the
// host). Runs at copy rate (a measured ~6.8 TB/s for 4096 x 4096).
// Non-finite x (inf, NaN): hi carries it, lo and hi' (the copy of hi in the cross term) are 0.
// The cross terms of its products are then 0 and the product is hi * bh alone, +-inf or NaN as
// the reference's TF32 product is; with lo = bf16(x - hi) and hi' = hi they would add inf * bl
// (NaN for bl = 0 or of the other sign) and bf16(inf - inf) = NaN. A finite x that rounds past
// bf16's largest value (|x| > (2 - 2^-8) 2^127) keeps hi = +-that largest value and
// lo = bf16(x - hi), so it stays finite as it does in TF32 (whose range is fp32's).
// One operand: X (rows x cols, leading dimension ldx, batch stride sx) -> Y (ldy, sy).
struct Split3Op {
  const float* X;
  int64_t ldx, sx;
  int rows, cols;
  uint16_t* Y;
  int64_t ldy, sy;
};
// Element group i (four columns) of batch b. X is read once, with non-temporal loads.
template <bool KCOLS>
__device__ __forceinline__ void split3_group(const Split3Op& o, unsigned i, int64_t b, int left) {
  const unsigned c4 = static_cast<unsigned>(o.cols) >> 2;
  if (i >= static_cast<unsigned>(o.rows) * c4) return;
  const unsigned r = i / c4, c = (i - r * c4) * 4;
  const f32x4_t v = __builtin_nontemporal_load(
      reinterpret_cast<const f32x4_t*>(o.X + b * o.sx + static_cast<int64_t>(r) * o.ldx + c));
  const int rows = o.rows, cols = o.cols;
  const int64_t ldy = o.ldy;
  uint16_t h[4], l[4], hc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    h[k] = hk::f32_to_bf16(v[k]);
    const bool x_finite = (__float_as_uint(v[k]) & 0x7f800000u) != 0x7f800000u;
    if (x_finite && (h[k] & 0x7f80u) == 0x7f80u) h[k] = (h[k] & 0x8000u) | 0x7f7fu;
    const bool finite = (h[k] & 0x7f80u) != 0x7f80u;
    l[k] = finite ? hk::f32_to_bf16(v[k] - hk::bf16_to_f32(h[k])) : uint16_t{0};
    hc[k] = finite ? h[k] : uint16_t{0};
  }
  auto pack = [](const uint16_t (&e)[4]) {
    return make_uint2(e[0] | (static_cast<uint32_t>(e[1]) << 16),
                      e[2] | (static_cast<uint32_t>(e[3]) << 16));
  };
  const uint2 H = pack(h), L = pack(l), Hc = pack(hc);
  uint16_t* Yb = o.Y + b * o.sy;
  const uint2 seg[3] = {H, left ? Hc : L, left ? L : Hc};
#pragma unroll
  for (int sg = 0; sg < 3; ++sg) {
    uint16_t* dst = KCOLS ? Yb + static_cast<int64_t>(r) * ldy + sg * cols + c
                          : Yb + (static_cast<int64_t>(sg) * rows + r) * ldy + c;
    *reinterpret_cast<uint2*>(dst) = seg[sg];
  }
}
// Both operands in one launch: blocks below nblk_a split A (the left operand), the rest B;
// batch in blockIdx.y. KA / KB: k runs along the columns of A / B. One launch instead of two
// and the non-temporal input loads: 4096^3 + bias 392 -> 386 us at the library's split and
// 495 -> 491 us at split-K 4 (same run, bit-equal).
template <bool KA, bool KB>
__global__ __launch_bounds__(256) void split3(Split3Op a, Split3Op bop, unsigned nblk_a) {
  const int64_t b = blockIdx.y;
  if (blockIdx.x < nblk_a)
    split3_group<KA>(a, blockIdx.x * 256u + threadIdx.x, b, 1);
  else
    split3_group<KB>(bop, (blockIdx.x - nblk_a) * 256u + threadIdx.x, b, 0);
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

// The three product paths of an fp32 GEMM and the k-split plan each runs.
enum class SgemmPath { kSimple, kBf16x3, kFp32Tiles };

// Which path takes a product. Tiles: 4-element multiples for every contiguous extent, leading
// dimension and batch stride, 16-byte aligned bases. bf16x3 additionally needs every dimension
// the split copies touch to be a multiple of 8 and the tripled k axis to fit the BF16 tiles'
// 32-bit per-lane offsets.
SgemmPath sgemm_path(bool ta, bool tb, int M, int N, int K, int64_t lda, int64_t ldb,
                     int64_t ldc, int64_t sA, int64_t sB, int64_t sC, int batchCount,
                     bool aligned) {
  const int contig_a = ta ? M : K, contig_b = tb ? K : N;
  const bool tiled_ok = (contig_a % 4 == 0) && (contig_b % 4 == 0) && (N % 4 == 0) &&
                        (lda % 4 == 0) && (ldb % 4 == 0) && (ldc % 4 == 0) && (sA % 4 == 0) &&
                        (sB % 4 == 0) && (sC % 4 == 0) && aligned && K > 0 &&
                        // per-lane source offsets inside a tile are 32-bit byte offsets
                        lda < (1 << 21) && ldb < (1 << 21);
  if (!tiled_ok) return SgemmPath::kSimple;
  const bool x3_ok = K % 8 == 0 && N % 8 == 0 && (!ta || M % 8 == 0) &&
                     3LL * K < (1 << 22) && (ta ? M : 3LL * K) < (1 << 22) &&
                     (tb ? 3LL * K : N) < (1 << 22) && batchCount <= 65535 &&
                     static_cast<int64_t>(M) * K < (int64_t{1} << 33) &&
                     static_cast<int64_t>(K) * N < (int64_t{1} << 33);
  return x3_ok ? SgemmPath::kBf16x3 : SgemmPath::kFp32Tiles;
}

// k-split plan of the fp32 MFMA tiles (BK = 32 fp32 per k-tile): split_k ranges of kps k, the
// `used` non-empty ones run (split_k == 0: the library's choice, the BF16 tiles' cost model on
// this path's k-tiles).
void fp32_split_plan(int M, int N, int K, int batch, int split_k, int* used, int* kps) {
  int s = split_k;
  if (s == 0) {
    int u = 1, kp = 0;
    // the BF16 planner counts 64-deep k-tiles: 2 K of them are this path's 32-deep ones
    hk::bgemm_split_plan(M, N, 2 * K, batch, 0, &u, &kp);
    s = u;
  }
  *kps = static_cast<int>(hk::ceil_div(hk::ceil_div(K, s), BK) * BK);
  *used = static_cast<int>(hk::ceil_div(K, *kps));
}

hipError_t sgemm_run(bool ta, bool tb, int M, int N, int K, float alpha, const float* A, int lda,
                     long long strideA, const float* B, int ldb, long long strideB, float beta,
                     float* C, int ldc, long long strideC, const float* bias,
                     long long bias_stride, float bias_scale, int batchCount, int splitK,
                     hipStream_t stream) {
  // splitK == 0: the library picks the split; otherwise K is cut into splitK ranges (rounded
  // to the k-tile) whose fp32 partials are summed in split order
  HK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batchCount >= 0 && splitK >= 0);
  if (M == 0 || N == 0 || batchCount == 0) return hipSuccess;
  HK_CHECK_ARG(C != nullptr && ldc >= N);
  HK_CHECK_ARG(K == 0 || (A != nullptr && B != nullptr));
  HK_CHECK_ARG(lda >= (ta ? M : K) && ldb >= (tb ? K : N));
  if (bias) {
    HK_CHECK_ARG(bias_stride == N || bias_stride == static_cast<long long>(M) * N ||
                 bias_stride == 1);
  }
  const Epilogue ep{alpha, beta, bias, bias ? static_cast<int64_t>(bias_stride) : 0, bias_scale};
  const SgemmPath path = sgemm_path(ta, tb, M, N, K, lda, ldb, ldc, strideA, strideB, strideC,
                                    batchCount,
                                    hk::aligned16(A) && hk::aligned16(B) && hk::aligned16(C));
  if (path == SgemmPath::kSimple) {
    dim3 grid((N + 15) / 16, (M + 15) / 16, batchCount);
    hipLaunchKernelGGL(sgemm_simple, grid, dim3(256), 0, stream, ta ? 1 : 0, tb ? 1 : 0, M, N, K,
                       A, static_cast<int64_t>(lda), static_cast<int64_t>(strideA), B,
                       static_cast<int64_t>(ldb), static_cast<int64_t>(strideB), C,
                       static_cast<int64_t>(ldc), static_cast<int64_t>(strideC), ep);
    return hk::launch_status();
  }
  // bf16x3 on the BF16 GEMM tiles when every dimension the split copies touch is a multiple
  // of 8: A and B are split into bf16 hi / lo operands over a tripled k axis and multiplied on
  // the BF16 GEMM tiles. With one k split the tiles write C (alpha, beta, bias) themselves;
  // with more, fp32 partials are finished (alpha, beta, bias once) by the split-K finalize.
  // The call's splitK cuts the tripled k axis into that many ranges (0: the library's choice).
  if (path == SgemmPath::kBf16x3) {
    const int K3 = 3 * K;
    // A' is [M][3K] (k-major) or [3K][M]; B' is [3K][N] or [N][3K]
    const int64_t la = ta ? M : K3, lb = tb ? K3 : N;
    const int64_t na = static_cast<int64_t>(M) * K3, nb = static_cast<int64_t>(K3) * N;
    int used = 1, kps = 0;
    hk::bgemm_split_plan(M, N, K3, batchCount, splitK, &used, &kps);
    // the plan never exceeds the k-tile count; refuse a grid the tiles cannot take before
    // anything is allocated or launched
    HK_CHECK_ARG(static_cast<int64_t>(batchCount) * used <= 65535);
    auto up = [](int64_t bytes) { return (bytes + 255) & ~int64_t{255}; };
    const int64_t a_bytes = up(na * batchCount * 2), b_bytes = up(nb * batchCount * 2);
    // Serial split-K: when the output tiles alone fill the device, concurrent k ranges add no
    // parallelism, so the ranges are added into C one after the other, in split order (the
    // first applies beta and the bias, the others beta = 1), with no fp32 partials and no
    // finalize pass. 4096^3 + bias at split-K 4: 489.7 -> 462.8 us, max-rel vs a float64
    // product 2.9e-6 both ways. Fewer tiles than CUs keep concurrent partials.
    const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const bool serial = used > 1 && tiles * batchCount >= hk::device_cu_count();
    // one split (or serial ranges): the GEMM tiles write C themselves, no partials
    const int64_t p_bytes =
        used == 1 || serial ? 0 : static_cast<int64_t>(used) * batchCount * M * N * 4;
    void* ws = nullptr;
    HK_RETURN_IF_ERROR(hk::device_workspace(static_cast<size_t>(a_bytes + b_bytes + p_bytes),
                                            stream, &ws));
    uint16_t* A3 = static_cast<uint16_t*>(ws);
    uint16_t* B3 = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + a_bytes);
    float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + a_bytes + b_bytes);
    // A and B (rows x cols as stored) in one launch; k runs along A's columns unless A is
    // transposed, along B's columns when B is
    {
      const int ra = ta ? K : M, ca = ta ? M : K, rb = tb ? N : K, cb = tb ? K : N;
      const Split3Op oa{A, static_cast<int64_t>(lda), static_cast<int64_t>(strideA), ra, ca,
                        A3, la, na};
      const Split3Op ob{B, static_cast<int64_t>(ldb), static_cast<int64_t>(strideB), rb, cb,
                        B3, lb, nb};
      const int64_t nba = hk::ceil_div(static_cast<int64_t>(ra) * (ca / 4), 256);
      const int64_t nbb = hk::ceil_div(static_cast<int64_t>(rb) * (cb / 4), 256);
      HK_CHECK_ARG(nba + nbb <= INT32_MAX);
      auto* k = !ta ? (tb ? split3<true, true> : split3<true, false>)
                    : (tb ? split3<false, true> : split3<false, false>);
      hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(nba + nbb), batchCount), dim3(256), 0,
                         stream, oa, ob, static_cast<unsigned>(nba));
      HK_RETURN_IF_ERROR(hk::launch_status());
    }
    const hk::F32Out out{C,        static_cast<int64_t>(ldc), static_cast<int64_t>(strideC),
                         ep.alpha, ep.beta, ep.bias, ep.bias_stride, ep.bias_scale};
    if (serial) {
      for (int r = 0; r < used; ++r) {
        // k range [k0, k0 + kr) of the tripled axis: columns of a k-major operand, rows else
        const int64_t k0 = static_cast<int64_t>(r) * kps;
        const int kr = static_cast<int>(K3 - k0 < kps ? K3 - k0 : kps);
        const uint16_t* Ar = A3 + (ta ? k0 * la : k0);
        const uint16_t* Br = B3 + (tb ? k0 : k0 * lb);
        hk::F32Out o = out;
        if (r > 0) {
          o.beta = 1.0f;
          o.bias = nullptr;
        }
        constexpr int kBf16KTile = 64;  // the BF16 tiles' k step: kps must be a multiple
        HK_RETURN_IF_ERROR(hk::bgemm_partials(
            ta, tb, M, N, kr, Ar, la, na, Br, lb, nb, batchCount, 1,
            (kr + kBf16KTile - 1) / kBf16KTile * kBf16KTile, nullptr, &o, stream));
      }
      return hipSuccess;
    }
    HK_RETURN_IF_ERROR(hk::bgemm_partials(ta, tb, M, N, K3, A3, la, na, B3, lb, nb, batchCount,
                                          used, kps, part, &out, stream));
    if (used == 1) return hipSuccess;
    return launch_finalize(stream, part, used, batchCount, M, N, C, static_cast<int64_t>(ldc),
                           static_cast<int64_t>(strideC), ep);
  }
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int used = 1, kps = K;
  fp32_split_plan(M, N, K, batchCount, splitK, &used, &kps);
  HK_CHECK_ARG(tiles <= INT32_MAX && static_cast<int64_t>(batchCount) * used <= 65535);
  if (used == 1) {
    dim3 grid(static_cast<unsigned>(tiles), 1, batchCount);
    return dispatch_layout<false>(ta, tb, grid, stream, M, N, K, A, lda, strideA, B, ldb, strideB,
                                  C, ldc, strideC, ep, 1, K, nullptr);
  }
  void* ws = nullptr;
  HK_RETURN_IF_ERROR(hk::device_workspace(
      static_cast<size_t>(used) * batchCount * M * N * sizeof(float), stream, &ws));
  float* part = static_cast<float*>(ws);
  dim3 grid(static_cast<unsigned>(tiles), 1, batchCount * used);
  HK_RETURN_IF_ERROR(dispatch_layout<true>(ta, tb, grid, stream, M, N, K, A, lda, strideA, B, ldb,
                                           strideB, C, ldc, strideC, ep, used, kps, part));
  return launch_finalize(stream, part, used, batchCount, M, N, C, static_cast<int64_t>(ldc),
                         static_cast<int64_t>(strideC), ep);
}

bool layout_trans(int layout, bool* ta, bool* tb) {
  if (layout < HK_LAYOUT_NT || layout > HK_LAYOUT_NN) return false;
  *ta = layout == HK_LAYOUT_TN;
  *tb = layout == HK_LAYOUT_NT;
  return true;
}

}  // namespace

extern "C" int hk_sgemm_split_count(int layout, int M, int N, int K, int batchCount, int splitK) {
  bool ta, tb;
  if (!layout_trans(layout, &ta, &tb) || M < 0 || N < 0 || K < 0 || batchCount < 0 || splitK < 0)
    return -1;
  if (M == 0 || N == 0 || batchCount == 0) return 0;
  const int64_t lda = ta ? M : K, ldb = tb ? K : N;
  const SgemmPath path = sgemm_path(ta, tb, M, N, K, lda, ldb, N, lda * (ta ? K : M),
                                    ldb * (tb ? N : K), static_cast<int64_t>(M) * N, batchCount,
                                    true);
  int used = 1, kps = 0;
  if (path == SgemmPath::kBf16x3)
    hk::bgemm_split_plan(M, N, 3 * K, batchCount, splitK, &used, &kps);
  else if (path == SgemmPath::kFp32Tiles)
    fp32_split_plan(M, N, K, batchCount, splitK, &used, &kps);
  return used;
}

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
                   strideC, bias, bias_numel, beta, batchCount, 0, stream);
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
