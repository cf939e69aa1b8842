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
//   - Workgroup tile 256 x 256, k-tile 64, 8 waves (2 x 4, two per SIMD); each wave owns a
//     128 x 64 block of C as 4 x 2 tiles of v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators
//     per lane). Per 16-deep k step a wave issues 8 MFMAs against 6 operand reads from LDS.
//     Two waves per SIMD let one issue MFMAs while the other waits on LDS or the barrier: 4-9%
//     faster than 4 waves of 128 x 128 at the BASELINE shapes and at 8192^3.
//   - HBM/L2 -> LDS copies bypass registers (global_load_lds_dwordx4, 16 bytes per lane) into
//     a 2-stage LDS ring: tile kt + 2 is copied while tile kt is multiplied, with one barrier
//     per k-tile. K-major operands are stored [row][k] and read with ds_read_b128; M/N-major
//     operands are stored as they lie in HBM, [k][row], and read with the gfx950 transposing
//     LDS read (ds_read_b64_tr_b16), so no layout needs a register transpose. The bank
//     placement of both is chosen through the per-lane source addresses of the copies.
//   - Operand reads of the next k step are interleaved with the current step's MFMAs
//     (sched_group_barrier), and the copies of the next tiles with the MFMAs of the last
//     step and of the first two.
//   - Epilogue through LDS: with the MFMA inputs swapped, each lane holds 4 consecutive
//     columns of one output row per accumulator quad; each wave stages its rows in LDS and
//     reads them back as 8 consecutive columns per lane. alpha / beta are applied in fp32 with
//     one rounding to bf16 (v_cvt_pk_bf16_f32, round to nearest even) and 16 bytes are stored
//     per lane, non-temporal (the reference rounds alpha * acc to bf16 and then blends beta * C
//     in bf16 arithmetic).
//   - Columns that would leave a last round of 256-wide tiles partly empty run as 128-wide
//     tiles in the same launch (column_split, bgemm_mixed).
//   - Edges: rows past M (N) are read clamped to the last row and their outputs are not
//     stored; k past the end of the (split's) range is zero-filled in LDS on the last k-tile.
//   - Workgroup order: consecutive tiles go to one XCD (the hardware deals workgroups to the 8
//     XCDs round-robin) in groups of 8 tile-rows, so each XCD's L2 sees a compact C region.
//   - Split-K (the core-template entry point with splitK > 1): each split writes fp32 partials
//     to the library workspace; a second kernel sums them in split order and applies
//     alpha/beta (deterministic; the reference accumulates with lossy bf16 atomics).
// Shapes the tiled kernel does not take (a contiguous extent or leading dimension that is not
// a multiple of 8, pointers not 16-byte aligned) run on a simple fp32-accumulating kernel.
#include <mutex>
#include <type_traits>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int BM = 256, BN = 256, BK = 64;             // BN: the full tile width
constexpr int kStages = 2;                             // LDS ring depth (k-tiles)
constexpr int kWaves = 8;                              // 2 x 4 over the tile, 2 per SIMD
constexpr int kThreads = kWaves * 64;

// Tile height BMT (256, or 192 for products whose 256-row tiles would leave many CUs idle, see
// row_tile; 192 only with a k-major A): each wave owns BMT / 2 rows of C, kBlkM MFMA tiles of
// 32 rows.
template <int BMT>
struct TileM {
  static_assert(BMT == 256 || BMT == 192, "tile heights");
  static constexpr int kWaveM = BMT / 2;
  static constexpr int kBlkM = kWaveM / 32;
  static constexpr int kStageBytes = BMT * BK * 2;                   // A, one k-tile
  static constexpr int kLoadsPerWave = kStageBytes / 1024 / kWaves;  // 16-byte lane copies of A
};

// Tile width BNT (256, or 128 for the half-width tiles that fill a last round, see
// column_split): each wave owns BMT / 2 x BNT / 4 of C, kBlkN MFMA tiles of 32 columns.
template <int BNT, int BMT = 256>
struct TileN {
  static constexpr int kWaveN = BNT / 4;
  static constexpr int kBlkN = kWaveN / 32;
  static constexpr int kStageBytesB = BNT * BK * 2;
  static constexpr int kLoadsB = kStageBytesB / 1024 / kWaves;
  static constexpr size_t kLdsBytes =
      static_cast<size_t>(kStages) * (TileM<BMT>::kStageBytes + kStageBytesB);
};

typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#define HK_LDS __attribute__((address_space(3)))

// 16-byte global -> LDS copy of one lane (global_load_lds_dwordx4): the wave's 64 lanes write
// 1 KiB of LDS at m0 + 16 * lane. Written as inline asm on purpose: for the builtin, the
// compiler assumes every later LDS read may alias the copy and waits for ALL of them to land
// before any LDS read, which would serialise the load pipeline against the MFMA loop. Here the
// kernel waits for the copies itself (vmcnt) before the barrier that publishes a stage.
// Address = sbase (wave-uniform 64-bit, SGPRs) + voff (per-lane byte offset).
__device__ __forceinline__ void copy16_to_lds(const void* sbase, int voff, unsigned lds_addr) {
  // m0 (the LDS destination) is an input operand, so the compiler knows the asm sets it. Its
  // hazard checks do not see inside the asm, so the asm supplies the wait states itself: an
  // SALU write of m0 needs 1 before an LDS-DMA load, and an SGPR of sbase written by a VALU
  // (v_readlane, when the compiler reloads a spilled SGPR) needs 5 before a VMEM read of it.
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "{m0}"(lds_addr));
}

// One operand of a k-tile in LDS: 256 rows of M (or N) by BK = 64 k, bf16, 32 KiB.
//
// gfx950's LDS has 64 banks of 4 bytes: a ds_read_b128 is served 16 lanes (256 bytes) per
// cycle and a ds_read_b64(_tr) 32 lanes per cycle, so each such lane group must cover all 64
// banks once (a 2-way conflict halves the read rate; measured 134 against 222 B/clk/CU).
//
// K-major operands (element (row, k) at base[row * ld + k]) are stored [row][64 k]: 128-byte
// rows whose eight 16-byte chunks sit at chunk ^ ((row >> 1) & 7). A wave's copy instruction
// moves 8 rows (lane l: row l / 8, stored chunk l % 8, which is global chunk
// (l % 8) ^ ((row >> 1) & 7), so each row's 128 contiguous bytes are read by 8 lanes). The
// MFMA operand of a lane is 8 consecutive k of one row, one ds_read_b128; the 16 lanes of one
// read cycle take 16 consecutive rows at one logical chunk: the even rows fill one 128-byte
// bank half at 8 distinct chunk positions and the odd rows the other.
//
// M/N-major operands (element at base[k * ld + row]) are stored as in HBM, [64 k][256 rows]:
// 512-byte k-rows (256 bytes for a 128-wide B tile) whose 16-byte chunk c sits at
// c ^ (2 * (krow & 3)) ^ (8 * ((c >> 1) & 1)). Both row pitches are whole multiples of the 64
// banks, so a chunk's banks depend on its stored position mod 16 alone and the placement below
// holds for both. A copy instruction moves 2 k-rows (4 for 256-byte rows; 32 or 16 lanes read
// one contiguous row segment). The
// MFMA operand (8 consecutive k of one row/column) is gathered with two ds_read_b64_tr_b16:
// within each 16-lane group, lane j reads 4 bf16 of k-row kb + j / 4 at columns
// c0 + 4 (j % 4) and the hardware transposes the 16 x 4 block so lane i receives column
// c0 + i, k = kb .. kb + 3. One group covers 4 k-rows x 32 bytes, which the (krow & 3) term
// spreads over 32 banks; the two groups of a read cycle sit 16 columns (2 chunks) apart and
// the (c >> 1) term places them in opposite bank halves.
template <bool KMAJOR, int ROWS = 256>
struct TileOperand {
  // M/N-major: a copy instruction (1 KiB) covers kRowsPerCopy k-rows of ROWS * 2 bytes.
  static constexpr int kKRowBytes = ROWS * 2;
  static constexpr int kRowsPerCopy = 1024 / kKRowBytes;
  static constexpr int kLanesPerRow = 64 / kRowsPerCopy;
  // M/N-major: stored position of logical 16-byte chunk c of k-row krow, and its inverse.
  __device__ static int stored_chunk(int c, int krow) {
    return c ^ (2 * (krow & 3)) ^ (8 * ((c >> 1) & 1));
  }
  __device__ static int logical_chunk(int p, int krow) {
    return p ^ (8 * (((p >> 1) ^ krow) & 1)) ^ (2 * (krow & 3));
  }
  // Byte offset of lane `lane`'s 16 bytes of copy instruction ii (0 .. 31) from the tile's
  // global base at k = 0, and the (row, k) of its first element.
  __device__ static void source(int ii, int lane, int& row, int& k) {
    if (KMAJOR) {
      row = ii * 8 + (lane >> 3);
      k = ((lane & 7) ^ ((row >> 1) & 7)) * 8;
    } else {
      k = ii * kRowsPerCopy + lane / kLanesPerRow;
      row = logical_chunk(lane % kLanesPerRow, k) * 8;
    }
  }
  __device__ static int64_t byte_offset(int row, int k, int64_t ld) {
    return KMAJOR ? 2 * (static_cast<int64_t>(row) * ld + k)
                  : 2 * (static_cast<int64_t>(k) * ld + row);
  }
  // Global step of one k-tile (elements).
  __device__ static int64_t ktile_step(int64_t ld) { return KMAJOR ? BK : BK * ld; }
  // LDS byte offset of the MFMA operand of MFMA block b (32 rows at wave offset wo),
  // 16-deep k step s; `half` selects the second 4-k read of an M/N-major operand.
  __device__ static int frag(int wo, int b, int s, int half, int lane) {
    if (KMAJOR) {
      const int row = wo + b * 32 + (lane & 31);
      const int c = 2 * s + (lane >> 5);
      return row * 128 + ((c ^ ((row >> 1) & 7)) * 16);
    } else {
      const int g = lane >> 4, j = lane & 15;
      const int col = wo + b * 32 + 16 * (g & 1) + 4 * (j & 3);
      const int krow = 16 * s + 8 * (g >> 1) + (j >> 2) + 4 * half;
      return krow * kKRowBytes + stored_chunk(col >> 3, krow) * 16 + (col & 7) * 2;
    }
  }
  __device__ static bf16x8_t read(const unsigned char HK_LDS* st, int wo, int b, int s,
                                  int lane) {
    if (KMAJOR) {
      return *reinterpret_cast<const bf16x8_t HK_LDS*>(st + frag(wo, b, s, 0, lane));
    } else {
      const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (bf16x4_t HK_LDS*)(st + frag(wo, b, s, 0, lane)));
      const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (bf16x4_t HK_LDS*)(st + frag(wo, b, s, 1, lane)));
      return bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
};

// Linear tile id t -> (tile_m, tile_n): consecutive ids to one XCD, grouped 8 tile-rows. The
// hardware deals workgroups to the 8 XCDs round-robin, so t % 8 is the XCD when t is a
// workgroup id or one offset by a multiple of 8.
__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
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

// Output transform: C = alpha * acc + beta * C, or, with a bias (bias != NULL),
// C = alpha * acc + beta * bias and C is written without being read. The bias element of
// output (row, col) is bias[row * brow + col * bcol]: (brow, bcol) = (0, 1) for a per-column
// bias (numel N), (1, 0) per row (numel M), (0, 0) scalar (numel 1), (N, 1) full (numel M*N,
// the same for every batch).
struct Epi {
  float alpha, beta;
  const uint16_t* bias;
  int64_t brow, bcol;
};

__device__ __forceinline__ float bias_at(const Epi& ep, int row, int col) {
  return hk::bf16_to_f32(ep.bias[row * ep.brow + col * ep.bcol]);
}

// Bias element of column col of batch b for an fp32 output (hk::F32Out).
__device__ __forceinline__ float f32out_bias(const hk::F32Out& fo, int M, int N, int b, int col) {
  if (fo.bias_stride == N) return fo.bias[col];
  if (fo.bias_stride == static_cast<int64_t>(M) * N)
    return fo.bias[static_cast<int64_t>(b % M) * N + col];
  if (fo.bias_stride == 1) return fo.bias[0];
  return 0.f;
}

// Scheduling hint: NR LDS reads spread over NM MFMAs (reads first in each pair), so the
// operands of the next k step are fetched while the current one multiplies.
template <int NM, int NR, int Q = 0>
__device__ __forceinline__ void interleave_reads() {
  if constexpr (Q < NM) {
    constexpr int per = (NR + NM - 1) / NM;
    constexpr int left = NR - Q * per;
    constexpr int n = left <= 0 ? 0 : (left < per ? left : per);
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    interleave_reads<NM, NR, Q + 1>();
  }
}

// Hands the accumulators of a wave to `out` through LDS, one 32-row MFMA block row at a time:
// the wave stores its block row into its own fp32 staging area (32 rows, pitch kWaveN * 4 + 16
// bytes, so the 16 lanes of one 16-byte write cycle start 4 banks apart) and reads it back as 8
// consecutive columns per lane: out(row, col, a, b) gets the wave-relative row and column of
// values a[0..3], b[0..3], and kWaveN / 8 consecutive lanes hold one row segment, so the
// outputs can be written 16 (bf16) or 32 (fp32) bytes per lane in whole lines. Stored straight
// from the MFMA layout instead, every store touched 32 rows and each 128-byte line of C was
// assembled from 8 stores (bf16): 23% of the BASELINE product. The area is the wave's own, so
// it needs no barrier beyond the one that ends the main loop.
template <int kWaveN, int kBlkM, typename Out>
__device__ __forceinline__ void staged_rows(const f32x16_t (&acc)[kBlkM][kWaveN / 32],
                                            unsigned char HK_LDS* area, int lane, Out&& out) {
  constexpr int kBlkN = kWaveN / 32;
  constexpr int P = kWaveN * 4 + 16;        // staging pitch (bytes)
  constexpr int LPR = kWaveN / 8;           // lanes per row
  constexpr int RPP = 64 / LPR;             // rows per pass
  const int r = lane & 31, h = lane >> 5;
  const int rr0 = lane / LPR, cc = (lane % LPR) * 8;
#pragma unroll
  for (int i = 0; i < kBlkM; ++i) {
#pragma unroll
    for (int j = 0; j < kBlkN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4_t HK_LDS*>(area + r * P + (32 * j + 8 * q + 4 * h) * 4) =
            f32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                    acc[i][j][4 * q + 3]};
#pragma unroll
    for (int p = 0; p < 32 / RPP; ++p) {
      const int rr = p * RPP + rr0;
      const f32x4_t a = *reinterpret_cast<const f32x4_t HK_LDS*>(area + rr * P + cc * 4);
      const f32x4_t b = *reinterpret_cast<const f32x4_t HK_LDS*>(area + rr * P + cc * 4 + 16);
      out(32 * i + rr, cc, a, b);
    }
  }
}

// The bf16 epilogue on staged rows: C = alpha * acc + beta * C (or + beta * bias) in fp32,
// one rounding to bf16 (v_cvt_pk_bf16_f32, round to nearest even), 16-byte stores.
template <bool BIAS>
struct Bf16RowOut {
  const Epi& ep;
  uint16_t* Cb;
  int64_t ldc;
  int M, N, wrow0, wcol0;
  __device__ void operator()(int rr, int cc, const f32x4_t& a, const f32x4_t& b) const {
    const int row = wrow0 + rr, col = wcol0 + cc;
    if (row >= M || col >= N) return;  // N % 8 == 0: the 8 columns are all in or all out
    f32x2_t v[4] = {f32x2_t{a[0], a[1]} * ep.alpha, f32x2_t{a[2], a[3]} * ep.alpha,
                    f32x2_t{b[0], b[1]} * ep.alpha, f32x2_t{b[2], b[3]} * ep.alpha};
    uint4* dst = reinterpret_cast<uint4*>(Cb + static_cast<int64_t>(row) * ldc + col);
    if (BIAS) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] += ep.beta * f32x2_t{bias_at(ep, row, col + 2 * e), bias_at(ep, row, col + 2 * e + 1)};
    } else if (ep.beta != 0.0f) {
      const uint4 old = *dst;
      const uint32_t o[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] += ep.beta * f32x2_t{__uint_as_float(o[e] << 16), __uint_as_float(o[e] & 0xffff0000u)};
    }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16x2_t bv = __builtin_convertvector(v[e], bf16x2_t);
      __builtin_memcpy(&w[e], &bv, 4);
    }
    // non-temporal: C is not read again by this product, and keeping it out of the caches
    // leaves them to the operands (8192^3 NN: 742 -> 714 us on MI355X). The fp32 split-K
    // partials below are read back by the finalize kernel and keep ordinary stores (with
    // non-temporal ones the 8192 x 1280 x 5120 dA product went from 130 to 149 us).
    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4_t{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_t*>(dst));
  }
};

// Main loop per k-tile kt (ring slot kt % 2), 4 k steps of 16 MFMAs each:
//   steps 0-2: operands of step s+1 are read from LDS between the MFMAs of step s; steps 0
//              and 1 first issue the second half of tile kt+1's copies (into slot (kt+1) % 2,
//              free since the barrier that ended tile kt-1);
//   step 3:    wait for this wave's copies of tile kt+1, barrier (tile kt+1 visible to all,
//              every wave done reading slot kt % 2), read step 0 of tile kt+1, and issue the
//              first half of tile kt+2's copies into slot kt % 2 between the MFMAs.
// A copy instruction (1 KiB) keeps the CU's address unit busy ~25 cycles (TA_TA_BUSY on
// MI355X), so a k-tile's 64 take ~1,600 of its ~2,048 MFMA cycles. Issued all in step 3 they
// held that step at ~1,160 cycles against 512 of MFMA work; split over steps 3, 0 and 1 the
// product runs ~1.5% faster (8192^3: 733 -> 721 us).
// The operands are swapped in the MFMA (B block as the "A" input), so each lane ends up
// holding 4 consecutive output columns of one output row per register quad; the epilogue
// hands them to the output through LDS (staged_rows).
// One workgroup's tile: tile `wg` of the BMT x BNT tiles that cover the columns
// [n_base, n_end) of C (N bounds the stores).
template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL, int BNT, int BMT = 256>
__device__ __forceinline__ void tile_body(
    int M, int N, int K, const Epi& ep, const uint16_t* __restrict__ A, int64_t lda, int64_t sA,
    const uint16_t* __restrict__ B, int64_t ldb, int64_t sB, uint16_t* __restrict__ C,
    int64_t ldc, int64_t sC, int split_k, int k_per_split, float* __restrict__ part,
    const hk::F32Out& fo, int n_base, int n_end, int wg) {
  static_assert(BMT == 256 || A_KMAJOR, "192-row tiles need a k-major A");
  using OA = TileOperand<A_KMAJOR>;
  using OB = TileOperand<B_KMAJOR, BNT>;
  constexpr int kWaveN = TileN<BNT, BMT>::kWaveN, kBlkN = TileN<BNT, BMT>::kBlkN;
  constexpr int kStageBytesB = TileN<BNT, BMT>::kStageBytesB, kLoadsB = TileN<BNT, BMT>::kLoadsB;
  constexpr int kWaveM = TileM<BMT>::kWaveM, kBlkM = TileM<BMT>::kBlkM;
  constexpr int kStageBytes = TileM<BMT>::kStageBytes, kLoadsPerWave = TileM<BMT>::kLoadsPerWave;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  unsigned char HK_LDS* ldsA = (unsigned char HK_LDS*)lds_raw;
  unsigned char HK_LDS* ldsB = ldsA + kStages * kStageBytes;

  const int batch = blockIdx.z / split_k;
  const int split = blockIdx.z - batch * split_k;
  const int tiles_m = (M + BMT - 1) / BMT, tiles_n = (n_end - n_base + BNT - 1) / BNT;
  int tm, tn;
  tile_coords(wg, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BMT, n0 = n_base + tn * BNT;
  const int kbeg = split * k_per_split;
  const int klen = min(K, kbeg + k_per_split) - kbeg;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // Tile bases at k = kbeg (wave-uniform) and per-lane source offsets of this wave's copy
  // instructions. Rows past M (N) are clamped to the last row: they only feed outputs that
  // are not stored. k past the split's end is zero-filled on the last k-tile (tail_fill).
  const unsigned char* gA = reinterpret_cast<const unsigned char*>(
      A + static_cast<int64_t>(batch) * sA +
      (A_KMAJOR ? static_cast<int64_t>(m0) * lda + kbeg : static_cast<int64_t>(kbeg) * lda + m0));
  const unsigned char* gB = reinterpret_cast<const unsigned char*>(
      B + static_cast<int64_t>(batch) * sB +
      (B_KMAJOR ? static_cast<int64_t>(n0) * ldb + kbeg : static_cast<int64_t>(kbeg) * ldb + n0));
  int offA[kLoadsPerWave], offB[kLoadsB];
  int kA[kLoadsPerWave], kB[kLoadsB];
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    int row, k;
    OA::source(wave * kLoadsPerWave + i, lane, row, k);
    row = min(row, (A_KMAJOR ? M - 8 + 7 : M - 8) - m0);  // k-major: a row; else an 8-row chunk
    offA[i] = static_cast<int>(OA::byte_offset(row, k, lda));
    kA[i] = k;
  }
#pragma unroll
  for (int i = 0; i < kLoadsB; ++i) {
    int row, k;
    OB::source(wave * kLoadsB + i, lane, row, k);
    row = min(row, (B_KMAJOR ? N - 8 + 7 : N - 8) - n0);
    offB[i] = static_cast<int>(OB::byte_offset(row, k, ldb));
    kB[i] = k;
  }
  const int64_t stepA = 2 * OA::ktile_step(lda), stepB = 2 * OB::ktile_step(ldb);
  const unsigned ldsA_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ldsA));
  const unsigned ldsB_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ldsB));
  const int ktiles = (klen + BK - 1) / BK;
  const bool tail = (klen % BK) != 0;  // last k-tile is partial

  // Copy q (0 .. kLoadsPerWave + kLoadsB - 1) of k-tile kt into ring slot `slot`. On a partial
  // last k-tile (fill), lanes whose 8 k values lie past the split's end store zeros instead.
  auto copy = [&](int kt, int slot, int q, bool fill) {
    const bool isA = q < kLoadsPerWave;
    const int i = isA ? q : q - kLoadsPerWave;
    const unsigned char* base = (isA ? gA + kt * stepA : gB + kt * stepB);
    const int off = isA ? offA[i] : offB[i];
    const unsigned lds = isA ? ldsA_addr + slot * kStageBytes + (wave * kLoadsPerWave + i) * 1024
                             : ldsB_addr + slot * kStageBytesB + (wave * kLoadsB + i) * 1024;
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
  constexpr int kCopies = kLoadsPerWave + kLoadsB;
  // a k-tile's copies: kH3 in the last k step of the k-tile two before it, the other kRest in
  // the first two k steps of the k-tile before it
  constexpr int kH3 = (kCopies + 1) / 2, kRest = kCopies - kH3;

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
  // Wait for k-tile 0 only; k-tile 1 lands while tile 0 is multiplied (waited for at its end).
  // A partial (fill) k-tile 1 may have issued fewer copies than kCopies: wait for all then.
  if (ktiles >= 2 && !(tail && ktiles == 2))
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kCopies) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();

  bf16x8_t fa[2][kBlkM], fb[2][kBlkN];
  if (ktiles > 0) {
#pragma unroll
    for (int i = 0; i < kBlkM; ++i) fa[0][i] = OA::read(ldsA, wm * kWaveM, i, 0, lane);
#pragma unroll
    for (int j = 0; j < kBlkN; ++j) fb[0][j] = OB::read(ldsB, wn * kWaveN, j, 0, lane);
  }
  constexpr int kReadsPerStep = (A_KMAJOR ? 1 : 2) * kBlkM + (B_KMAJOR ? 1 : 2) * kBlkN;
  constexpr int kMfmaPerStep = kBlkM * kBlkN;

  // One k-tile. STEADY (compile-time): tile kt + kStages exists and is whole, so its 32 copies
  // are issued with no per-copy condition; otherwise whether it exists (more) and whether it is
  // the partial last k-tile (fill) are tested at run time.
  auto ktile = [&](int kt, auto steady_tag) {
    constexpr bool STEADY = decltype(steady_tag)::value;
    const bool more = STEADY || kt + kStages < ktiles;
    const bool fill = !STEADY && tail && kt + kStages == ktiles - 1;
    const int slot = kt & 1;
    const unsigned char HK_LDS* sa = ldsA + slot * kStageBytes;
    const unsigned char HK_LDS* sb = ldsB + slot * kStageBytesB;
    // the copies of tile kt + 1 that the previous k-tile's last step left (kt >= 1)
    const bool rest = kt > 0 && (STEADY || kt + 1 < ktiles);
    const bool rest_fill = !STEADY && tail && kt + 1 == ktiles - 1;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s < 2 && kRest > 0) {
        constexpr int kRest0 = (kRest + 1) / 2;
        const int q0 = kH3 + (s == 0 ? 0 : kRest0), q1 = s == 0 ? kH3 + kRest0 : kCopies;
        if (rest) {
#pragma unroll
          for (int q = q0; q < q1; ++q) copy(kt + 1, slot ^ 1, q, rest_fill);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < kBlkM; ++i) fa[nxt][i] = OA::read(sa, wm * kWaveM, i, s + 1, lane);
#pragma unroll
        for (int j = 0; j < kBlkN; ++j) fb[nxt][j] = OB::read(sb, wn * kWaveN, j, s + 1, lane);
#pragma unroll
        for (int i = 0; i < kBlkM; ++i)
#pragma unroll
          for (int j = 0; j < kBlkN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[cur][j], fa[cur][i],
                                                                acc[i][j], 0, 0, 0);
        interleave_reads<kMfmaPerStep, kReadsPerStep>();
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < ktiles) {
          const unsigned char HK_LDS* na = ldsA + (slot ^ 1) * kStageBytes;
          const unsigned char HK_LDS* nb = ldsB + (slot ^ 1) * kStageBytesB;
#pragma unroll
          for (int i = 0; i < kBlkM; ++i) fa[nxt][i] = OA::read(na, wm * kWaveM, i, 0, lane);
#pragma unroll
          for (int j = 0; j < kBlkN; ++j) fb[nxt][j] = OB::read(nb, wn * kWaveN, j, 0, lane);
        }
#pragma unroll
        for (int i = 0; i < kBlkM; ++i)
#pragma unroll
          for (int j = 0; j < kBlkN; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[cur][j], fa[cur][i],
                                                                acc[i][j], 0, 0, 0);
            const int q = i * kBlkN + j;
            if (more && q < kH3) copy(kt + kStages, slot, q, fill);
            // steady state: keep each copy next to its MFMA, so that a wave's copies are spread
            // over the step (the copies are inline asm, which the scheduler does not group)
            if constexpr (STEADY) __builtin_amdgcn_sched_barrier(0);
          }
        if (kH3 > kMfmaPerStep && more) {
#pragma unroll
          for (int q = kMfmaPerStep; q < kH3; ++q) copy(kt + kStages, slot, q, fill);
        }

      }
    }
  };
  // steady state: every k-tile kt < steady has a whole k-tile kt + kStages to copy
  const int steady = ktiles - kStages - (tail ? 1 : 0);
  int kt = 0;
  for (; kt < steady; ++kt) ktile(kt, std::true_type{});
  for (; kt < ktiles; ++kt) ktile(kt, std::false_type{});

  // Epilogue. Lane l holds, for MFMA block (i, j) and quad q, output row
  // wm*128 + 32 i + l % 32 and columns wn*kWaveN + 32 j + 8 q + 4 (l / 32) .. +3; the rows go
  // out through LDS (staged_rows).
  // every wave is done with the LDS ring: its start becomes the waves' staging areas
  static_assert(kWaves * 32 * (kWaveN * 4 + 16) <= TileN<BNT, BMT>::kLdsBytes, "staging fits");
  __syncthreads();
  unsigned char HK_LDS* area = ldsA + wave * (32 * (kWaveN * 4 + 16));
  const int wrow0 = m0 + wm * kWaveM, wcol0 = n0 + wn * kWaveN;
  if (PARTIAL && fo.C) {
    // one split: fp32 C with alpha, beta and the bias applied here
    float* cb = fo.C + static_cast<int64_t>(batch) * fo.sC;
    staged_rows<kWaveN, kBlkM>(acc, area, lane, [&](int rr, int cc, const f32x4_t& a, const f32x4_t& b) {
      const int row = wrow0 + rr, col = wcol0 + cc;
      if (row >= M || col >= N) return;  // N % 8 == 0
      f32x4_t* dst = reinterpret_cast<f32x4_t*>(cb + static_cast<int64_t>(row) * fo.ldc + col);
      f32x4_t v0 = fo.alpha * a, v1 = fo.alpha * b;
      if (fo.beta != 0.0f) {
        v0 += fo.beta * dst[0];
        v1 += fo.beta * dst[1];
      }
      if (fo.bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v0[e] += fo.bias_scale * f32out_bias(fo, M, N, batch, col + e);
          v1[e] += fo.bias_scale * f32out_bias(fo, M, N, batch, col + 4 + e);
        }
      }
      dst[0] = v0;
      dst[1] = v1;
    });
    return;
  }
  if (PARTIAL) {
    float* out = part + (static_cast<int64_t>(split) * (gridDim.z / split_k) + batch) *
                            static_cast<int64_t>(M) * N;
    staged_rows<kWaveN, kBlkM>(acc, area, lane, [&](int rr, int cc, const f32x4_t& a, const f32x4_t& b) {
      const int row = wrow0 + rr, col = wcol0 + cc;
      if (row >= M || col >= N) return;
      f32x4_t* dst = reinterpret_cast<f32x4_t*>(out + static_cast<int64_t>(row) * N + col);
      dst[0] = a;
      dst[1] = b;
    });
    return;
  }
  uint16_t* Cb = C + static_cast<int64_t>(batch) * sC;
  if (ep.bias)
    staged_rows<kWaveN, kBlkM>(acc, area, lane, Bf16RowOut<true>{ep, Cb, ldc, M, N, wrow0, wcol0});
  else
    staged_rows<kWaveN, kBlkM>(acc, area, lane, Bf16RowOut<false>{ep, Cb, ldc, M, N, wrow0, wcol0});
}

// One column region: workgroup x takes tile x.
template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL, int BNT, int BMT>
__global__ __launch_bounds__(kThreads, 1) void bgemm_tiled(
    int M, int N, int K, Epi ep, const uint16_t* __restrict__ A, int64_t lda, int64_t sA,
    const uint16_t* __restrict__ B, int64_t ldb, int64_t sB, uint16_t* __restrict__ C,
    int64_t ldc, int64_t sC, int split_k, int k_per_split, float* __restrict__ part,
    hk::F32Out fo, int n_base, int n_end) {
  tile_body<A_KMAJOR, B_KMAJOR, PARTIAL, BNT, BMT>(M, N, K, ep, A, lda, sA, B, ldb, sB, C, ldc,
                                                  sC, split_k, k_per_split, part, fo, n_base,
                                                  n_end, blockIdx.x);
}

// Both column regions in one launch (column_split): workgroups [0, nfull) take the 256-wide
// tiles of columns [0, n_split), the rest the 128-wide tiles of [n_split, N). The 128-wide
// tiles start on CUs as the 256-wide ones finish, with no drain and launch between two
// kernels (about 2% of the 8192 x 5120 x 1280 product on MI355X). tile_coords' XCD grouping
// of the 128-wide region assumes that its first workgroup sits on XCD 0, which holds when
// nfull is a multiple of 8; otherwise only that region's L2 grouping is off, not which tiles
// it covers.
template <bool A_KMAJOR, bool B_KMAJOR, bool PARTIAL>
__global__ __launch_bounds__(kThreads, 1) void bgemm_mixed(
    int M, int N, int K, Epi ep, const uint16_t* __restrict__ A, int64_t lda, int64_t sA,
    const uint16_t* __restrict__ B, int64_t ldb, int64_t sB, uint16_t* __restrict__ C,
    int64_t ldc, int64_t sC, int split_k, int k_per_split, float* __restrict__ part,
    hk::F32Out fo, int n_split, int nfull) {
  const int wg = blockIdx.x;
  if (wg < nfull)
    tile_body<A_KMAJOR, B_KMAJOR, PARTIAL, 256>(M, N, K, ep, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                               split_k, k_per_split, part, fo, 0, n_split, wg);
  else
    tile_body<A_KMAJOR, B_KMAJOR, PARTIAL, 128>(M, N, K, ep, A, lda, sA, B, ldb, sB, C, ldc, sC,
                                               split_k, k_per_split, part, fo, n_split, N,
                                               wg - nfull);
}

// ---- 256 x 160 tiles on 16 x 16 x 32 MFMAs (A and B both k-major, C = alpha A B^T + ...) ----
// For products whose 256 x 256 tiles leave CUs idle while 256 x 160 tiles fill one round
// (8192 x 1280: 160 tiles of 256 x 256, 215 of 192 x 256, 256 of 256 x 160 on 256 CUs). 160
// columns are 5 blocks of 16, so the waves sit 4 (rows) x 2 (columns), each owning 64 x 80 of C
// as 4 x 5 blocks of v_mfma_f32_16x16x32_bf16. Whole tiles only (M % 256, N % 160, K % 64 == 0).
// LDS: a 3-slot ring of k-tiles (3 x 52 KiB, which only this tile shape fits in 160 KiB), each
// A [256][64 k] then B [160][64 k], bf16, stored as the k-major TileOperand layout (128-byte
// rows, chunk c of row r at c ^ ((r >> 1) & 7)); a 16-row operand block is one ds_read_b128
// per lane (lane l: row l % 16, logical chunk 4 s + l / 16 of k step s), 16 consecutive rows
// per read cycle, conflict-free as in the 32-row form.
// Copies: A is 32 copy instructions per k-tile (4 per wave), B 20: wave w issues B copies w,
// w + 8 and, for w < 4, w + 16, so waves 0-3 issue 7 per k-tile and waves 4-7 issue 6 (their
// vmcnt waits count 6).
// Per k-tile kt (2 k steps of 32): step 0 reads step 1's operands and runs step 0's 20 MFMAs
// with the last copies of tile kt + 2 between them; step 1 waits for this wave's copies of
// tile kt + 1 (tile kt + 2's may still be in flight), meets the others at the barrier (tile
// kt + 1 visible, slot kt % 3 free), reads tile kt + 1's step-0 operands and issues the first
// two copies of tile kt + 3 into slot kt % 3 between its MFMAs. Each copy so has more than a
// k-tile to land and the address unit's work is spread over both steps. On MI355X, 8192 x 1280
// x 5120: 96.2 us on 215 tiles of 192 x 256, 96.7 with these tiles on a 2-slot ring and every
// copy in step 1, 90.1 with 3 slots, 92.8 with 3 slots and every copy in step 1, 87.5 as here.
// The MFMA takes the B block as its first operand, so lane l holds C row l % 16 of its block,
// columns 4 (l / 16) .. + 3.
namespace w160 {
constexpr int kBM = 256, kBN = 160;
constexpr int kStageA = kBM * BK * 2;  // 32 KiB
constexpr int kStageB = kBN * BK * 2;  // 20 KiB
constexpr int kStage = kStageA + kStageB;
constexpr int kRing = 3;
constexpr size_t kLdsBytes = kRing * static_cast<size_t>(kStage);  // 156 KiB
constexpr int kCopiesA = kStageA / 1024 / kWaves;                  // 4
constexpr int kCopiesB = 3;                                        // 20 over 8 waves, see above
constexpr int kCopies = kCopiesA + kCopiesB;                       // 7 (6 for waves 4-7)
constexpr int kFirst = 2;  // copies of a k-tile issued in step 1, the rest in the next step 0
constexpr int kBlkM = 4, kBlkN = 5;                             // 16 x 16 blocks per wave
constexpr int kWaveM = 16 * kBlkM, kWaveN = 16 * kBlkN;         // 64 x 80
constexpr int kPitch = kWaveN * 4 + 16;                         // fp32 staging row, bytes
static_assert(kStageB / 1024 == 20 && kCopiesA * kWaves * 1024 == kStageA, "copy split");
static_assert(kLdsBytes <= 160 * 1024, "fits gfx950's 160 KiB of LDS");
static_assert(kWaves * 16 * kPitch <= static_cast<int>(kLdsBytes), "staging fits");

// LDS byte offset of lane `lane`'s 16 bytes of the 16-row block at row `r0`, k step s (0, 1).
__device__ __forceinline__ int frag16(int r0, int s, int lane) {
  const int row = r0 + (lane & 15);
  const int c = 4 * s + (lane >> 4);
  return row * 128 + ((c ^ ((row >> 1) & 7)) << 4);
}
}  // namespace w160

__global__ __launch_bounds__(kThreads, 1) void bgemm_nt_w160(
    int M, int N, int K, Epi ep, const uint16_t* __restrict__ A, int64_t lda, int64_t sA,
    const uint16_t* __restrict__ B, int64_t ldb, int64_t sB, uint16_t* __restrict__ C,
    int64_t ldc, int64_t sC) {
  using namespace w160;
  using OK = TileOperand<true>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  unsigned char HK_LDS* lds = (unsigned char HK_LDS*)lds_raw;
  const int batch = blockIdx.z;
  const int tiles_m = M / kBM, tiles_n = N / kBN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const unsigned char* gA = reinterpret_cast<const unsigned char*>(
      A + static_cast<int64_t>(batch) * sA + static_cast<int64_t>(m0) * lda);
  const unsigned char* gB = reinterpret_cast<const unsigned char*>(
      B + static_cast<int64_t>(batch) * sB + static_cast<int64_t>(n0) * ldb);
  // per-lane source offsets (bytes, from the tile base at k = 0) and LDS destinations of this
  // wave's copies; rows stay inside the tile (whole tiles), so no clamping is needed
  int off[kCopies];
  unsigned dst[kCopies];
  const unsigned lds_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
#pragma unroll
  for (int q = 0; q < kCopies; ++q) {
    int row, k;
    if (q < kCopiesA) {
      const int ii = wave * kCopiesA + q;
      OK::source(ii, lane, row, k);
      off[q] = static_cast<int>(OK::byte_offset(row, k, lda));
      dst[q] = lds_addr + ii * 1024;
    } else {
      int ii = wave + 8 * (q - kCopiesA);
      if (ii >= 20) ii = wave + 8;  // waves 4-7 have no third B copy (never issued)
      OK::source(ii, lane, row, k);
      off[q] = static_cast<int>(OK::byte_offset(row, k, ldb));
      dst[q] = lds_addr + kStageA + ii * 1024;
    }
  }
  const int ktiles = K / BK;
  const bool six = wave >= 4;  // waves 4-7 issue 6 copies per k-tile
  auto copy = [&](int kt, int slot, int q) {
    if (q == kCopies - 1 && six) return;
    const unsigned char* base = (q < kCopiesA ? gA : gB) + kt * (2 * BK);
    copy16_to_lds(base, off[q], dst[q] + slot * kStage);
  };
  // wait until at most n k-tiles of this wave's copies are in flight
  auto wait_tiles = [&](int n) {
    if (n == 2) {
      if (six) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * kCopies - 2) : "memory");
      else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * kCopies) : "memory");
    } else if (n == 1) {
      if (six) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kCopies - 1) : "memory");
      else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kCopies) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    }
  };

  f32x4_t acc[kBlkM][kBlkN];
#pragma unroll
  for (int i = 0; i < kBlkM; ++i)
#pragma unroll
    for (int j = 0; j < kBlkN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int p = 0; p < kRing; ++p)
    if (p < ktiles) {
#pragma unroll
      for (int q = 0; q < kCopies; ++q) copy(p, p, q);
    }
  wait_tiles(ktiles >= 3 ? 2 : ktiles - 1);  // k-tile 0 landed
  __builtin_amdgcn_s_barrier();

  bf16x8_t fa[2][kBlkM], fb[2][kBlkN];
  auto read_ops = [&](int slot, int s, int buf) {
    const unsigned char HK_LDS* sa = lds + slot * kStage;
    const unsigned char HK_LDS* sb = sa + kStageA;
#pragma unroll
    for (int i = 0; i < kBlkM; ++i)
      fa[buf][i] = *reinterpret_cast<const bf16x8_t HK_LDS*>(
          sa + frag16(wm * kWaveM + 16 * i, s, lane));
#pragma unroll
    for (int j = 0; j < kBlkN; ++j)
      fb[buf][j] = *reinterpret_cast<const bf16x8_t HK_LDS*>(
          sb + frag16(wn * kWaveN + 16 * j, s, lane));
  };
  read_ops(0, 0, 0);
  int slot = 0;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int nslot = slot == kRing - 1 ? 0 : slot + 1;
    const int slot2 = nslot == kRing - 1 ? 0 : nslot + 1;
    // step 0: operands of step 1 read while step 0 multiplies, with the rest of tile kt + 2's
    // copies between the MFMAs (its first kFirst went out in tile kt - 1's step 1; tile 2's
    // all in the prologue)
    const bool rest = kt >= 1 && kt + 2 < ktiles;
    read_ops(slot, 1, 1);
#pragma unroll
    for (int i = 0; i < kBlkM; ++i)
#pragma unroll
      for (int j = 0; j < kBlkN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[0][j], fa[0][i], acc[i][j], 0, 0,
                                                            0);
        const int q = kFirst + 2 * (i * kBlkN + j);
        if (q < kCopies && rest) copy(kt + 2, slot2, q);
        if (q + 1 < kCopies && rest) copy(kt + 2, slot2, q + 1);
      }
    // step 1: tile kt + 1 landed (tile kt + 2's copies may still be in flight), slot free
    wait_tiles(kt + 2 < ktiles ? 1 : 0);
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < ktiles) read_ops(nslot, 0, 0);
    const bool more = kt + kRing < ktiles;
#pragma unroll
    for (int i = 0; i < kBlkM; ++i)
#pragma unroll
      for (int j = 0; j < kBlkN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0,
                                                            0);
        const int q = i * kBlkN + j;
        if (q < kFirst && more) copy(kt + kRing, slot, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    slot = nslot;
  }

  // Epilogue: each wave stages one 16-row block row (16 x 80 fp32) in its own LDS area and
  // reads it back as 8 consecutive columns per lane (10 lanes per row, 6 rows per pass), so the
  // bf16 outputs go out 16 bytes per lane in row segments.
  __syncthreads();
  unsigned char HK_LDS* area = lds + wave * (16 * kPitch);
  uint16_t* Cb = C + static_cast<int64_t>(batch) * sC;
  const int wrow0 = m0 + wm * kWaveM, wcol0 = n0 + wn * kWaveN;
  auto emit = [&](auto&& out) {
#pragma unroll
    for (int i = 0; i < kBlkM; ++i) {
#pragma unroll
      for (int j = 0; j < kBlkN; ++j)
        *reinterpret_cast<f32x4_t HK_LDS*>(area + (lane & 15) * kPitch +
                                          (16 * j + 4 * (lane >> 4)) * 4) = acc[i][j];
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const int rr = 6 * p + lane / 10, cc = (lane % 10) * 8;
        if (lane < 60 && rr < 16) {
          const f32x4_t a = *reinterpret_cast<const f32x4_t HK_LDS*>(area + rr * kPitch + cc * 4);
          const f32x4_t b =
              *reinterpret_cast<const f32x4_t HK_LDS*>(area + rr * kPitch + cc * 4 + 16);
          out(16 * i + rr, cc, a, b);
        }
      }
    }
  };
  if (ep.bias)
    emit(Bf16RowOut<true>{ep, Cb, ldc, M, N, wrow0, wcol0});
  else
    emit(Bf16RowOut<false>{ep, Cb, ldc, M, N, wrow0, wcol0});
}

// C = alpha * sum_s part[s] + beta * C (split order), fp32 -> bf16.
// I: the index type, uint32_t when every index of the launch fits in 31 bits (a 64-bit
// division costs several times a 32-bit one).
template <typename I>
__global__ __launch_bounds__(256) void bgemm_splitk_finalize(const float* __restrict__ part,
                                                             int split_k, int batch, int M, int N,
                                                             Epi ep, uint16_t* __restrict__ C,
                                                             int64_t ldc, int64_t sC) {
  // 4 consecutive outputs per thread (N is a multiple of 8 on the tiled path)
  const I idx = (static_cast<I>(blockIdx.x) * 256 + threadIdx.x) * 4;
  const I mn = static_cast<I>(M) * N;
  if (idx >= mn * batch) return;
  const I b = idx / mn;
  const I e = idx - b * mn;
  const int row = static_cast<int>(e / N), col = static_cast<int>(e - static_cast<I>(row) * N);
  f32x2_t lo = f32x2_t{0.f, 0.f}, hi = f32x2_t{0.f, 0.f};
  for (int k = 0; k < split_k; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(part + (static_cast<int64_t>(k) * batch + b) * mn + e);
    lo += f32x2_t{v.x, v.y};
    hi += f32x2_t{v.z, v.w};
  }
  lo *= ep.alpha;
  hi *= ep.alpha;
  uint2* dst = reinterpret_cast<uint2*>(C + b * sC + static_cast<int64_t>(row) * ldc + col);
  if (ep.bias) {
    lo += ep.beta * f32x2_t{bias_at(ep, row, col), bias_at(ep, row, col + 1)};
    hi += ep.beta * f32x2_t{bias_at(ep, row, col + 2), bias_at(ep, row, col + 3)};
  } else if (ep.beta != 0.0f) {
    const float beta = ep.beta;
    const uint2 old = *dst;
    lo += beta * f32x2_t{__uint_as_float(old.x << 16), __uint_as_float(old.x & 0xffff0000u)};
    hi += beta * f32x2_t{__uint_as_float(old.y << 16), __uint_as_float(old.y & 0xffff0000u)};
  }
  const bf16x2_t blo = __builtin_convertvector(lo, bf16x2_t);
  const bf16x2_t bhi = __builtin_convertvector(hi, bf16x2_t);
  uint2 v;
  __builtin_memcpy(&v.x, &blo, 4);
  __builtin_memcpy(&v.y, &bhi, 4);
  *dst = v;
}

// Fallback: one thread per output, fp32 accumulation in k order.
__global__ __launch_bounds__(256) void bgemm_simple(int ta, int tb, int M, int N, int K, Epi ep,
                                                    const uint16_t* __restrict__ A,
                                                    int64_t lda, int64_t sA,
                                                    const uint16_t* __restrict__ B, int64_t ldb,
                                                    int64_t sB, uint16_t* __restrict__ C,
                                                    int64_t ldc, int64_t sC) {
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
  float f = ep.alpha * acc;
  if (ep.bias) f += ep.beta * bias_at(ep, row, col);
  else if (ep.beta != 0.0f) f += ep.beta * hk::bf16_to_f32(*dst);
  *dst = hk::f32_to_bf16(f);
}

float bf16_bits_to_float(hk_bf16 h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// BNT 256 or 128: one column region (bgemm_tiled); BNT 0: both regions (bgemm_mixed), with
// n_base = n_split and n_end = nfull.
template <bool AK, bool BKM, bool P, int BNT, int BMT = 256>
hipError_t launch_tiled(dim3 grid, hipStream_t stream, int M, int N, int K, const Epi& ep,
                        const uint16_t* A, int64_t lda, int64_t sA, const uint16_t* B,
                        int64_t ldb, int64_t sB, uint16_t* C, int64_t ldc,
                        int64_t sC, int split_k, int kps, float* part, const hk::F32Out& fo,
                        int n_base, int n_end) {
  static_assert(BNT != 0 || BMT == 256, "the mixed-width launch uses 256-row tiles");
  constexpr size_t kLds = TileN<BNT == 0 ? 256 : BNT, BMT>::kLdsBytes;
  const void* fn;
  if constexpr (BNT == 0) fn = reinterpret_cast<const void*>(&bgemm_mixed<AK, BKM, P>);
  else fn = reinterpret_cast<const void*>(&bgemm_tiled<AK, BKM, P, BNT, BMT>);
  static std::once_flag once;
  static hipError_t attr_status = hipSuccess;
  std::call_once(once, [fn] {
    attr_status = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLds));
  });
  HK_RETURN_IF_ERROR(attr_status);
  if constexpr (BNT == 0)
    hipLaunchKernelGGL((bgemm_mixed<AK, BKM, P>), grid, dim3(kThreads), kLds, stream, M, N, K, ep,
                       A, lda, sA, B, ldb, sB, C, ldc, sC, split_k, kps, part, fo, n_base, n_end);
  else
    hipLaunchKernelGGL((bgemm_tiled<AK, BKM, P, BNT, BMT>), grid, dim3(kThreads), kLds, stream, M,
                       N, K, ep, A, lda, sA, B, ldb, sB, C, ldc, sC, split_k, kps, part, fo,
                       n_base, n_end);
  return hk::launch_status();
}

template <bool P, int BNT, int BMT = 256>
hipError_t dispatch_layout(bool ta, bool tb, dim3 grid, hipStream_t stream, int M, int N, int K,
                           const Epi& ep, const uint16_t* A, int64_t lda, int64_t sA,
                           const uint16_t* B, int64_t ldb, int64_t sB, uint16_t* C,
                           int64_t ldc, int64_t sC, int split_k, int kps, float* part,
                           const hk::F32Out& fo, int n_base, int n_end) {
  // A is k-major unless transposed; B is k-major only when transposed.
  if (!ta && !tb)
    return launch_tiled<true, false, P, BNT, BMT>(grid, stream, M, N, K, ep, A, lda, sA, B, ldb,
                                                  sB, C, ldc, sC, split_k, kps, part, fo, n_base,
                                                  n_end);
  if (!ta && tb)
    return launch_tiled<true, true, P, BNT, BMT>(grid, stream, M, N, K, ep, A, lda, sA, B, ldb,
                                                 sB, C, ldc, sC, split_k, kps, part, fo, n_base,
                                                 n_end);
  if constexpr (BMT != 256) {
    return hipErrorInvalidValue;  // row_tile keeps 256-row tiles for an M-major A
  } else {
    if (ta && !tb)
      return launch_tiled<false, false, P, BNT>(grid, stream, M, N, K, ep, A, lda, sA, B, ldb,
                                                sB, C, ldc, sC, split_k, kps, part, fo, n_base,
                                                n_end);
    return launch_tiled<false, true, P, BNT>(grid, stream, M, N, K, ep, A, lda, sA, B, ldb, sB,
                                             C, ldc, sC, split_k, kps, part, fo, n_base, n_end);
  }
}

// Columns [0, n_split) of C take 256 x 256 tiles and [n_split, N) 256 x 128 tiles. One
// workgroup runs per CU (its LDS ring is 128 KiB), so a launch takes ceil(tiles / CUs) rounds;
// when the last round of 256-wide tiles would be partly empty, the trailing tile columns run
// as twice as many 128-wide tiles, which fill a round of half the length (8192 x 5120: 640
// tiles are 3 rounds, 512 tiles + 256 half tiles are 2.5). Costs in full-tile rounds, a half
// tile counted as 0.55 of one; a split is taken only if it saves at least 3%. Returns N for
// no split.
int column_split(int M, int N, int work_per_tile) {
  const int64_t cus = hk::device_cu_count();
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  auto rounds = [&](int64_t tiles) { return static_cast<double>(hk::ceil_div(tiles * work_per_tile, cus)); };
  const double whole = rounds(tiles_m * tiles_n);
  double best = whole;
  int64_t best_c = 0;
  for (int64_t c = 1; c <= tiles_n; ++c) {
    const int64_t n_split = (tiles_n - c) * BN;
    const double cost = rounds(tiles_m * (tiles_n - c)) +
                        0.55 * rounds(tiles_m * hk::ceil_div(N - n_split, int64_t{128}));
    if (cost < best) {
      best = cost;
      best_c = c;
    }
  }
  if (best_c == 0 || best > 0.97 * whole) return N;
  return static_cast<int>((tiles_n - best_c) * BN);
}

// Rows per tile. 256 x 256 tiles that do not fill one round of the CUs leave the rest idle
// (8192 x 1280: 160 tiles on 256 CUs). 192-row tiles cut each workgroup's work to 3/4 and
// raise the tile count (215 there), so they are used when their rounds, each costed 0.75 of a
// 256-row round, save at least 10%. They need a k-major A (the M-major LDS layout holds 256 or
// 128 rows) and a single k split.
int row_tile(bool ta, int M, int N, int grid_z, int split_k) {
  if (ta || split_k != 1) return 256;
  const int64_t cus = hk::device_cu_count();
  const int64_t tiles_n = (N + BN - 1) / BN;
  const int64_t t256 = static_cast<int64_t>((M + 255) / 256) * tiles_n * grid_z;
  if (t256 >= cus) return 256;
  const int64_t t192 = static_cast<int64_t>((M + 191) / 192) * tiles_n * grid_z;
  return 0.75 * static_cast<double>(hk::ceil_div(t192, cus)) <= 0.9 ? 192 : 256;
}

// 256 x 160 tiles (bgemm_nt_w160): both operands k-major, one k split, bf16 C, whole tiles,
// when 256 x 256 tiles leave CUs idle and 256 x 160 tiles fit one round. Each such workgroup
// carries 5/8 of a 256 x 256 tile's work (3/4 for the 192-row tiles, which then give way).
bool w160_plan(bool ta, bool tb, int M, int N, int K, int grid_z, int split_k) {
  if (ta || !tb || split_k != 1) return false;
  if (M % w160::kBM != 0 || N % w160::kBN != 0 || K % BK != 0) return false;
  const int64_t cus = hk::device_cu_count();
  const int64_t t256 = static_cast<int64_t>((M + 255) / 256) * ((N + BN - 1) / BN) * grid_z;
  const int64_t t160 = static_cast<int64_t>(M / w160::kBM) * (N / w160::kBN) * grid_z;
  return t256 < cus && t160 <= cus;
}

hipError_t launch_w160(int grid_z, hipStream_t stream, int M, int N, int K, const Epi& ep,
                       const uint16_t* A, int64_t lda, int64_t sA, const uint16_t* B,
                       int64_t ldb, int64_t sB, uint16_t* C, int64_t ldc, int64_t sC) {
  static std::once_flag once;
  static hipError_t attr_status = hipSuccess;
  std::call_once(once, [] {
    attr_status = hipFuncSetAttribute(reinterpret_cast<const void*>(&bgemm_nt_w160),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(w160::kLdsBytes));
  });
  HK_RETURN_IF_ERROR(attr_status);
  const dim3 grid(static_cast<unsigned>((M / w160::kBM) * (N / w160::kBN)), 1, grid_z);
  hipLaunchKernelGGL(bgemm_nt_w160, grid, dim3(kThreads), w160::kLdsBytes, stream, M, N, K, ep,
                     A, lda, sA, B, ldb, sB, C, ldc, sC);
  return hk::launch_status();
}

// The product over its column regions (column_split), in one launch; grid.z covers batches
// and splits. A split into partials (P with split_k > 1) keeps one region.
template <bool P>
hipError_t run_regions(bool ta, bool tb, int grid_z, hipStream_t stream, int M, int N, int K,
                       const Epi& ep, const uint16_t* A, int64_t lda, int64_t sA,
                       const uint16_t* B, int64_t ldb, int64_t sB, uint16_t* C, int64_t ldc,
                       int64_t sC, int split_k, int kps, float* part, const hk::F32Out& fo) {
  if constexpr (!P) {
    if (w160_plan(ta, tb, M, N, K, grid_z, split_k))
      return launch_w160(grid_z, stream, M, N, K, ep, A, lda, sA, B, ldb, sB, C, ldc, sC);
  }
  if (row_tile(ta, M, N, grid_z, split_k) == 192) {
    const int64_t tiles = static_cast<int64_t>((M + 191) / 192) * ((N + BN - 1) / BN);
    const dim3 grid(static_cast<unsigned>(tiles), 1, grid_z);
    return dispatch_layout<P, 256, 192>(ta, tb, grid, stream, M, N, K, ep, A, lda, sA, B, ldb, sB,
                                        C, ldc, sC, split_k, kps, part, fo, 0, N);
  }
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int n_split = split_k == 1 ? column_split(M, N, grid_z) : N;
  const int64_t nfull = tiles_m * ((n_split + BN - 1) / BN);
  const int64_t nhalf = tiles_m * hk::ceil_div(N - n_split, int64_t{128});
  if (nhalf == 0) {
    const dim3 grid(static_cast<unsigned>(nfull), 1, grid_z);
    return dispatch_layout<P, 256>(ta, tb, grid, stream, M, N, K, ep, A, lda, sA, B, ldb, sB, C,
                                   ldc, sC, split_k, kps, part, fo, 0, N);
  }
  if (nfull == 0) {
    const dim3 grid(static_cast<unsigned>(nhalf), 1, grid_z);
    return dispatch_layout<P, 128>(ta, tb, grid, stream, M, N, K, ep, A, lda, sA, B, ldb, sB, C,
                                   ldc, sC, split_k, kps, part, fo, 0, N);
  }
  const dim3 grid(static_cast<unsigned>(nfull + nhalf), 1, grid_z);
  return dispatch_layout<P, 0>(ta, tb, grid, stream, M, N, K, ep, A, lda, sA, B, ldb, sB, C,
                               ldc, sC, split_k, kps, part, fo, n_split,
                               static_cast<int>(nfull));
}

// Split-K chosen by the library when the caller gives none: the split with the least modelled
// time (us), summed over the rounds of 256 x 256 work items on the CUs:
//   - a round costs (k-tiles per split) x t(busy) plus a fixed prologue / epilogue (8 us with
//     bf16 C, 12 us with a 256 KiB fp32 partial per tile);
//   - t, a workgroup's time per k-tile, grows with the share of the CUs that are busy (clock
//     and shared-cache headroom): ~0.875 us with 100 of 256 CUs busy, ~1.62 us with all;
//   - splits add the finalize, an HBM pass over the partials (4 s + 2 bytes per output at
//     ~6 TB/s).
// Calibrated on the 8192 x 1280 x 5120 and 1280 x 5120 x 8192 products (160 and 100 tiles):
// measured 123 / 149 / 131 us at 1 / 2 / 3 splits for the first, 120 / 115 / 151 / 137 / 135
// us at 1 to 5 for the second; the model picks 1 and 2.
int auto_split_k(int64_t work_tiles, int64_t ktiles, int64_t outputs) {
  const int64_t cus = hk::device_cu_count();
  auto t_kt = [&](int64_t busy) {
    const double f = static_cast<double>(busy) / static_cast<double>(cus);
    const double x = (f - 0.39) / 0.61;
    return 0.875 + 0.745 * (x < 0.0 ? 0.0 : x > 1.0 ? 1.0 : x);
  };
  double best = 0.0;
  int best_s = 1;
  for (int s = 1; s <= 8; ++s) {
    if (s > 1 && ktiles / s < 4) break;
    const int64_t items = work_tiles * s, kps = hk::ceil_div(ktiles, static_cast<int64_t>(s));
    const double fixed = s > 1 ? 12.0 : 8.0;
    double cost = 0.0;
    for (int64_t done = 0; done < items; done += cus) {
      const int64_t busy = items - done < cus ? items - done : cus;
      cost += static_cast<double>(kps) * t_kt(busy) + fixed;
    }
    if (s > 1) cost += static_cast<double>(4 * s + 2) * static_cast<double>(outputs) / 6.0e6;
    if (s == 1 || cost < best) {
      best = cost;
      best_s = s;
    }
  }
  return best_s;
}

// Whether a product takes the 256 x 256 MFMA tiles (else the fp32-accumulating bgemm_simple):
// 8-element multiples for every contiguous extent, leading dimension and batch stride, 16-byte
// aligned bases, and leading dimensions whose per-lane 32-bit byte offsets fit.
bool tiled_path(bool ta, bool tb, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                int64_t sA, int64_t sB, int64_t sC, bool aligned) {
  const int contig_a = ta ? M : K, contig_b = tb ? K : N;
  return (contig_a % 8 == 0) && (contig_b % 8 == 0) && (N % 8 == 0) && (lda % 8 == 0) &&
         (ldb % 8 == 0) && (ldc % 8 == 0) && (sA % 8 == 0) && (sB % 8 == 0) &&
         (sC % 8 == 0) && aligned && K > 0 && lda < (1 << 22) && ldb < (1 << 22);
}

// Number of k splits the tiled path runs for a product (split_k == 0: the library's choice).
int tiled_splits(int M, int N, int K, int batch, int split_k) {
  int used = 1, kps = 0;
  hk::bgemm_split_plan(M, N, K, batch, split_k, &used, &kps);
  return used;
}

// bias == NULL: C = alpha * op(A) op(B) + beta * C. Otherwise C = alpha * op(A) op(B) +
// beta * bias with bias_numel N (per column), M (per row), 1 (scalar) or M*N (full, shared by
// all batches), tested in that order; C is then only written.
hipError_t bgemm_run(int transA, int transB, int M, int N, int K, hk_bf16 alpha_bits,
                     const hk_bf16* A, int lda, long long strideA, const hk_bf16* B, int ldb,
                     long long strideB, hk_bf16 beta_bits, const hk_bf16* bias,
                     int64_t bias_numel, hk_bf16* C, int ldc, long long strideC, int batchCount,
                     int splitK, hipStream_t stream) {
  HK_CHECK_ARG(transA >= 0 && transA <= 2 && transB >= 0 && transB <= 2);
  // splitK == 0: the library picks the split (auto_split_k)
  HK_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batchCount >= 0 && splitK >= 0);
  if (M == 0 || N == 0 || batchCount == 0) return hipSuccess;
  HK_CHECK_ARG(C != nullptr && ldc >= N);
  const bool ta = transA != 0, tb = transB != 0;  // OP_C is OP_T for real bf16
  HK_CHECK_ARG(K == 0 || (A != nullptr && B != nullptr));
  HK_CHECK_ARG(lda >= (ta ? M : K) && ldb >= (tb ? K : N));
  if (!bias && splitK == 0 && (M == 1 || N == 1)) {
    // A one-row or one-column product streams one operand once: the GEMV kernels
    if (M == 1)  // C[0][n] = sum_k op(A)[0][k] op(B)[k][n]
      return hk::bgemv_run(tb, N, K, alpha_bits, beta_bits, B, ldb, strideB, A, ta ? lda : 1,
                           strideA, C, 1, strideC, batchCount, stream);
    // C[m][0] = sum_k op(A)[m][k] op(B)[k][0]
    return hk::bgemv_run(!ta, M, K, alpha_bits, beta_bits, A, lda, strideA, B, tb ? 1 : ldb,
                         strideB, C, ldc, strideC, batchCount, stream);
  }
  Epi ep{bf16_bits_to_float(alpha_bits), bf16_bits_to_float(beta_bits), bias, 0, 0};
  if (bias) {
    if (bias_numel == N) ep.bcol = 1;
    else if (bias_numel == M) ep.brow = 1;
    else if (bias_numel == 1) { /* scalar: (0, 0) */ }
    else if (bias_numel == static_cast<int64_t>(M) * N) { ep.brow = N; ep.bcol = 1; }
    else return hipErrorInvalidValue;
  }

  const bool tiled_ok = tiled_path(ta, tb, M, N, K, lda, ldb, ldc, strideA, strideB, strideC,
                                   hk::aligned16(A) && hk::aligned16(B) && hk::aligned16(C));
  if (!tiled_ok) {
    if (K == 0) splitK = 1;
    dim3 grid((N + 15) / 16, (M + 15) / 16, batchCount);
    hipLaunchKernelGGL(bgemm_simple, grid, dim3(256), 0, stream, ta ? 1 : 0, tb ? 1 : 0, M, N,
                       K, ep, A, static_cast<int64_t>(lda), static_cast<int64_t>(strideA), B,
                       static_cast<int64_t>(ldb), static_cast<int64_t>(strideB), C,
                       static_cast<int64_t>(ldc), static_cast<int64_t>(strideC));
    return hk::launch_status();
  }
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  // k range per split rounded to the k-tile; `used` splits are not empty
  int used = 1, kps = K;
  hk::bgemm_split_plan(M, N, K, batchCount, splitK, &used, &kps);
  HK_CHECK_ARG(2 * tiles <= INT32_MAX && static_cast<int64_t>(batchCount) * used <= 65535);
  if (used == 1)
    return run_regions<false>(ta, tb, batchCount, stream, M, N, K, ep, A, lda, strideA, B, ldb,
                              strideB, C, ldc, strideC, 1, K, nullptr, hk::F32Out{});
  void* ws = nullptr;
  const size_t part_bytes = static_cast<size_t>(used) * batchCount * M * N * sizeof(float);
  HK_RETURN_IF_ERROR(hk::device_workspace(part_bytes, stream, &ws));
  float* part = static_cast<float*>(ws);
  HK_RETURN_IF_ERROR(run_regions<true>(ta, tb, batchCount * used, stream, M, N, K, ep, A, lda,
                                       strideA, B, ldb, strideB, C, ldc, strideC, used, kps,
                                       part, hk::F32Out{}));
  const int64_t total = static_cast<int64_t>(M) * N * batchCount;
  const dim3 fgrid(static_cast<unsigned>(hk::ceil_div(total, 1024)));
  if (total < (int64_t{1} << 31))
    hipLaunchKernelGGL(bgemm_splitk_finalize<uint32_t>, fgrid, dim3(256), 0, stream, part, used,
                       batchCount, M, N, ep, C, static_cast<int64_t>(ldc),
                       static_cast<int64_t>(strideC));
  else
    hipLaunchKernelGGL(bgemm_splitk_finalize<int64_t>, fgrid, dim3(256), 0, stream, part, used,
                       batchCount, M, N, ep, C, static_cast<int64_t>(ldc),
                       static_cast<int64_t>(strideC));
  return hk::launch_status();
}

}  // namespace

namespace hk {

void bgemm_split_plan(int M, int N, int K, int batch, int split_k, int* used, int* kps) {
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int s = split_k > 0 ? split_k
                            : auto_split_k(tiles * batch, hk::ceil_div(K, BK),
                                           static_cast<int64_t>(M) * N * batch);
  *kps = static_cast<int>(hk::ceil_div(hk::ceil_div(K, s), BK) * BK);
  *used = static_cast<int>(hk::ceil_div(K, *kps));
}

hipError_t bgemm_partials(bool ta, bool tb, int M, int N, int K, const hk_bf16* A, int64_t lda,
                          int64_t sA, const hk_bf16* B, int64_t ldb, int64_t sB, int batch,
                          int used, int kps, float* part, const F32Out* out,
                          hipStream_t stream) {
  const int contig_a = ta ? M : K, contig_b = tb ? K : N;
  HK_CHECK_ARG(M > 0 && N > 0 && K > 0 && batch > 0 && used >= 1 && kps % BK == 0);
  HK_CHECK_ARG(contig_a % 8 == 0 && contig_b % 8 == 0 && N % 8 == 0 && lda % 8 == 0 &&
               ldb % 8 == 0 && sA % 8 == 0 && sB % 8 == 0 && hk::aligned16(A) &&
               hk::aligned16(B) && lda < (1 << 22) && ldb < (1 << 22));
  const int64_t tiles = static_cast<int64_t>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  HK_CHECK_ARG(2 * tiles <= INT32_MAX && static_cast<int64_t>(batch) * used <= 65535);
  const Epi ep{1.0f, 0.0f, nullptr, 0, 0};
  const F32Out fo = used == 1 && out ? *out : F32Out{};
  return run_regions<true>(ta, tb, batch * used, stream, M, N, K, ep, A, lda, sA, B, ldb, sB,
                           nullptr, 0, 0, used, kps, part, fo);
}

}  // namespace hk

extern "C" int hk_bgemm_split_count(int transA, int transB, int M, int N, int K, int batchCount,
                                    int splitK) {
  if (transA < 0 || transA > 2 || transB < 0 || transB > 2 || M < 0 || N < 0 || K < 0 ||
      batchCount < 0 || splitK < 0)
    return -1;
  if (M == 0 || N == 0 || batchCount == 0) return 0;
  const bool ta = transA != 0, tb = transB != 0;
  if (splitK == 0 && (M == 1 || N == 1)) return 1;  // the GEMV kernels
  const int64_t lda = ta ? M : K, ldb = tb ? K : N;
  if (!tiled_path(ta, tb, M, N, K, lda, ldb, N, lda * (ta ? K : M), ldb * (tb ? N : K),
                  static_cast<int64_t>(M) * N, true))
    return 1;
  return tiled_splits(M, N, K, batchCount, splitK);
}

extern "C" int hk_bgemm_tile_rows(int transA, int transB, int M, int N, int K, int batchCount,
                                  int splitK) {
  const int splits = hk_bgemm_split_count(transA, transB, M, N, K, batchCount, splitK);
  if (splits < 0) return -1;
  if (splits == 0) return 0;
  const bool ta = transA != 0, tb = transB != 0;
  const int64_t lda = ta ? M : K, ldb = tb ? K : N;
  if ((splitK == 0 && (M == 1 || N == 1)) ||
      !tiled_path(ta, tb, M, N, K, lda, ldb, N, lda * (ta ? K : M), ldb * (tb ? N : K),
                  static_cast<int64_t>(M) * N, true))
    return 0;
  if (w160_plan(ta, tb, M, N, K, batchCount * splits, splits)) return w160::kBM;
  return row_tile(ta, M, N, batchCount * splits, splits);
}

extern "C" int hk_bgemm_tile_cols(int transA, int transB, int M, int N, int K, int batchCount,
                                  int splitK) {
  const int rows = hk_bgemm_tile_rows(transA, transB, M, N, K, batchCount, splitK);
  if (rows <= 0) return rows;
  const int splits = hk_bgemm_split_count(transA, transB, M, N, K, batchCount, splitK);
  return w160_plan(transA != 0, transB != 0, M, N, K, batchCount * splits, splits) ? w160::kBN
                                                                                   : BN;
}

extern "C" hipError_t hk_bgemm(int transA, int transB, int M, int N, int K, hk_bf16 alpha,
                               const hk_bf16* A, int lda, long long strideA, const hk_bf16* B,
                               int ldb, long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                               long long strideC, int batchCount, hipStream_t stream) {
  return bgemm_run(transA, transB, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta,
                   nullptr, 0, C, ldc, strideC, batchCount, 0, stream);
}

extern "C" hipError_t hk_bgemm_core(int layout, int splitK, int M, int N, int K, hk_bf16 alpha,
                                    const hk_bf16* A, int lda, long long strideA,
                                    const hk_bf16* B, int ldb, long long strideB, hk_bf16 beta,
                                    hk_bf16* C, int ldc, long long strideC, int batchCount,
                                    hipStream_t stream) {
  // BgemmLayout { NT, TN, NN } (blas/bf16/bgemm_core_template.cu:59)
  HK_CHECK_ARG(layout >= HK_LAYOUT_NT && layout <= HK_LAYOUT_NN);
  HK_CHECK_ARG(splitK >= 1);
  const int ta = layout == HK_LAYOUT_TN ? 1 : 0;
  const int tb = layout == HK_LAYOUT_NT ? 1 : 0;
  return bgemm_run(ta, tb, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, nullptr, 0,
                   C, ldc, strideC, batchCount, splitK, stream);
}

extern "C" hipError_t hk_bgemm_nt_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                           int lda, long long strideA, const hk_bf16* B, int ldb,
                                           long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                           long long strideC, int batchCount,
                                           hipStream_t stream) {
  return bgemm_run(0, 1, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, nullptr, 0,
                   C, ldc, strideC, batchCount, 0, stream);
}

extern "C" hipError_t hk_bgemm_tn_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                           int lda, long long strideA, const hk_bf16* B, int ldb,
                                           long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                           long long strideC, int batchCount,
                                           hipStream_t stream) {
  return bgemm_run(1, 0, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, nullptr, 0,
                   C, ldc, strideC, batchCount, 0, stream);
}

extern "C" hipError_t hk_bgemm_addmm(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                     long long strideA, const hk_bf16* B, int ldb,
                                     long long strideB, hk_bf16 beta, const hk_bf16* bias,
                                     int64_t bias_numel, hk_bf16* C, int ldc, long long strideC,
                                     int batchCount, hipStream_t stream) {
  // C is only written: without a bias the product is C = alpha * A B (bgemm_addmm…:214-300)
  if (!bias) beta = 0;
  return bgemm_run(0, 0, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, bias,
                   bias_numel, C, ldc, strideC, batchCount, 0, stream);
}

extern "C" hipError_t hk_bgemm_core_bias(int layout, int splitK, int M, int N, int K, hk_bf16 alpha,
                                         const hk_bf16* A, int lda, long long strideA,
                                         const hk_bf16* B, int ldb, long long strideB,
                                         hk_bf16 beta, const hk_bf16* bias, int64_t bias_numel,
                                         hk_bf16* C, int ldc, long long strideC, int batchCount,
                                         hipStream_t stream) {
  HK_CHECK_ARG(layout >= HK_LAYOUT_NT && layout <= HK_LAYOUT_NN);
  HK_CHECK_ARG(splitK >= 1);
  const int ta = layout == HK_LAYOUT_TN ? 1 : 0;
  const int tb = layout == HK_LAYOUT_NT ? 1 : 0;
  return bgemm_run(ta, tb, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, bias,
                   bias_numel, C, ldc, strideC, batchCount, splitK, stream);
}
