// attention_bwd.hip - fused attention backward (key-tile-centric), fp32 I/O, head_dim 64.
//
// Reference behaviour: OwnTensor::mem_efficient_bwd_unified_kernel_exp12<64, Causal>
// (kernels/attention/mem_efficient_bwd_unified_kernel_exp12.cu:54-329): for a tile of keys,
// loop over query tiles; P = exp(scale * Q K^T - LSE), dP = dO V^T, dS = P (dP - D) * scale;
// dV += P^T dO and dK += dS^T Q stay on chip, dQ += dS K is added to global memory atomically
// (the caller zeroes dQ); dK, dV are stored once at the end.
//
// Design (gfx950): one workgroup = 8 waves owns 128 keys of one (batch, head): wave w takes key
// group w % 4 (32 keys) and query half w / 4 of every 64-query tile, so each SIMD runs two
// waves. gfx950 has no TF32 MFMA; every product runs as a bf16x3 split on
// v_mfma_f32_32x32x16_bf16 (x = hi + lo in bf16, a b = ah bh + ah bl + al bh accumulated in
// fp32, relative error ~1e-5). K and V of the tile are split and staged into LDS once. Q and dO
// are split once per call by a pre-pass into bf16 hi / lo planes ([b, h][T][64], plus LSE log2(e)
// and D as contiguous [b, h][T] rows), and each query tile is copied from them straight into LDS
// (global_load_lds, no registers): the copies of tile i + 1 are issued once every wave is done
// reading tile i's Q / dO and land during tile i's dQ phase. Splitting in every key-tile
// workgroup instead (8 x per query row at T = 1024) cost 14% of the kernel in VALU and LDS
// stores, and holding the next tile's fp32 rows in registers another 15% at the BASELINE shape.
// All LDS operands are bf16 hi / lo pairs of [rows][64] arrays (128-byte rows) read two
// ways: 16-byte reads for a contraction over the head dimension, and the gfx950 transposing read
// ds_read_b64_tr_b16 for a contraction over rows, so each tensor is stored once. Per query tile
// a wave forms S = Q K^T and dP = dO V^T for its 32 x 32 block (accumulators hold one key column
// per lane), P and dS in registers, then its query half's share of dV += P^T dO and
// dK += dS^T Q with P / dS as the register operand (the contraction over queries runs in the
// order the lane holds them; the dO / Q operand is read in the same order). The dP, dV and dK
// MFMAs are issued one at a time with the P / dS work that does not depend on them in between,
// so each wave overlaps its own VALU and matrix work (measured 2-3% faster than issuing each
// product's MFMAs together after the VALU work it needs). dS^T goes through
// LDS once, and dQ = dS K is formed on 16 x 16 x 32 MFMA blocks, each wave owning 16 queries x
// 32 d over all 128 keys of the tile, so each dQ element receives one atomic add per key tile
// with no exchange between waves. The two query halves' dK / dV partials are summed through LDS
// at the end. 128-key tiles mean 8 dQ passes per query row at T = 1024 (the reference's 16-key tiles
// make 64). Workgroups are ordered key tile major, so under causal masking the longest ones are
// dispatched first.
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kHD = 64;
constexpr int kBKV = 128;        // keys per workgroup
constexpr int kBQ = 64;          // queries per inner tile
constexpr int kThreads = 512;    // 8 waves: 4 key groups x 2 query halves
constexpr float kLog2e = 1.4426950408889634f;

// LDS (bytes). Every [rows][64] bf16 array has 128-byte rows whose 16-byte chunk c of row r sits
// at chunk c ^ swz(r); each has a hi and a lo plane.
constexpr int kRowBytes = 128;
constexpr int kKPlane = kBKV * kRowBytes;  // 16 KiB
constexpr int kQPlane = kBQ * kRowBytes;   // 8 KiB
constexpr int kOffKh = 0, kOffKl = kOffKh + kKPlane;
constexpr int kOffVh = kOffKl + kKPlane, kOffVl = kOffVh + kKPlane;
constexpr int kOffQh = kOffVl + kKPlane, kOffQl = kOffQh + kQPlane;
constexpr int kOffOh = kOffQl + kQPlane, kOffOl = kOffOh + kQPlane;  // dO
constexpr int kOffSh = kOffOl + kQPlane, kOffSl = kOffSh + kKPlane;  // dS^T [key][query]
constexpr int kOffL = kOffSl + kKPlane;
constexpr int kOffD = kOffL + kBQ * 4;
constexpr size_t kLdsBytes = kOffD + kBQ * 4;  // 131,584 bytes
// The final dK / dV exchange reuses the start of LDS (4 key groups x 2 x 32 x 65 floats).
static_assert(4 * 2 * 32 * 65 * 4 <= kLdsBytes, "dK / dV exchange fits");
static_assert(kLdsBytes <= 160 * 1024, "fits gfx950's 160 KiB of LDS");

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define HK_LDS __attribute__((address_space(3)))

// Chunk permutation of row r. 16 consecutive rows at one logical chunk (a 16-byte operand read)
// and 4 consecutive rows x 4 consecutive chunks (a transposing read of 32 lanes) both land on
// distinct banks.
__device__ __forceinline__ int swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int off128(int r, int chunk) { return r * kRowBytes + ((chunk ^ swz(r)) << 4); }

// x = hi + lo, both bf16 rounded to nearest even (|x - hi - lo| <= 2^-18 |x|); returns the
// {hi pair, lo pair} of two values, element 0 in the low half.
__device__ __forceinline__ u32x2_t split2(float x0, float x1) {
  const uint32_t hi = __builtin_bit_cast(uint32_t,
                                         __builtin_convertvector(f32x2_t{x0, x1}, bf16x2_t));
  const float r0 = x0 - __uint_as_float(hi << 16);
  const float r1 = x1 - __uint_as_float(hi & 0xffff0000u);
  return u32x2_t{hi, __builtin_bit_cast(uint32_t,
                                        __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t))};
}
// Eight values -> {hi x8, lo x8}.
__device__ __forceinline__ void split8(const float* x, u32x4_t& hi, u32x4_t& lo) {
  const u32x2_t a = split2(x[0], x[1]), b = split2(x[2], x[3]);
  const u32x2_t c = split2(x[4], x[5]), d = split2(x[6], x[7]);
  hi = u32x4_t{a.x, b.x, c.x, d.x};
  lo = u32x4_t{a.y, b.y, c.y, d.y};
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// v_mfma_f32_32x32x16_bf16: A (32 x 16) lane l holds row l % 32, k = 8 (l / 32) .. + 7; B (16 x 32)
// lane l holds column l % 32, same k; C element i of lane l is (row 8 (i / 4) + 4 (l / 32) + i % 4,
// column l % 32).
// v_mfma_f32_16x16x32_bf16 (dQ): A (16 x 32) lane l holds row l % 16 and B (32 x 16) column
// l % 16, each with 8 k values of lane group l / 16 (the pairing of A and B values is all the
// sum over k needs); C element r of lane l is (row 4 (l / 16) + r, column l % 16).
__device__ __forceinline__ f32x16_t mfma3(bf16x8_t ah, bf16x8_t al, bf16x8_t bh, bf16x8_t bl,
                                          f32x16_t c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, c, 0, 0, 0);
}

// Stages rows [r0, r0 + ROWS) x 64 floats of a strided tensor into a hi / lo plane pair:
// thread t handles row t / TPR, TPR threads per row, 64 / TPR floats (whole 16-byte chunks)
// each. Rows at or past T are zero. `reg` holds the fp32 values between load and store so that
// the global loads of the next tile can be in flight during the current one.
template <int ROWS>
struct Stager {
  static constexpr int kTPR = kThreads / ROWS;     // threads per row: 8 (Q, dO) or 4 (K, V)
  static constexpr int kFloats = kHD / kTPR;       // 8 or 16
  static constexpr int kVec = kFloats / 4;
  f32x4_t reg[kVec];
  __device__ void load(const float* base, int64_t stride, int64_t r0, int64_t T) {
    const int64_t row = r0 + threadIdx.x / kTPR;
    const int col = (threadIdx.x % kTPR) * kFloats;
    const int64_t rr = row < T ? row : T - 1;  // in bounds; zeroed below
    const float* src = base + rr * stride + col;
#pragma unroll
    for (int v = 0; v < kVec; ++v) reg[v] = *reinterpret_cast<const f32x4_t*>(src + 4 * v);
    if (row >= T) {
#pragma unroll
      for (int v = 0; v < kVec; ++v) reg[v] = f32x4_t{};
    }
  }
  __device__ void store(char HK_LDS* hi, char HK_LDS* lo) const {
    const int row = threadIdx.x / kTPR;
    const int chunk0 = (threadIdx.x % kTPR) * (kFloats / 8);
#pragma unroll
    for (int cc = 0; cc < kFloats / 8; ++cc) {
      const float x[8] = {reg[2 * cc][0], reg[2 * cc][1], reg[2 * cc][2], reg[2 * cc][3],
                          reg[2 * cc + 1][0], reg[2 * cc + 1][1], reg[2 * cc + 1][2],
                          reg[2 * cc + 1][3]};
      u32x4_t h, l;
      split8(x, h, l);
      const int off = off128(row, chunk0 + cc);
      *reinterpret_cast<u32x4_t HK_LDS*>(hi + off) = h;
      *reinterpret_cast<u32x4_t HK_LDS*>(lo + off) = l;
    }
  }
};

// 16-byte (4-byte) global -> LDS copy of one lane (global_load_lds_dwordx4 / _dword): the wave's
// 64 lanes write 1 KiB (256 bytes) of LDS at m0 + 16 (4) * lane. Address = sbase (wave-uniform,
// SGPRs) + voff (per-lane byte offset). Inline asm, so the compiler does not wait for every copy
// before each LDS read; the kernel waits for the copies itself (vmcnt) before the barrier that
// publishes a tile. m0 is an input operand, so the compiler knows the asm sets it.
// The compiler's hazard checks do not see inside the asm: when sbase was just reloaded from a
// spill slot (v_readlane, a VALU write of the SGPRs), the VMEM read of it needs 5 wait states,
// which the leading s_nop 4 provides (without it the copy can use a stale address).
__device__ __forceinline__ void copy16_to_lds(const void* sbase, int voff, unsigned lds_addr) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "{m0}"(lds_addr));
}
__device__ __forceinline__ void copy4_to_lds(const void* sbase, int voff, unsigned lds_addr) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase),
               "{m0}"(lds_addr));
}

// Pre-split query-side operands of one call: bf16 hi / lo planes of Q and dO, [b, h][T][64]
// (128-byte rows), and LSE * log2(e) and D as [b, h][T].
struct QPlanes {
  const char* qh;
  const char* ql;
  const char* oh;
  const char* ol;
  const float* l2;
  const float* d;
};

// Vector memory operations each lane issues after a tile's copies: the dQ atomics. A wave
// waits with vmcnt(kAtomicsPerTile) for its copies of the next tile (vector memory operations
// complete in issue order), so the atomics themselves are never waited for.
constexpr int kAtomicsPerTile = 8;

// The pre-pass: grid (ceil(T * 8 / 256), B * nh); thread t of the row-chunk index covers 8
// consecutive d of one row of Q and of dO.
__global__ __launch_bounds__(256) void attn_bwd_prepare(hk_attn_bwd_params p, char* qh, char* ql,
                                                        char* oh, char* ol, float* l2, float* dd) {
  const int bh = blockIdx.y;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = idx >> 3;
  const int chunk = static_cast<int>(idx & 7);
  if (row >= p.T) return;
  const float* q = p.Q + b * p.q_strideB + h * p.q_strideH + row * p.q_strideM + 8 * chunk;
  const float* o = p.dO + b * p.do_strideB + h * p.do_strideH + row * p.do_strideM + 8 * chunk;
  const int64_t dst = ((static_cast<int64_t>(bh) * p.T + row) * 8 + chunk) * 16;
  const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(q);
  const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(q + 4);
  const f32x4_t o0 = *reinterpret_cast<const f32x4_t*>(o);
  const f32x4_t o1 = *reinterpret_cast<const f32x4_t*>(o + 4);
  const float xq[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
  const float xo[8] = {o0[0], o0[1], o0[2], o0[3], o1[0], o1[1], o1[2], o1[3]};
  u32x4_t hi, lo;
  split8(xq, hi, lo);
  *reinterpret_cast<u32x4_t*>(qh + dst) = hi;
  *reinterpret_cast<u32x4_t*>(ql + dst) = lo;
  split8(xo, hi, lo);
  *reinterpret_cast<u32x4_t*>(oh + dst) = hi;
  *reinterpret_cast<u32x4_t*>(ol + dst) = lo;
  if (chunk == 0) {
    const int64_t r = static_cast<int64_t>(bh) * p.T + row;
    l2[r] = p.LSE[b * p.lse_strideB + h * p.lse_strideH + row] * kLog2e;
    dd[r] = p.D[b * p.d_strideB + h * p.d_strideH + row];
  }
}

__global__ __launch_bounds__(kThreads, 1) void attn_bwd_kernel(hk_attn_bwd_params p, int nbh,
                                                                QPlanes qp) {
  extern __shared__ __attribute__((aligned(16))) char lds_generic[];
  char HK_LDS* lds = (char HK_LDS*)lds_generic;
  char HK_LDS* sKh = lds + kOffKh;
  char HK_LDS* sKl = lds + kOffKl;
  char HK_LDS* sVh = lds + kOffVh;
  char HK_LDS* sVl = lds + kOffVl;
  char HK_LDS* sSh = lds + kOffSh;
  char HK_LDS* sSl = lds + kOffSl;
  float HK_LDS* sL = (float HK_LDS*)(lds + kOffL);
  float HK_LDS* sD = (float HK_LDS*)(lds + kOffD);

  const int64_t T = p.T;
  // Linear order: all (batch, head)s of key tile 0 first, then key tile 1, ... Under causal
  // masking the first key tiles meet the most query tiles, so the hardware's in-order dispatch
  // hands out the longest workgroups first (longest-processing-time-first scheduling).
  const int kt = static_cast<int>(blockIdx.x) / nbh;
  const int bh = static_cast<int>(blockIdx.x) - kt * nbh;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t k0 = static_cast<int64_t>(kt) * kBKV;

  const float* Kb = p.K + b * p.k_strideB + h * p.k_strideH;
  const float* Vb = p.V + b * p.v_strideB + h * p.v_strideH;
  float* dQb = p.dQ + b * p.dq_strideB + h * p.dq_strideH;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int hh = lane >> 5;
  const int kg = wave & 3, qh = wave >> 2;
  const float sl2 = p.scale * kLog2e;

  // K and V tiles (128 x 64) once
  {
    Stager<kBKV> st;
    st.load(Kb, p.k_strideM, k0, T);
    st.store(sKh, sKl);
    st.load(Vb, p.v_strideM, k0, T);
    st.store(sVh, sVl);
  }

  // query tiles: causal starts at the tile holding the first key of this workgroup
  const int64_t q_first = p.is_causal ? (k0 / kBQ) * kBQ : 0;
  const int nq = static_cast<int>((T - q_first + kBQ - 1) / kBQ);
  // Without causal masking every key tile of a head visits all query tiles; key tile kt starts
  // at query tile 2 kt (mod nq), so the key tiles of one head add into different dQ rows at
  // any one time (measured ~2% faster than all starting at tile 0).
  const int rot = p.is_causal || nq == 0 ? 0 : (2 * kt) % nq;
  auto tile_q = [&](int it) -> int64_t {
    const int j = it + rot >= nq ? it + rot - nq : it + rot;
    return q_first + static_cast<int64_t>(j) * kBQ;
  };

  // Copies of query tile q0 into LDS: wave w moves rows 8 w .. 8 w + 7 of each of the four
  // planes (lane l: row 8 w + l / 8, stored chunk l % 8, which holds logical chunk
  // (l % 8) ^ swz(row)); waves 0 and 1 also move the 64 LSE * log2(e) and D values. Rows past
  // T read row T - 1: they only meet masked keys / queries and are never stored.
  const int64_t plane_row0 = static_cast<int64_t>(bh) * T;
  const int crow = 8 * wave + (lane >> 3);
  const int cchunk = (lane & 7) ^ swz(crow);
  const unsigned lds_base = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
  auto copy_tile = [&](int64_t q0) {
    const int64_t r = q0 + crow < T ? q0 + crow : T - 1;
    const int voff = static_cast<int>(r * kRowBytes) + (cchunk << 4);
    const int64_t head = plane_row0 * kRowBytes;
    const unsigned dst = lds_base + 1024 * wave;
    copy16_to_lds(qp.qh + head, voff, dst + kOffQh);
    copy16_to_lds(qp.ql + head, voff, dst + kOffQl);
    copy16_to_lds(qp.oh + head, voff, dst + kOffOh);
    copy16_to_lds(qp.ol + head, voff, dst + kOffOl);
    if (wave < 2) {
      const int64_t rr = q0 + lane < T ? q0 + lane : T - 1;
      copy4_to_lds((wave == 0 ? qp.l2 : qp.d) + plane_row0, static_cast<int>(rr * 4),
                   lds_base + (wave == 0 ? kOffL : kOffD));
    }
  };
  if (nq > 0) copy_tile(tile_q(0));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // dV, dK: C layout of (A = P^T or dS^T: rows = keys, B = dO or Q: columns = d):
  // key 32 kg + 8 (i/4) + 4 hh + i%4, d 32 db + c
  f32x16_t dv[2] = {f32x16_t{}, f32x16_t{}};
  f32x16_t dk[2] = {f32x16_t{}, f32x16_t{}};

  // ---- per-lane LDS byte offsets, formed once; each read below adds compile-time or
  // wave-uniform terms only -------------------------------------------------------------------
  // Rows R + c (R a multiple of 32) share swz(c). 16-byte reads of chunk 2 ks + hh:
  const int sw_c = swz(c);
  int roff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) roff[ks] = c * kRowBytes + (((2 * ks + hh) ^ sw_c) << 4);
  // Transposed reads (ds_read_b64_tr_b16): within each 16-lane group, lane j reads 4 bf16 of
  // row rb + j / 4 at columns cb + 4 (j % 4), and lane i of the group receives column cb + i of
  // rows rb .. rb + 3. Lane (group bit g1, index j) addresses row rb + j / 4 at column
  // cb + 16 g1 + 4 (j % 4); x = chunk of that column within a 32-column block.
  const int j15 = lane & 15, jj = j15 >> 2;
  const int colin = 16 * ((lane >> 4) & 1) + 4 * (j15 & 3);
  const int x = colin >> 3, colb = (colin & 7) * 2;
  const int sbit = ((jj >> 1) & 1) << 2;
  // dV / dK: rows 32 qh + 16 ks + 4 hh + {0..3} (elements 0-3) and + 8 (elements 4-7),
  // columns 32 db + ...
  int tva[2], tvb[2];
#pragma unroll
  for (int db = 0; db < 2; ++db) {
    tva[db] = (4 * hh + jj) * kRowBytes + (((4 * db + x) ^ (sbit | hh)) << 4) + colb;
    tvb[db] = (4 * hh + 8 + jj) * kRowBytes + (((4 * db + x) ^ (sbit | ((hh + 2) & 3))) << 4) + colb;
  }
  // dQ on 16 x 16 x 32 MFMA blocks: wave w owns queries 16 (w / 2) .. + 15 and d 32 (w % 2) .. + 31
  // (two 16 x 16 blocks sharing the dS operand) over all 128 keys, so no exchange between
  // waves is needed. Both operands are read transposed (contraction over their rows = keys):
  // lane group g = lane / 16 takes keys 32 ks + 8 g .. + 7 of its column, as two 4-row reads.
  const int qb16 = wave >> 1, dh = wave & 1;
  const int g16 = lane >> 4, c4 = (j15 & 3) >> 1, cb8 = 8 * (j15 & 1);
  const int s16a = sbit | (2 * (g16 & 1)), s16b = sbit | (2 * (g16 & 1) + 1);
  const int tsa = (8 * g16 + jj) * kRowBytes + (((2 * qb16 + c4) ^ s16a) << 4) + cb8;
  const int tsb = (8 * g16 + 4 + jj) * kRowBytes + (((2 * qb16 + c4) ^ s16b) << 4) + cb8;
  int tka[2], tkb[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    tka[jb] = (8 * g16 + jj) * kRowBytes + (((4 * dh + 2 * jb + c4) ^ s16a) << 4) + cb8;
    tkb[jb] = (8 * g16 + 4 + jj) * kRowBytes + (((4 * dh + 2 * jb + c4) ^ s16b) << 4) + cb8;
  }
  // dS^T writes: row 32 kg + c, queries 32 qh + 8 g + 4 hh .. + 3
  int wsd[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) wsd[g] = c * kRowBytes + (((4 * qh + g) ^ sw_c) << 4) + 8 * hh;

  const char HK_LDS* qrow = lds + kOffQh + 32 * qh * kRowBytes;  // + plane step for lo / dO
  const char HK_LDS* krow = lds + kOffKh + 32 * kg * kRowBytes;
  auto rd16 = [&](const char HK_LDS* base, int off) {
    return *reinterpret_cast<const bf16x8_t HK_LDS*>(base + off);
  };
  auto rdtr = [&](const char HK_LDS* base, int offa, int offb) {
    const bf16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((bf16x4_t HK_LDS*)(base + offa));
    const bf16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((bf16x4_t HK_LDS*)(base + offb));
    return bf16x8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  };

  for (int it = 0; it < nq; ++it) {
    const int64_t q0 = tile_q(it);
    // This tile's copies were issued before the previous tile's atomics: with those still in
    // flight they are done once at most kAtomicsPerTile operations are outstanding. The barrier
    // then publishes every wave's copies (and orders the previous tile's dQ exchange reads).
    if (it > 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAtomicsPerTile) : "memory");
    __syncthreads();

    // This wave's block: keys k0 + 32 kg .. + 31, queries q0 + 32 qh .. + 31. Under causal
    // masking a block whose keys all follow its queries is zero; one whose keys all precede
    // them (and lies inside T) needs no mask.
    const int64_t kw = k0 + 32 * kg, qw = q0 + 32 * qh;
    const bool dead = p.is_causal && kw > qw + 31;
    const bool clean = (!p.is_causal || kw + 31 <= qw) && kw + 32 <= T && qw + 32 <= T;

    bf16x8_t ph[2], pl[2], sh[2], sl[2];
    if (!dead) {
      // S = Q K^T and dP = dO V^T for this wave's 32 queries x 32 keys, contraction over d:
      // lane (c, hh) holds key column 32 kg + c, queries 32 qh + 8 (i/4) + 4 hh + i%4.
      f32x16_t s = f32x16_t{}, dp = f32x16_t{};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s = mfma3(rd16(qrow, roff[ks]), rd16(qrow + kQPlane, roff[ks]), rd16(krow, roff[ks]),
                  rd16(krow + kKPlane, roff[ks]), s);
        __builtin_amdgcn_sched_barrier(0);  // keeps the operand reads of later steps from all
                                            // being hoisted here (they would not fit registers)
      }
      // Edge blocks: a pair outside the mask (query or key past T, key after the query under
      // causal masking) gets the score -inf, so P = exp2(-inf) = 0 and dS = 0 below; interior
      // blocks (clean, wave-uniform) skip this. Offsets are relative to the block, 32-bit.
      if (!clean) {
        const int key_lim = T - kw < 32 ? static_cast<int>(T - kw) : 32;  // keys kw + c < T
        const int q_lim = T - qw < 32 ? static_cast<int>(T - qw) : 32;    // queries qw + r < T
        const int cdiff = static_cast<int>(kw - qw);  // key - query = cdiff + c - r
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = 8 * (i >> 2) + 4 * hh + (i & 3);  // query row within the block
          const bool valid = r < q_lim && c < key_lim && (!p.is_causal || cdiff + c - r <= 0);
          s[i] = valid ? s[i] : -INFINITY;
        }
      }
      // dP = dO V^T, dV += P^T dO and dK += dS^T Q, in a fixed issue order: each MFMA is
      // followed by a share of VALU work that does not depend on it (P = exp2(s sl2 - L) and
      // its split under dP, dS = P (dP - D) and its split under dV) and by the operand reads of
      // later steps, so one wave keeps the matrix core and the VALU busy together while the
      // other wave of its SIMD sits in the same phase. Each MFMA result is passed to an empty
      // volatile asm, which holds the MFMA between its neighbours (instruction selection
      // otherwise sinks these pure operations below the VALU work, whatever sched_barrier says).
      // P^T / dS^T are the A operands (rows = keys): k-step ks covers the lane's elements
      // 8 ks .. 8 ks + 7, i.e. queries 32 qh + 16 ks + 4 hh + {0..3} and + 8 + {0..3}; the dO / Q
      // operand is read transposed (contraction over its rows = queries) in the same order.
      auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
      auto mf = [](bf16x8_t a, bf16x8_t bb, f32x16_t& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bb, acc, 0, 0, 0);
        asm volatile("" ::"v"(acc));
      };
      // exponent <= ~0 (scores minus the row's log-sum-exp); hardware exp2
      auto p_group = [&](int g) {
        const f32x4_t lv = *reinterpret_cast<const f32x4_t HK_LDS*>(sL + 32 * qh + 8 * g + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * g + e] = __builtin_amdgcn_exp2f(s[4 * g + e] * sl2 - lv[e]);
      };
      auto ds_group = [&](int g) {
        const f32x4_t dv4 = *reinterpret_cast<const f32x4_t HK_LDS*>(sD + 32 * qh + 8 * g + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; ++e) dp[4 * g + e] = s[4 * g + e] * (dp[4 * g + e] - dv4[e]);
      };
      u32x4_t phu[2], plu[2], shu[2], slu[2];
      auto p_split = [&](int ks, int j) {  // elements 8 ks + 2 j, + 1 of P
        const u32x2_t r = split2(s[8 * ks + 2 * j], s[8 * ks + 2 * j + 1]);
        phu[ks][j] = r.x;
        plu[ks][j] = r.y;
      };
      auto ds_split = [&](int ks, int j) {
        const u32x2_t r = split2(dp[8 * ks + 2 * j], dp[8 * ks + 2 * j + 1]);
        shu[ks][j] = r.x;
        slu[ks][j] = r.y;
      };
      struct Fr { bf16x8_t ah, al, bh, bl; };  // dP operands: dO hi / lo (A), V hi / lo (B)
      auto dp_frag = [&](int ks) {
        return Fr{rd16(qrow + 2 * kQPlane, roff[ks]), rd16(qrow + 3 * kQPlane, roff[ks]),
                  rd16(krow + 2 * kKPlane, roff[ks]), rd16(krow + 3 * kKPlane, roff[ks])};
      };
      struct Tr { bf16x8_t h, l; };  // transposed dO (plane 2) or Q (plane 0) of (ks, db)
      auto tr_frag = [&](int plane, int ks, int db) {
        const char HK_LDS* qb0 = qrow + ks * 16 * kRowBytes + plane * kQPlane;
        return Tr{rdtr(qb0, tva[db], tvb[db]), rdtr(qb0 + kQPlane, tva[db], tvb[db])};
      };
      // ---- dP, with P and its split
      Fr f0 = dp_frag(0), f1 = dp_frag(1);
      fence();
      mf(f0.ah, f0.bh, dp); p_group(0); fence();
      mf(f0.ah, f0.bl, dp); p_group(1); fence();
      mf(f0.al, f0.bh, dp); p_group(2); f0 = dp_frag(2); fence();
      mf(f1.ah, f1.bh, dp); p_group(3); fence();
      mf(f1.ah, f1.bl, dp); p_split(0, 0); p_split(0, 1); fence();
      mf(f1.al, f1.bh, dp); p_split(0, 2); p_split(0, 3); f1 = dp_frag(3); fence();
      mf(f0.ah, f0.bh, dp); p_split(1, 0); p_split(1, 1); fence();
      mf(f0.ah, f0.bl, dp); p_split(1, 2); p_split(1, 3); fence();
      Tr o0 = tr_frag(2, 0, 0);
      mf(f0.al, f0.bh, dp); fence();
      Tr o1 = tr_frag(2, 0, 1);
      mf(f1.ah, f1.bh, dp); fence();
      mf(f1.ah, f1.bl, dp); fence();
      mf(f1.al, f1.bh, dp); fence();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        ph[ks] = as_bf16x8(phu[ks]);
        pl[ks] = as_bf16x8(plu[ks]);
      }
      // ---- dV, with dS and its split
      mf(ph[0], o0.h, dv[0]); ds_group(0); fence();
      mf(ph[0], o0.l, dv[0]); ds_group(1); fence();
      mf(pl[0], o0.h, dv[0]); ds_group(2); o0 = tr_frag(2, 1, 0); fence();
      mf(ph[0], o1.h, dv[1]); ds_group(3); fence();
      mf(ph[0], o1.l, dv[1]); ds_split(0, 0); ds_split(0, 1); fence();
      mf(pl[0], o1.h, dv[1]); ds_split(0, 2); ds_split(0, 3); o1 = tr_frag(2, 1, 1); fence();
      mf(ph[1], o0.h, dv[0]); ds_split(1, 0); ds_split(1, 1); fence();
      mf(ph[1], o0.l, dv[0]); ds_split(1, 2); ds_split(1, 3); fence();
      Tr q0t = tr_frag(0, 0, 0);
      mf(pl[1], o0.h, dv[0]); fence();
      Tr q1t = tr_frag(0, 0, 1);
      mf(ph[1], o1.h, dv[1]); fence();
      mf(ph[1], o1.l, dv[1]); fence();
      mf(pl[1], o1.h, dv[1]); fence();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        sh[ks] = as_bf16x8(shu[ks]);
        sl[ks] = as_bf16x8(slu[ks]);
      }
      // ---- dK
      mf(sh[0], q0t.h, dk[0]); fence();
      mf(sh[0], q0t.l, dk[0]); fence();
      mf(sl[0], q0t.h, dk[0]); q0t = tr_frag(0, 1, 0); fence();
      mf(sh[0], q1t.h, dk[1]); fence();
      mf(sh[0], q1t.l, dk[1]); fence();
      mf(sl[0], q1t.h, dk[1]); q1t = tr_frag(0, 1, 1); fence();
      mf(sh[1], q0t.h, dk[0]); fence();
      mf(sh[1], q0t.l, dk[0]); fence();
      mf(sl[1], q0t.h, dk[0]); fence();
      mf(sh[1], q1t.h, dk[1]); fence();
      mf(sh[1], q1t.l, dk[1]); fence();
      mf(sl[1], q1t.h, dk[1]); fence();
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ph[ks] = pl[ks] = sh[ks] = sl[ks] = bf16x8_t{};
    }
    // dS^T -> LDS [key][query]: the lane's 4 consecutive queries of group g are one 8-byte
    // write per plane (already split: group g is half of A operand g / 2)
    {
      char HK_LDS* wh = sSh + 32 * kg * kRowBytes;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x4_t hv = __builtin_bit_cast(u32x4_t, sh[g >> 1]);
        const u32x4_t lv = __builtin_bit_cast(u32x4_t, sl[g >> 1]);
        const int half = g & 1;
        *reinterpret_cast<u32x2_t HK_LDS*>(wh + wsd[g]) = u32x2_t{hv[2 * half], hv[2 * half + 1]};
        *reinterpret_cast<u32x2_t HK_LDS*>(wh + kKPlane + wsd[g]) =
            u32x2_t{lv[2 * half], lv[2 * half + 1]};
      }
    }
    __syncthreads();
    // every wave is done with this tile's Q / dO / LSE / D: the next tile's copies land while
    // the dQ phase runs
    if (it + 1 < nq) copy_tile(tile_q(it + 1));
    // dQ (queries 16 qb16 .., d 32 dh + 16 jb ..) = dS[q][keys] K[keys][d] over the 128 keys
    f32x4_t dq[2] = {f32x4_t{}, f32x4_t{}};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int rb = 32 * ks * kRowBytes;
      const bf16x8_t ah = rdtr(sSh + rb, tsa, tsb), al = rdtr(sSl + rb, tsa, tsb);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const bf16x8_t bh = rdtr(sKh + rb, tka[jb], tkb[jb]), bl = rdtr(sKl + rb, tka[jb], tkb[jb]);
        dq[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, dq[jb], 0, 0, 0);
        dq[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, dq[jb], 0, 0, 0);
        dq[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, dq[jb], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    {
      // dq[jb][r]: query 16 qb16 + 4 g16 + r, d 32 dh + 16 jb + j15. Every lane issues exactly
      // kAtomicsPerTile atomics (the count the next tile's vmcnt wait assumes): a row past T
      // adds 0 to row T - 1 instead.
      const int64_t qblk = q0 + 16 * qb16 + 4 * g16;
      const int rows_left = T - qblk < 4 ? static_cast<int>(T - qblk) : 4;  // may be <= 0
      float* dqu = dQb + qblk * p.dq_strideM + 32 * dh + j15;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool in = r < rows_left;
          const float v = in ? dq[jb][r] * p.scale : 0.f;
          float* dst = in ? dqu + r * p.dq_strideM + 16 * jb
                          : dQb + (T - 1) * p.dq_strideM + 32 * dh + 16 * jb + j15;
          unsafeAtomicAdd(dst, v);
        }
    }
  }

  // Sum the two query halves' dK / dV partials of each key group through LDS (the tiles are no
  // longer needed), then store dK (scaled) and dV rows of this wave's keys.
  __syncthreads();
  float HK_LDS* pk = (float HK_LDS*)lds + kg * (2 * 32 * 65);  // [2 (dk, dv)][32 keys][65]
  if (qh == 1) {
#pragma unroll
    for (int d2 = 0; d2 < 2; ++d2)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i >> 2) + 4 * hh + (i & 3);
        pk[r * 65 + 32 * d2 + c] = dk[d2][i];
        pk[32 * 65 + r * 65 + 32 * d2 + c] = dv[d2][i];
      }
  }
  __syncthreads();
  if (qh == 0) {
    float* dKb = p.dK + b * p.dk_strideB + h * p.dk_strideH;
    float* dVb = p.dV + b * p.dv_strideB + h * p.dv_strideH;
    const int64_t krow0 = k0 + 32 * kg + 4 * hh;
    float* dkp = dKb + krow0 * p.dk_strideM + c;
    float* dvp = dVb + krow0 * p.dv_strideM + c;
#pragma unroll
    for (int d2 = 0; d2 < 2; ++d2)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rs = 8 * (i >> 2) + (i & 3);
        const int r = rs + 4 * hh;
        if (krow0 + rs < T) {
          dkp[rs * p.dk_strideM + 32 * d2] = (dk[d2][i] + pk[r * 65 + 32 * d2 + c]) * p.scale;
          dvp[rs * p.dv_strideM + 32 * d2] = dv[d2][i] + pk[32 * 65 + r * 65 + 32 * d2 + c];
        }
      }
  }
}

bool rows_aligned(const void* base, int64_t strideB, int64_t strideH, int64_t strideM) {
  return hk::aligned16(base) && strideB % 4 == 0 && strideH % 4 == 0 && strideM % 4 == 0;
}

}  // namespace

extern "C" hipError_t hk_attn_backward(const hk_attn_bwd_params* params, int head_dim,
                                       hipStream_t stream) {
  HK_CHECK_ARG(params != nullptr);
  const hk_attn_bwd_params& p = *params;
  HK_CHECK_ARG(head_dim == kHD);
  HK_CHECK_ARG(p.B >= 0 && p.nh >= 0 && p.T >= 0);
  if (p.B == 0 || p.nh == 0 || p.T == 0) return hipSuccess;
  HK_CHECK_ARG(p.Q && p.K && p.V && p.dO && p.LSE && p.D && p.dQ && p.dK && p.dV);
  HK_CHECK_ARG(rows_aligned(p.Q, p.q_strideB, p.q_strideH, p.q_strideM) &&
               rows_aligned(p.K, p.k_strideB, p.k_strideH, p.k_strideM) &&
               rows_aligned(p.V, p.v_strideB, p.v_strideH, p.v_strideM) &&
               rows_aligned(p.dO, p.do_strideB, p.do_strideH, p.do_strideM));
  const int64_t bh = static_cast<int64_t>(p.B) * p.nh;
  HK_CHECK_ARG(bh <= 65535);
  HK_CHECK_ARG(p.dq_strideM >= 0 && p.dq_strideM < (int64_t{1} << 28));  // 32-bit lane offsets
  HK_CHECK_ARG(p.T <= (1 << 24));  // 32-bit plane offsets
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kLdsBytes));
  });
  HK_RETURN_IF_ERROR(attr);
  const int64_t nkt = (static_cast<int64_t>(p.T) + kBKV - 1) / kBKV;
  HK_CHECK_ARG(nkt * bh <= INT32_MAX);
  // the query-side planes in the stream's workspace: 4 x [b, h][T][64] bf16, 2 x [b, h][T] fp32
  const int64_t rows = bh * p.T;
  const size_t plane = static_cast<size_t>(rows) * kRowBytes;
  void* ws = nullptr;
  HK_RETURN_IF_ERROR(hk::device_workspace(4 * plane + 2 * static_cast<size_t>(rows) * 4, stream,
                                          &ws));
  char* wsb = static_cast<char*>(ws);
  float* l2 = reinterpret_cast<float*>(wsb + 4 * plane);
  hipLaunchKernelGGL(attn_bwd_prepare,
                     dim3(static_cast<unsigned>(hk::ceil_div(static_cast<int64_t>(p.T) * 8, 256)),
                          static_cast<unsigned>(bh)),
                     dim3(256), 0, stream, p, wsb, wsb + plane, wsb + 2 * plane, wsb + 3 * plane, l2,
                     l2 + rows);
  HK_RETURN_IF_ERROR(hk::launch_status());
  const QPlanes qp{wsb, wsb + plane, wsb + 2 * plane, wsb + 3 * plane, l2, l2 + rows};
  hipLaunchKernelGGL(attn_bwd_kernel, dim3(static_cast<unsigned>(nkt * bh)), dim3(kThreads),
                     kLdsBytes, stream, p, static_cast<int>(bh), qp);
  return hk::launch_status();
}
