// attention_fwd.hip - fused attention forward, fp32 I/O, head_dim 64, causal or not, with the
// saved log-sum-exp; plus the backward pre-pass D = rowsum(dO * O).
//
// Reference behaviour:
//   fused_attn_forward_kernel_tc_sm89<64, 64, 64, 1>
//       kernels/attention/fused_attn_forward_kernel_tc_sm89.cu:72-426 (params :8-29):
//       O = softmax(scale * Q K^T, key j <= query i when causal) V, LSE = max + ln(sum);
//       with dropout_p > 0 and a dropout_mask, the masked exp terms are normalised by their own
//       sum (:316-334).
//   mem_efficient_bwd_precompute_D_sm89<64>
//       kernels/attention/mem_efficient_bwd_precompute_D_sm89.cu:45-91: D = rowsum(dO * O).
//
// Design (gfx950): one workgroup = 4 waves = 128 query rows of one (batch, head); a wave owns 32
// queries. gfx950 has no TF32 MFMA; the products run as a bf16x3 split on
// v_mfma_f32_32x32x16_bf16: each fp32 operand x becomes hi + lo (two bf16) and a product is
// ah bh + ah bl + al bh, three bf16 MFMA products accumulated in fp32. That is fp32-class
// accuracy (relative error ~1e-5, measured O max-rel 5e-6 against the fp32 CPU reference) at
// 16 / 3 the throughput of the fp32 MFMA (v_mfma_f32_32x32x2_f32); the reference itself rounds
// its operands to TF32. The score tile is formed transposed, S^T = K Q^T, so each lane owns one
// query column: the online-softmax max is one 16-value register reduction plus a single
// cross-half shuffle and the exponentiated scores are already laid out as the B operand of the
// next product, O^T += V^T P^T (no LDS round trip of P). Q stays in registers (pre-scaled by
// scale * log2 e, so the softmax uses the hardware exp2, split once); each K / V tile of 32 keys
// is split while it is staged into LDS (K as [key][d], V transposed as [d][key]), with the next
// tile's global loads in flight. 36 KB of LDS and <= 168 VGPRs per workgroup let 3 workgroups
// share a CU, so the BASELINE grid (768 workgroups) runs in one round on 256 CUs. Causal
// workgroups stop at the diagonal; their order is described at snake_item.
#include <initializer_list>
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

static_assert(offsetof(hk_attn_fwd_params, T) == 48, "hk_attn_fwd_params layout");
static_assert(offsetof(hk_attn_fwd_params, dropout_mask) == 72, "hk_attn_fwd_params layout");
static_assert(sizeof(hk_attn_fwd_params) == 192, "hk_attn_fwd_params layout");
static_assert(offsetof(hk_attn_bwd_params, B) == 80, "hk_attn_bwd_params layout");
static_assert(offsetof(hk_attn_bwd_params, q_strideB) == 104, "hk_attn_bwd_params layout");
static_assert(sizeof(hk_attn_bwd_params) == 328, "hk_attn_bwd_params layout");

namespace {

constexpr int kHD = 64;
constexpr int kBQ = 128;   // queries per workgroup (4 waves x 32)
constexpr int kBKV = 32;   // keys per K/V tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// LDS stage: K hi / K lo as [key][64 d] bf16 with a 144-byte row pitch, then V^T hi / V^T lo
// as [d][32 keys] bf16 with a 72-byte row pitch. gfx950's LDS serves 256 bytes per cycle over
// 64 banks (16 lanes of a 16-byte read, 32 lanes of an 8-byte read): row c of K starts at
// bank 36 c mod 64 and row d of V^T at 18 d mod 64, so the 16 (32) rows of one read cycle hit
// distinct banks, and a lane's K fragments of the 4 k-steps sit at constant offsets from one
// base address (immediate offsets, one address register).
constexpr int kKPitch = 144;                        // bytes per K row
constexpr int kKBytes = kBKV * kKPitch;             // 4608
constexpr int kVtPitch = 72;                        // bytes per V^T row
constexpr int kVtBytes = kHD * kVtPitch;            // 4608
constexpr int kStageBytes = 2 * kKBytes + 2 * kVtBytes;  // 18432
constexpr size_t kLdsBytes = 2 * kStageBytes;             // 36864, two stages
// Dropout: each wave's 32 x 32 block of mask factors passes through a wave-private LDS area
// (32 rows, 144-byte pitch: row r starts at bank 36 r mod 64), written as coalesced 128-byte
// row segments and read back as the lane's 16 factors.
constexpr int kMaskPitch = 144;
constexpr int kMaskWaveBytes = 32 * kMaskPitch;           // 4608
constexpr size_t kLdsBytesDrop = kLdsBytes + 4 * kMaskWaveBytes;  // 55296

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 2^x with the hardware exp2 (v_exp_f32, ~1 ulp). Arguments are scores minus a running max, so
// they are <= 0; results below 2^-126 flush to zero, which only drops terms that are at most
// 2^-126 of the row's largest one.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- bf16x3 split ------------------------------------------------------------------------------
// x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest even: |x - hi - lo|
// <= 2^-18 |x|. A product a b is then ah bh + ah bl + al bh (the dropped al bl is below 2^-16 of
// it), three bf16 MFMA products that are exact in fp32. Two fp32 values per call, packed as
// bf16 pairs (element 0 in the low half).
// Returns {hi pair, lo pair}.
__device__ __forceinline__ u32x2_t split2(float x0, float x1) {
  const uint32_t hi = __builtin_bit_cast(uint32_t,
                                         __builtin_convertvector(f32x2_t{x0, x1}, bf16x2_t));
  const float r0 = x0 - __uint_as_float(hi << 16);
  const float r1 = x1 - __uint_as_float(hi & 0xffff0000u);
  return u32x2_t{hi, __builtin_bit_cast(uint32_t,
                                        __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t))};
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// v_mfma_f32_32x32x16_bf16: A (32 x 16) lane l holds row l % 32, k = 8 (l / 32) .. + 7; B (16 x 32)
// lane l holds column l % 32, same k; C element i of lane l is (row 8 (i / 4) + 4 (l / 32) + i % 4,
// column l % 32).
__device__ __forceinline__ f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma3(bf16x8_t ah, bf16x8_t al, bf16x8_t bh, bf16x8_t bl,
                                          f32x16_t c) {
  c = mfma(ah, bh, c);
  c = mfma(ah, bl, c);
  return mfma(al, bh, c);
}

// K/V tile staging: thread t owns key rows 2 (t / 16) and 2 (t / 16) + 1 at d = 4 (t % 16) .. + 3
// of both K and V (four 16-byte global loads, coalesced 256 bytes per 16 threads). K is split and
// written as it lies; V is split and written transposed, the two keys of a d packed in one 32-bit
// store. Rows are permuted in LDS so that both stores are free of bank conflicts, and the
// operand reads apply the same permutations:
//   - key k of K sits in row k_slot(k), k with bits 1 and 3 exchanged: the 32 lanes of one
//     8-byte store cycle write keys 4 u + j and 4 u + 2 + j, which then lie 8 rows (32 banks at
//     the 144-byte pitch) apart instead of 2 rows (24 of their 32 banks shared); the 16 keys of
//     one operand read cycle still fill 16 distinct rows mod 16;
//   - d row of V^T sits in row vt_slot(d) = d ^ 2 for d >= 32: the lanes storing d >= 32
//     (t % 16 >= 8) then sit 4 banks away from the lanes t % 16 - 8 at the 72-byte pitch instead
//     of on the same bank.
__device__ __forceinline__ int k_slot(int k) {
  return (k & ~0xA) | (((k >> 1) & 1) << 3) | (((k >> 3) & 1) << 1);
}
__device__ __forceinline__ int vt_slot(int d) { return d ^ (d >> 4 & 2); }
struct KVLoader {
  const float* k0p;  // this thread's first K row (key 2 (t / 16)) at its column
  const float* v0p;
  int64_t ks, vs;    // row strides (elements)
  int64_t T;

  __device__ KVLoader(const float* k, const float* v, int64_t ks_, int64_t vs_, int64_t T_)
      : ks(ks_), vs(vs_), T(T_) {
    const int pr = threadIdx.x >> 4, col = (threadIdx.x & 15) * 4;
    k0p = k + 2 * pr * ks + col;
    v0p = v + 2 * pr * vs + col;
  }
  // Rows at or past T (only in the last tile) read row T - 1, always in bounds, and are zeroed
  // by value, so the loads stay unconditional 16-byte global loads.
  __device__ void load(int64_t k0, f32x4_t (&rk)[2], f32x4_t (&rv)[2]) const {
    const float* kp = k0p + k0 * ks;
    const float* vp = v0p + k0 * vs;
    if (k0 + kBKV <= T) {  // whole tile in range (uniform)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        rk[j] = *reinterpret_cast<const f32x4_t*>(kp + j * ks);
        rv[j] = *reinterpret_cast<const f32x4_t*>(vp + j * vs);
      }
      return;
    }
    const int pr = threadIdx.x >> 4;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t row = k0 + 2 * pr + j;
      const int64_t back = row < T ? 0 : row - (T - 1);  // rows to step back to T - 1
      rk[j] = *reinterpret_cast<const f32x4_t*>(kp + (j - back) * ks);
      rv[j] = *reinterpret_cast<const f32x4_t*>(vp + (j - back) * vs);
      if (row >= T) rk[j] = rv[j] = f32x4_t{};
    }
  }
  __device__ static void store(char* st, const f32x4_t (&rk)[2], const f32x4_t (&rv)[2]) {
    const int pr = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 4;
    char* kh = st;
    char* kl = st + kKBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int key = 2 * pr + j;
      const u32x2_t s0 = split2(rk[j].x, rk[j].y), s1 = split2(rk[j].z, rk[j].w);
      const u32x2_t h = {s0.x, s1.x}, l = {s0.y, s1.y};
      const int off = k_slot(key) * kKPitch + d0 * 2;
      *reinterpret_cast<u32x2_t*>(kh + off) = h;
      *reinterpret_cast<u32x2_t*>(kl + off) = l;
    }
    char* vh = st + 2 * kKBytes;
    char* vl = vh + kVtBytes;
    const float a[4] = {rv[0].x, rv[0].y, rv[0].z, rv[0].w};
    const float c[4] = {rv[1].x, rv[1].y, rv[1].z, rv[1].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2_t hl = split2(a[i], c[i]);  // keys 2 pr and 2 pr + 1 of d0 + i
      const int off = vt_slot(d0 + i) * kVtPitch + 4 * pr;
      *reinterpret_cast<uint32_t*>(vh + off) = hl.x;
      *reinterpret_cast<uint32_t*>(vl + off) = hl.y;
    }
  }
};

// Work order. Workgroup L of the 1-D grid gets item snake(L): with P = number of CUs, round
// r = L / P is traversed forwards for even r and backwards for odd r (a boustrophedon). Items
// are numbered heaviest first (under causal masking q-tile nqt-1 of every (batch, head) first,
// then q-tile nqt-2, ...). When the whole grid is resident at once and the dispatcher places
// workgroup L on CU L % P, CU j receives items j, 2P-1-j, 2P+j, ...: heavy, light, heavy...,
// which evens out the per-CU sums; any placement still computes every item exactly once.
__device__ __forceinline__ int snake_item(int L, int n, int P) {
  const int r = L / P, j = L - r * P;
  if ((r & 1) == 0) return L;
  const int m = min(P, n - r * P);  // items in this round
  return r * P + (m - 1 - j);
}

// Per 32-key tile and wave (32 queries):
//   S^T = K Q^T: one 32 x 32 accumulator block, 4 k-steps of 16 d, 3 MFMAs each (bf16x3);
//   P^T = exp2(S^T - m) stays in that block: lane (q = l % 32, h = l / 32) holds keys
//     8 (i / 4) + 4 h + i % 4, i = 0..15;
//   O^T += V^T P^T: two 32 x 32 blocks (d halves), 2 k-steps of 16 keys, 3 MFMAs each.
// The P V product sums over keys in any order, so its k index runs over the keys in the order
// the lane already holds them: k-step s, k = 8 h + j is key 16 s + 4 h + j (j < 4) or
// 16 s + 8 + 4 h + (j - 4). The B operand of k-step s is then P elements 8 s .. 8 s + 7 as they
// are, and the V^T fragment is two 8-byte reads at those key offsets.
// DROP: the reference's dropout path (fused_attn…:316-334): each exp term is multiplied by
// dropout_mask[(bh*T + q)*T + key] before it enters the row sum, so O is normalised by the
// post-dropout sum and a row with nothing kept gets O = 0 and LSE = -inf. mvec: mask rows are
// 16-byte aligned (T % 4 == 0, aligned base), so four keys load at once.
template <bool DROP>
__global__ __launch_bounds__(256, DROP ? 2 : 3) void attn_fwd_kernel(hk_attn_fwd_params p,
                                                                     int nbh, int ncu, int mvec) {
  extern __shared__ __attribute__((aligned(16))) char lds[];

  const int64_t T = p.T;
  const int nqt = static_cast<int>((T + kBQ - 1) / kBQ);
  const int item = snake_item(static_cast<int>(blockIdx.x), nqt * nbh, ncu);
  const int qt = nqt - 1 - item / nbh;
  const int bh = item - (nqt - 1 - qt) * nbh;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const float* Qb = p.Q + b * p.q_strideB + h * p.q_strideH;
  float* Ob = p.O + b * p.o_strideB + h * p.o_strideH;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int hh = lane >> 5;
  const int64_t q0w = static_cast<int64_t>(qt) * kBQ + wave * 32;
  const int64_t q = q0w + c;

  // Q^T operands (B of S^T = K Q^T): k-step s holds d = 16 s + 8 hh .. + 7 of query q, scaled so
  // that scores are in log2 units, split into bf16 hi / lo.
  bf16x8_t qh[4], ql[4];
  {
    const float qs = p.scale * kLog2e;
    const float* qp = Qb + (q < T ? q : T - 1) * p.q_strideM + 8 * hh;  // row T-1: in bounds
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(qp + 16 * s);
      f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(qp + 16 * s + 4);
      if (q >= T) v0 = v1 = f32x4_t{};
      const u32x2_t a0 = split2(v0.x * qs, v0.y * qs), a1 = split2(v0.z * qs, v0.w * qs);
      const u32x2_t a2 = split2(v1.x * qs, v1.y * qs), a3 = split2(v1.z * qs, v1.w * qs);
      qh[s] = as_bf16x8(u32x4_t{a0.x, a1.x, a2.x, a3.x});
      ql[s] = as_bf16x8(u32x4_t{a0.y, a1.y, a2.y, a3.y});
    }
  }

  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};  // O^T: d = 32 db + 8 (i/4) + 4 hh + i%4
  float m = -INFINITY, l = 0.f;

  const int64_t kv_end = p.is_causal ? (static_cast<int64_t>(qt) * kBQ + kBQ < T ? static_cast<int64_t>(qt) * kBQ + kBQ : T) : T;
  const int nkv = static_cast<int>((kv_end + kBKV - 1) / kBKV);
  const KVLoader ld(p.K + b * p.k_strideB + h * p.k_strideH,
                    p.V + b * p.v_strideB + h * p.v_strideH, p.k_strideM, p.v_strideM, T);
  f32x4_t rk[2], rv[2];
  // per-lane LDS offsets: K fragment (key c, d = 16 s + 8 hh), V^T fragments (row 32 db + c)
  const int k_row = k_slot(c) * kKPitch + 16 * hh;
  const int vt_row[2] = {vt_slot(c) * kVtPitch + 8 * hh, vt_slot(32 + c) * kVtPitch + 8 * hh};
  // a wave whose queries all precede key tile kt has nothing to add there (causal)
  auto active = [&](int kt) {
    return !p.is_causal || static_cast<int64_t>(kt) * kBKV <= q0w + 31;
  };
  // Scores of a tile relative to the running reference m: the accumulator starts at -m (0
  // while this query has no reference yet), so the MFMAs deliver s - m directly.
  auto base_of = [&](float mm) { return mm == -INFINITY ? 0.f : -mm; };
  // K fragments are read one k-step ahead of their MFMAs (the sched_group_barrier sequence
  // keeps the compiler from sinking each read next to its use, which would expose the full LDS
  // latency before every MFMA).
  auto qk = [&](const char* st, float c0) {
    f32x16_t sc = c0 + f32x16_t{};  // splat
    bf16x8_t kh[4], kl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int off = k_row + 32 * ks;
      kh[ks] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(st + off));
      kl[ks] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(st + kKBytes + off));
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sc = mfma3(kh[ks], kl[ks], qh[ks], ql[ks], sc);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
    return sc;
  };

  // Online softmax with a lazily moved reference (log2 units): m changes only when a tile's
  // scores exceed it by more than kTau or on the query's first tile, so exp2(s - m) <= 2^kTau
  // and most tiles need neither a subtraction per score nor a rescale of O.
  constexpr float kTau = 8.f;
  // Dropout factors of key tile kt. mvec (16-byte rows): coalesced, lane L loads part g = row
  // q0w + 8 g + L / 8, keys k0 + 4 (L % 8) .. + 3 (8 lanes per 128-byte row segment), and
  // mask_to_lanes redistributes them through LDS. Otherwise: the lane's own 16 factors (query q,
  // keys k0 + 8 g + 4 hh .. + 3), element by element.
  auto load_mask = [&](int kt, float4 (&mk)[4]) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBKV;
    if (mvec) {
      const int64_t key = k0 + 4 * (lane & 7);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t r = q0w + 8 * g + (lane >> 3);
        mk[g] = r < T && key < T ? *reinterpret_cast<const float4*>(
                                       p.dropout_mask + (static_cast<int64_t>(bh) * T + r) * T + key)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      return;
    }
    const float* mrow = p.dropout_mask + (static_cast<int64_t>(bh) * T + q) * T;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t key = k0 + 8 * g + 4 * hh;
      const bool ok = q < T;
      mk[g].x = ok && key + 0 < T ? mrow[key + 0] : 0.f;
      mk[g].y = ok && key + 1 < T ? mrow[key + 1] : 0.f;
      mk[g].z = ok && key + 2 < T ? mrow[key + 2] : 0.f;
      mk[g].w = ok && key + 3 < T ? mrow[key + 3] : 0.f;
    }
  };
  // mvec: the coalesced parts -> this lane's factors (query c, keys 8 g + 4 hh .. + 3). The
  // wave's LDS area is reused every tile; a wave's LDS operations complete in order, so the
  // reads of one tile precede the writes of the next.
  auto mask_to_lanes = [&](float4 (&mk)[4]) {
    if (!mvec) return;
    char* reg = lds + kLdsBytes + wave * kMaskWaveBytes;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(reg + (8 * g + (lane >> 3)) * kMaskPitch + 16 * (lane & 7)) =
          mk[g];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      mk[g] = *reinterpret_cast<const float4*>(reg + c * kMaskPitch + (8 * g + 4 * hh) * 4);
  };
  auto softmax_pv = [&](int kt, f32x16_t& sc, float c0, const char* st, const float4 (&mk)[4]) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBKV;
    // V^T fragments (keys 16 ks + 4 hh .. + 3 and 16 ks + 8 + 4 hh .. + 3 of row d = 32 db + c,
    // hi and lo) are read ahead of the exps, so that the exp / split work covers their LDS
    // latency.
    const char* vh = st + 2 * kKBytes;
    const char* vl = vh + kVtBytes;
    u32x4_t vfh[2][2], vfl[2][2];
    auto vread = [&](int db) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int off = vt_row[db] + 32 * ks;
        const u32x2_t a0 = *reinterpret_cast<const u32x2_t*>(vh + off);
        const u32x2_t a1 = *reinterpret_cast<const u32x2_t*>(vh + off + 16);
        const u32x2_t b0 = *reinterpret_cast<const u32x2_t*>(vl + off);
        const u32x2_t b1 = *reinterpret_cast<const u32x2_t*>(vl + off + 16);
        vfh[db][ks] = u32x4_t{a0.x, a0.y, a1.x, a1.y};
        vfl[db][ks] = u32x4_t{b0.x, b0.y, b1.x, b1.y};
      }
    };
    // scores formed against an older reference are moved onto the current one
    const float cnow = base_of(m);
    if (__builtin_amdgcn_ballot_w64(c0 != cnow) != 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] += cnow - c0;
    }
    // mask (causal: key > query; any: key >= T)
    const bool need_mask = (p.is_causal && k0 + kBKV - 1 > q0w) || k0 + kBKV > T;
    if (need_mask) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t key = k0 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (key >= T || (p.is_causal && key > q)) sc[i] = -INFINITY;
      }
    }
    float mt = sc[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mt = fmaxf(mt, sc[i]);
    mt = hk::half32_reduce(mt, hk::MaxOp{});
    // The reference moves on the query's first tile with an unmasked score, and when a score
    // exceeds it by more than kTau; otherwise (most tiles) it stays.
    const bool first = m == -INFINITY;
    const bool move = mt != -INFINITY && (first || mt > kTau);
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float shift = move ? mt : 0.f;
      const float alpha = move && !first ? fast_exp2(-shift) : 1.f;
      if (move) m = first ? shift : m + shift;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] -= shift;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db] *= alpha;
    }
    vread(0);
    vread(1);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float e = fast_exp2(sc[i]);
      if (DROP) {
        const float4 f = mk[i >> 2];
        const float dm = (i & 3) == 0 ? f.x : (i & 3) == 1 ? f.y : (i & 3) == 2 ? f.z : f.w;
        e = sc[i] == -INFINITY ? 0.f : e * dm;  // masked scores never read their factor
      }
      sc[i] = e;
      ls += e;
    }
    l += ls;
    // P^T operands (B of O^T += V^T P^T): k-step ks = elements 8 ks .. 8 ks + 7, split
    bf16x8_t ph[2], pl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x2_t a0 = split2(sc[8 * ks + 0], sc[8 * ks + 1]);
      const u32x2_t a1 = split2(sc[8 * ks + 2], sc[8 * ks + 3]);
      const u32x2_t a2 = split2(sc[8 * ks + 4], sc[8 * ks + 5]);
      const u32x2_t a3 = split2(sc[8 * ks + 6], sc[8 * ks + 7]);
      ph[ks] = as_bf16x8(u32x4_t{a0.x, a1.x, a2.x, a3.x});
      pl[ks] = as_bf16x8(u32x4_t{a0.y, a1.y, a2.y, a3.y});
    }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        o[db] = mfma3(as_bf16x8(vfh[db][ks]), as_bf16x8(vfl[db][ks]), ph[ks], pl[ks], o[db]);
    // V^T reads ahead of the exps, the exps ahead of the MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x400, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
  };

  // Two LDS stages: step kt forms and finishes tile kt from one stage while the global loads
  // of tile kt + 1 are in flight; they land in the other stage at the end of the step.
  if (nkv > 0) {
    ld.load(0, rk, rv);
    KVLoader::store(lds, rk, rv);
  }
  __syncthreads();
  // dropout: the mask factors of tile kt + 1 are loaded while tile
  // kt is computed
  float4 mk_next[4];
  if (DROP && nkv > 0 && active(0)) load_mask(0, mk_next);
  for (int kt = 0; kt < nkv; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkv;
    if (more) ld.load(static_cast<int64_t>(kt + 1) * kBKV, rk, rv);
    float4 mk[4];
    if (DROP) {
#pragma unroll
      for (int g = 0; g < 4; ++g) mk[g] = mk_next[g];
      if (more && active(kt + 1)) load_mask(kt + 1, mk_next);
      if (active(kt)) mask_to_lanes(mk);
    }
    const char* st = lds + cur * kStageBytes;
    if (active(kt)) {
      const float c0 = base_of(m);
      f32x16_t sc = qk(st, c0);
      softmax_pv(kt, sc, c0, st, mk);
    }
    if (more) KVLoader::store(lds + (cur ^ 1) * kStageBytes, rk, rv);
    __syncthreads();
  }

  const float lt = hk::half32_reduce(l, hk::AddOp{});
  if (q < T) {
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    float* orow = Ob + q * p.o_strideM;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hh;
        *reinterpret_cast<float4*>(orow + d) =
            make_float4(o[db][4 * g + 0] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                        o[db][4 * g + 3] * inv);
      }
    if (hh == 0) {
      float* lse = p.LSE + b * p.lse_strideB + h * p.lse_strideH;
      lse[q] = (m + log2f(lt)) * kLn2;
    }
  }
}

// D[row] = sum_d dO[row][d] * O[row][d]: a wave per 4 rows, 16 lanes per 64-float row.
__global__ __launch_bounds__(256) void attn_precompute_d_kernel(hk_attn_bwd_params p, int hd) {
  const int bh = blockIdx.y;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float s = 0.f;
  if (row < p.T) {
    const float* o = p.O + b * p.o_strideB + h * p.o_strideH + row * p.o_strideM;
    const float* d = p.dO + b * p.do_strideB + h * p.do_strideH + row * p.do_strideM;
    for (int k = sub * 4; k < hd; k += 64) {
      const float4 a = *reinterpret_cast<const float4*>(o + k);
      const float4 g = *reinterpret_cast<const float4*>(d + k);
      s += (a.x * g.x + a.y * g.y) + (a.z * g.z + a.w * g.w);
    }
  }
  s = hk::row16_sum(s);
  if (row < p.T && sub == 0) p.D[b * p.d_strideB + h * p.d_strideH + row] = s;
}

// Any strides: one lane per element pair, 16 lanes per row, scalar loads.
__global__ __launch_bounds__(256) void attn_precompute_d_scalar(hk_attn_bwd_params p, int hd) {
  const int bh = blockIdx.y;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float s = 0.f;
  if (row < p.T) {
    const float* o = p.O + b * p.o_strideB + h * p.o_strideH + row * p.o_strideM;
    const float* d = p.dO + b * p.do_strideB + h * p.do_strideH + row * p.do_strideM;
    for (int k = sub; k < hd; k += 16) s += o[k] * d[k];
  }
  s = hk::row16_sum(s);
  if (row < p.T && sub == 0) p.D[b * p.d_strideB + h * p.d_strideH + row] = s;
}

bool rows_aligned(const void* base, int64_t strideB, int64_t strideH, int64_t strideM) {
  return hk::aligned16(base) && strideB % 4 == 0 && strideH % 4 == 0 && strideM % 4 == 0;
}

}  // namespace

extern "C" hipError_t hk_fused_attn_forward(const hk_attn_fwd_params* params, int head_dim,
                                            hipStream_t stream) {
  HK_CHECK_ARG(params != nullptr);
  const hk_attn_fwd_params& p = *params;
  HK_CHECK_ARG(head_dim == kHD);
  HK_CHECK_ARG(p.B >= 0 && p.nh >= 0 && p.T >= 0);
  if (p.B == 0 || p.nh == 0 || p.T == 0) return hipSuccess;
  HK_CHECK_ARG(p.Q && p.K && p.V && p.O && p.LSE);
  // the reference applies its mask only when both are given (fused_attn…:321)
  const bool drop = p.dropout_p > 0.0f && p.dropout_mask != nullptr;
  const int mvec = drop && p.T % 4 == 0 && hk::aligned16(p.dropout_mask) ? 1 : 0;
  HK_CHECK_ARG(rows_aligned(p.Q, p.q_strideB, p.q_strideH, p.q_strideM) &&
               rows_aligned(p.K, p.k_strideB, p.k_strideH, p.k_strideM) &&
               rows_aligned(p.V, p.v_strideB, p.v_strideH, p.v_strideM) &&
               rows_aligned(p.O, p.o_strideB, p.o_strideH, p.o_strideM));
  const int64_t bh = static_cast<int64_t>(p.B) * p.nh;
  const int64_t nqt = (p.T + kBQ - 1) / kBQ;
  HK_CHECK_ARG(bh * nqt <= INT32_MAX);
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    for (int d = 0; d < 2; ++d) {
      const void* k = d ? reinterpret_cast<const void*>(&attn_fwd_kernel<true>)
                        : reinterpret_cast<const void*>(&attn_fwd_kernel<false>);
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(d ? kLdsBytesDrop : kLdsBytes));
      if (e != hipSuccess) attr = e;
    }
  });
  HK_RETURN_IF_ERROR(attr);
  hipLaunchKernelGGL(drop ? attn_fwd_kernel<true> : attn_fwd_kernel<false>,
                     dim3(static_cast<unsigned>(nqt * bh)), dim3(256),
                     drop ? kLdsBytesDrop : kLdsBytes, stream, p,
                     static_cast<int>(bh), hk::device_cu_count(), mvec);
  return hk::launch_status();
}

extern "C" hipError_t hk_attn_bwd_precompute_D(const hk_attn_bwd_params* params, int head_dim,
                                               hipStream_t stream) {
  HK_CHECK_ARG(params != nullptr);
  const hk_attn_bwd_params& p = *params;
  // The reference instantiates HeadDim in {16, 32, 48, 64, 80, 96, 128, 160, 192, 256}
  // (precompute_D…:93-102); any head_dim in [1, 256] is accepted here. Rows whose start is
  // 16-byte aligned with head_dim % 4 == 0 take 16-byte loads, anything else scalar loads.
  HK_CHECK_ARG(head_dim > 0 && head_dim <= 256);
  HK_CHECK_ARG(p.B >= 0 && p.nh >= 0 && p.T >= 0);
  if (p.B == 0 || p.nh == 0 || p.T == 0) return hipSuccess;
  HK_CHECK_ARG(p.O && p.dO && p.D);
  const int64_t bh = static_cast<int64_t>(p.B) * p.nh;
  HK_CHECK_ARG(bh <= 65535);
  const bool vec = head_dim % 4 == 0 &&
                   rows_aligned(p.O, p.o_strideB, p.o_strideH, p.o_strideM) &&
                   rows_aligned(p.dO, p.do_strideB, p.do_strideH, p.do_strideM);
  hipLaunchKernelGGL(vec ? attn_precompute_d_kernel : attn_precompute_d_scalar,
                     dim3(static_cast<unsigned>((p.T + 15) / 16), static_cast<unsigned>(bh)),
                     dim3(256), 0, stream, p, head_dim);
  return hk::launch_status();
}
