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
// queries. Products run on the fp32 MFMA v_mfma_f32_32x32x2_f32 (exact fp32 products; the
// reference rounds operands to TF32). The score tile is formed transposed, S^T = K Q^T, so
// each lane owns one query column: the online-softmax max is one 32-value register reduction
// plus a single cross-half shuffle, the rescale factor is per lane, and the exponentiated
// scores are already laid out as the B operand of the next product, O^T += V^T P^T, which
// keeps O^T per lane as well (no LDS round trip of P, no cross-lane gathers of the rescale).
// Q stays in registers (pre-scaled by scale * log2 e, so the softmax uses the hardware exp2); K
// and V tiles of 32 keys go through two LDS stages, K as [key][d] and V transposed as [d][key]
// (rows padded to 68 / 36 floats: conflict-free 16-byte fragment reads), with the next tile's
// global loads in flight. 35 KB of LDS and <= 168 VGPRs per workgroup let 3 workgroups share a
// CU, so the BASELINE grid (768 workgroups) runs in one round on 256 CUs. Causal workgroups stop
// at the diagonal; their order is described at snake_item.
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
constexpr int kBQ = 128;                 // queries per workgroup (4 waves x 32)
constexpr int kBKV = 32;                 // keys per K/V tile
constexpr int kKPitch = kHD + 4;         // K tile [key][d] row pitch (floats)
constexpr int kVPitch = kBKV + 4;        // V^T tile [d][key] row pitch (floats)
constexpr int kKFloats = kBKV * kKPitch;
constexpr int kVFloats = kHD * kVPitch;
constexpr int kStageFloats = kKFloats + kVFloats;
constexpr size_t kLdsBytes = 2 * kStageFloats * sizeof(float);  // two stages, 35,840 bytes
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 2^x with the hardware exp2 (v_exp_f32, ~1 ulp). Arguments are scores minus a running max, so
// they are <= 0; results below 2^-126 flush to zero, which only drops terms that are at most
// 2^-126 of the row's largest one.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K/V tile loader: 32 keys x 64 floats of each of K and V = 512 16-byte vectors per tensor;
// thread t moves vectors t and t + 256 (key f / 16, d (f % 16) * 4). K is stored as it lies
// ([key][d], pitch 68), V transposed ([d][key], pitch 36) so that the P V product reads four
// consecutive keys of one d with one 16-byte LDS read.
struct KVLoader {
  const float* k;
  const float* v;
  int64_t ks, vs;  // row strides (elements)
  int64_t T;

  __device__ void load(int64_t k0, float4 (&rk)[2], float4 (&rv)[2]) const {
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int f = threadIdx.x + 256 * j;
      const int64_t row = k0 + (f >> 4);
      const int col = (f & 15) * 4;
      rk[j] = row < T ? *reinterpret_cast<const float4*>(k + row * ks + col) : zero;
      rv[j] = row < T ? *reinterpret_cast<const float4*>(v + row * vs + col) : zero;
    }
  }
  __device__ static void store(float* st, const float4 (&rk)[2], const float4 (&rv)[2]) {
    float* sk = st;
    float* svt = st + kKFloats;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int f = threadIdx.x + 256 * j;
      const int key = f >> 4, d = (f & 15) * 4;
      *reinterpret_cast<float4*>(sk + key * kKPitch + d) = rk[j];
      svt[(d + 0) * kVPitch + key] = rv[j].x;
      svt[(d + 1) * kVPitch + key] = rv[j].y;
      svt[(d + 2) * kVPitch + key] = rv[j].z;
      svt[(d + 3) * kVPitch + key] = rv[j].w;
    }
  }
};

// Per 32-key tile and wave (32 queries): S^T = K Q^T is one 32 x 32 accumulator block (32 MFMAs
// over d), P^T = exp2(S^T - m) stays in that block's registers, and O^T += V^T P^T is two
// blocks (d halves) of 16 MFMAs each. Accumulator element i of a lane (query c = lane % 32,
// half hh = lane / 32) covers key 8 (i / 4) + 4 hh + i % 4 of the tile.
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

// DROP: the reference's dropout path (fused_attn…:316-334): each exp term is multiplied by
// dropout_mask[(bh*T + q)*T + key] before it enters the row sum, so O is normalised by the
// post-dropout sum and a row with nothing kept gets O = 0 and LSE = -inf. mvec: mask rows are
// 16-byte aligned (T % 4 == 0, aligned base), so four keys load at once.
// The mask factors take 16 more VGPRs: the dropout form runs 2 workgroups per CU, not 3.
template <bool DROP>
__global__ __launch_bounds__(256, DROP ? 2 : 3) void attn_fwd_kernel(hk_attn_fwd_params p,
                                                                     int nbh, int ncu, int mvec) {
  extern __shared__ __attribute__((aligned(16))) float lds[];

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

  // Q row (this lane's half of the head dim), scaled so that scores are in log2 units.
  float qr[32];
  {
    const float qs = p.scale * kLog2e;
    const float* qp = Qb + q * p.q_strideM + 32 * hh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 v = q < T ? *reinterpret_cast<const float4*>(qp + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
      qr[4 * j + 0] = v.x * qs;
      qr[4 * j + 1] = v.y * qs;
      qr[4 * j + 2] = v.z * qs;
      qr[4 * j + 3] = v.w * qs;
    }
  }

  f32x16_t o[2] = {f32x16_t{}, f32x16_t{}};  // O^T: d = 32 db + 8 (i/4) + 4 hh + i%4
  float m = -INFINITY, l = 0.f;

  const int64_t kv_end = p.is_causal ? (static_cast<int64_t>(qt) * kBQ + kBQ < T ? static_cast<int64_t>(qt) * kBQ + kBQ : T) : T;
  const int nkv = static_cast<int>((kv_end + kBKV - 1) / kBKV);
  KVLoader ld{p.K + b * p.k_strideB + h * p.k_strideH, p.V + b * p.v_strideB + h * p.v_strideH,
              p.k_strideM, p.v_strideM, T};
  float4 rk[2], rv[2];
  if (nkv > 0) {
    ld.load(0, rk, rv);
    KVLoader::store(lds, rk, rv);
  }
  __syncthreads();

  for (int kt = 0; kt < nkv; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkv;
    if (more) ld.load(static_cast<int64_t>(kt + 1) * kBKV, rk, rv);
    const int64_t k0 = static_cast<int64_t>(kt) * kBKV;
    const float* k_st = lds + cur * kStageFloats;
    const float* vt_st = k_st + kKFloats;
    // a wave whose queries all precede this tile has nothing to add (causal)
    if (!p.is_causal || k0 <= q0w + 31) {
      // dropout factors of this lane's 16 scores, loaded first so the score MFMAs hide them
      float4 mk[4];
      if (DROP) {
        const float* mrow = p.dropout_mask + (static_cast<int64_t>(bh) * T + q) * T;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t key = k0 + 8 * g + 4 * hh;
          if (q < T && mvec) {
            mk[g] = key < T ? *reinterpret_cast<const float4*>(mrow + key)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
          } else {
            const bool ok = q < T;
            mk[g].x = ok && key + 0 < T ? mrow[key + 0] : 0.f;
            mk[g].y = ok && key + 1 < T ? mrow[key + 1] : 0.f;
            mk[g].z = ok && key + 2 < T ? mrow[key + 2] : 0.f;
            mk[g].w = ok && key + 3 < T ? mrow[key + 3] : 0.f;
          }
        }
      }
      f32x16_t s = f32x16_t{};
      const float* krow = k_st + c * kKPitch + 32 * hh;
      float4 kf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) kf[j] = *reinterpret_cast<const float4*>(krow + 4 * j);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j].x, qr[4 * j + 0], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j].y, qr[4 * j + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j].z, qr[4 * j + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[j].w, qr[4 * j + 3], s, 0, 0, 0);
      }
      // V^T operands of this tile: row d = 32 db + c, keys 8 g + 4 hh .. +3
      float4 vf[2][4];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          vf[db][g] = *reinterpret_cast<const float4*>(vt_st + (32 * db + c) * kVPitch + 8 * g + 4 * hh);
      // mask (causal: key > query; any: key >= T), tile max over this query's 32 keys
      const bool need_mask = (p.is_causal && k0 + kBKV - 1 > q0w) || k0 + kBKV > T;
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t key = k0 + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (key >= T || (p.is_causal && key > q)) s[i] = -INFINITY;
        }
      }
      float mt = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mt = fmaxf(mt, s[i]);
      mt = fmaxf(mt, __shfl_xor(mt, 32, HK_WAVE));
      const float m_new = fmaxf(m, mt);
      // rows with nothing unmasked so far keep m = -inf and contribute nothing
      const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m - m_new);
      const float mref = (m_new == -INFINITY) ? 0.f : m_new;
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float e = fast_exp2(s[i] - mref);
        if (DROP) {
          const float4 f = mk[i >> 2];
          const float d = (i & 3) == 0 ? f.x : (i & 3) == 1 ? f.y : (i & 3) == 2 ? f.z : f.w;
          e = s[i] == -INFINITY ? 0.f : e * d;  // masked scores never read their factor
        }
        s[i] = e;
        ls += e;
      }
      l = l * alpha + ls;
      m = m_new;
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db] *= alpha;
      // O^T[d][q] += sum_key V^T[d][key] P^T[key][q]
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[db][g].x, s[4 * g + 0], o[db], 0, 0, 0);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[db][g].y, s[4 * g + 1], o[db], 0, 0, 0);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[db][g].z, s[4 * g + 2], o[db], 0, 0, 0);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[db][g].w, s[4 * g + 3], o[db], 0, 0, 0);
        }
    }
    if (more) KVLoader::store(lds + (cur ^ 1) * kStageFloats, rk, rv);
    __syncthreads();
  }

  const float lt = l + __shfl_xor(l, 32, HK_WAVE);
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
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 16);
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
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 16);
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
    for (const void* k : {reinterpret_cast<const void*>(&attn_fwd_kernel<false>),
                          reinterpret_cast<const void*>(&attn_fwd_kernel<true>)}) {
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(kLdsBytes));
      if (e != hipSuccess) attr = e;
    }
  });
  HK_RETURN_IF_ERROR(attr);
  hipLaunchKernelGGL(drop ? attn_fwd_kernel<true> : attn_fwd_kernel<false>,
                     dim3(static_cast<unsigned>(nqt * bh)), dim3(256), kLdsBytes, stream, p,
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
