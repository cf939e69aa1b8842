// attention_bwd.hip - fused attention backward (key-tile-centric), fp32 I/O, head_dim 64.
//
// Reference behaviour: OwnTensor::mem_efficient_bwd_unified_kernel_exp12<64, Causal>
// (kernels/attention/mem_efficient_bwd_unified_kernel_exp12.cu:54-329): for a tile of keys,
// loop over query tiles; P = exp(scale * Q K^T - LSE), dP = dO V^T, dS = P (dP - D) * scale;
// dV += P^T dO and dK += dS^T Q stay on chip, dQ += dS K is added to global memory atomically
// (the caller zeroes dQ); dK, dV are stored once at the end.
//
// Design (gfx950): one workgroup = 4 waves owns 128 keys of one (batch, head); each wave owns 32
// of them. K and V of the tile are loaded to LDS once. Query tiles of 64 rows (Q, dO, LSE, D)
// stream through LDS with the next tile's loads in flight. Per query tile a wave runs five
// products on the fp32 MFMA v_mfma_f32_32x32x2_f32 (exact fp32 products): S = Q K^T and
// dP = dO V^T for its 32 keys (accumulators hold one key column per lane), then dV += P^T dO
// and dK += dS^T Q straight from those accumulators (their register order is the MFMA operand
// order for a contraction over queries), then dS goes through LDS once so that dQ = dS K is
// formed per query block with lanes along the head dimension, which makes each dQ atomic add a
// contiguous 128-byte row segment. 128-key tiles mean 8 dQ passes per query row at T = 1024
// (the reference's 16-key tiles make 64).
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kHD = 64;
constexpr int kBKV = 128;                 // keys per workgroup
constexpr int kBQ = 64;                   // queries per inner tile
constexpr int kPitch = kHD + 4;           // LDS pitch for [rows][64] tiles (floats)
constexpr int kSPitch = kBKV + 4;         // LDS pitch for the dS tile [64 q][128 keys]
constexpr int kOffK = 0;
constexpr int kOffV = kOffK + kBKV * kPitch;
constexpr int kOffQ = kOffV + kBKV * kPitch;
constexpr int kOffdO = kOffQ + kBQ * kPitch;
constexpr int kOffdS = kOffdO + kBQ * kPitch;
constexpr int kOffL = kOffdS + kBQ * kSPitch;
constexpr int kOffD = kOffL + kBQ;
constexpr int kLdsFloats = kOffD + kBQ;
constexpr size_t kLdsBytes = kLdsFloats * sizeof(float);  // 142,336 bytes
constexpr float kLog2e = 1.4426950408889634f;

typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Loads rows [r0, r0 + n) x 64 floats of a strided [T][64] tensor: 16 lanes per 256-byte row;
// thread t moves vectors t + 256 j. Rows at or beyond T read as zero.
template <int NV>
__device__ __forceinline__ void load_rows(const float* base, int64_t stride, int64_t r0,
                                          int64_t T, float4 (&reg)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int f = threadIdx.x + 256 * j;
    const int64_t row = r0 + (f >> 4);
    reg[j] = row < T ? *reinterpret_cast<const float4*>(base + row * stride + (f & 15) * 4)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

template <int NV>
__device__ __forceinline__ void store_rows(float* lds, const float4 (&reg)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int f = threadIdx.x + 256 * j;
    *reinterpret_cast<float4*>(lds + (f >> 4) * kPitch + (f & 15) * 4) = reg[j];
  }
}

__global__ __launch_bounds__(256, 1) void attn_bwd_kernel(hk_attn_bwd_params p) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* sK = lds + kOffK;
  float* sV = lds + kOffV;
  float* sQ = lds + kOffQ;
  float* sdO = lds + kOffdO;
  float* sdS = lds + kOffdS;
  float* sL = lds + kOffL;
  float* sD = lds + kOffD;

  const int64_t T = p.T;
  const int nkt = static_cast<int>((T + kBKV - 1) / kBKV);
  // causal: the first key tiles see the most query tiles, so they are launched first
  const int kt = static_cast<int>(blockIdx.x);
  const int bh = blockIdx.y;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t k0 = static_cast<int64_t>(kt) * kBKV;
  (void)nkt;

  const float* Qb = p.Q + b * p.q_strideB + h * p.q_strideH;
  const float* Kb = p.K + b * p.k_strideB + h * p.k_strideH;
  const float* Vb = p.V + b * p.v_strideB + h * p.v_strideH;
  const float* dOb = p.dO + b * p.do_strideB + h * p.do_strideH;
  const float* Lb = p.LSE + b * p.lse_strideB + h * p.lse_strideH;
  const float* Db = p.D + b * p.d_strideB + h * p.d_strideH;
  float* dQb = p.dQ + b * p.dq_strideB + h * p.dq_strideH;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int hh = lane >> 5;
  const int64_t key = k0 + 32 * wave + c;  // this lane's key column in S / dP
  const float sl2 = p.scale * kLog2e;

  // K and V tiles (128 x 64) once
  {
    float4 r[8];
    load_rows<8>(Kb, p.k_strideM, k0, T, r);
    store_rows<8>(sK, r);
    load_rows<8>(Vb, p.v_strideM, k0, T, r);
    store_rows<8>(sV, r);
  }

  // query tiles: causal starts at the tile holding the first key of this workgroup
  const int64_t q_first = p.is_causal ? (k0 / kBQ) * kBQ : 0;
  const int nq = static_cast<int>((T - q_first + kBQ - 1) / kBQ);

  float4 rq[4], rdo[4];
  float rl = 0.f, rd = 0.f;
  auto fetch = [&](int64_t q0) {
    load_rows<4>(Qb, p.q_strideM, q0, T, rq);
    load_rows<4>(dOb, p.do_strideM, q0, T, rdo);
    if (threadIdx.x < kBQ) {
      const int64_t qq = q0 + threadIdx.x;
      rl = qq < T ? Lb[qq] * kLog2e : 0.f;
      rd = qq < T ? Db[qq] : 0.f;
    }
  };
  if (nq > 0) fetch(q_first);

  f32x16_t dv[2] = {f32x16_t{}, f32x16_t{}};  // dV: key 32w + 8(i/4) + 4hh + i%4, d 32db + c
  f32x16_t dk[2] = {f32x16_t{}, f32x16_t{}};

  for (int it = 0; it < nq; ++it) {
    const int64_t q0 = q_first + static_cast<int64_t>(it) * kBQ;
    __syncthreads();  // previous tile's LDS reads are done
    store_rows<4>(sQ, rq);
    store_rows<4>(sdO, rdo);
    if (threadIdx.x < kBQ) {
      sL[threadIdx.x] = rl;
      sD[threadIdx.x] = rd;
    }
    __syncthreads();
    if (it + 1 < nq) fetch(q0 + kBQ);

    // S = Q K^T and dP = dO V^T for this wave's 32 keys; lane (c, hh) holds key column c.
    f32x16_t s[2] = {f32x16_t{}, f32x16_t{}};
    f32x16_t dp[2] = {f32x16_t{}, f32x16_t{}};
    {
      const float* krow = sK + (32 * wave + c) * kPitch + 32 * hh;
      const float* vrow = sV + (32 * wave + c) * kPitch + 32 * hh;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 kf = *reinterpret_cast<const float4*>(krow + 4 * j);
        const float4 vf = *reinterpret_cast<const float4*>(vrow + 4 * j);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float4 qf = *reinterpret_cast<const float4*>(sQ + (32 * qb + c) * kPitch + 32 * hh + 4 * j);
          const float4 of = *reinterpret_cast<const float4*>(sdO + (32 * qb + c) * kPitch + 32 * hh + 4 * j);
          s[qb] = mfma(qf.x, kf.x, s[qb]);
          s[qb] = mfma(qf.y, kf.y, s[qb]);
          s[qb] = mfma(qf.z, kf.z, s[qb]);
          s[qb] = mfma(qf.w, kf.w, s[qb]);
          dp[qb] = mfma(of.x, vf.x, dp[qb]);
          dp[qb] = mfma(of.y, vf.y, dp[qb]);
          dp[qb] = mfma(of.z, vf.z, dp[qb]);
          dp[qb] = mfma(of.w, vf.w, dp[qb]);
        }
      }
    }
    // P and dS in place: register (qb, i) holds query q0 + 32 qb + 8 (i/4) + 4 hh + i%4.
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int qloc = 32 * qb + 8 * g + 4 * hh;
        const float4 lv = *reinterpret_cast<const float4*>(sL + qloc);
        const float4 dv4 = *reinterpret_cast<const float4*>(sD + qloc);
        const float la[4] = {lv.x, lv.y, lv.z, lv.w};
        const float da[4] = {dv4.x, dv4.y, dv4.z, dv4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * g + e;
          const int64_t qq = q0 + qloc + e;
          const bool valid = qq < T && key < T && (!p.is_causal || key <= qq);
          const float pv = valid ? exp2f(s[qb][i] * sl2 - la[e]) : 0.f;
          s[qb][i] = pv;
          dp[qb][i] = pv * (dp[qb][i] - da[e]);
        }
      }
    // dV += P^T dO, dK += dS^T Q (contraction over the 64 queries of the tile)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qloc = 32 * qb + 8 * (i >> 2) + 4 * hh + (i & 3);
          const float og = sdO[qloc * kPitch + 32 * db + c];
          const float qg = sQ[qloc * kPitch + 32 * db + c];
          dv[db] = mfma(s[qb][i], og, dv[db]);
          dk[db] = mfma(dp[qb][i], qg, dk[db]);
        }
    // dS -> LDS as [query][key]
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qloc = 32 * qb + 8 * (i >> 2) + 4 * hh + (i & 3);
        sdS[qloc * kSPitch + 32 * wave + c] = dp[qb][i];
      }
    __syncthreads();
    // dQ block (queries 32 qb.., d 32 db..) of this wave = dS[q][all 128 keys] K[keys][d]
    {
      const int qb = wave >> 1, db = wave & 1;
      f32x16_t dq = f32x16_t{};
      const float* srow = sdS + (32 * qb + c) * kSPitch + 64 * hh;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float4 sf = *reinterpret_cast<const float4*>(srow + 4 * j);
        const int kr = 64 * hh + 4 * j;
        dq = mfma(sf.x, sK[(kr + 0) * kPitch + 32 * db + c], dq);
        dq = mfma(sf.y, sK[(kr + 1) * kPitch + 32 * db + c], dq);
        dq = mfma(sf.z, sK[(kr + 2) * kPitch + 32 * db + c], dq);
        dq = mfma(sf.w, sK[(kr + 3) * kPitch + 32 * db + c], dq);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t qq = q0 + 32 * qb + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (qq < T) unsafeAtomicAdd(dQb + qq * p.dq_strideM + 32 * db + c, dq[i] * p.scale);
      }
    }
  }

  // dK (scaled) and dV rows of this wave's keys
  float* dKb = p.dK + b * p.dk_strideB + h * p.dk_strideH;
  float* dVb = p.dV + b * p.dv_strideB + h * p.dv_strideH;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t kk = k0 + 32 * wave + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (kk < T) {
        dKb[kk * p.dk_strideM + 32 * db + c] = dk[db][i] * p.scale;
        dVb[kk * p.dv_strideM + 32 * db + c] = dv[db][i];
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
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kLdsBytes));
  });
  HK_RETURN_IF_ERROR(attr);
  const unsigned nkt = static_cast<unsigned>((static_cast<int64_t>(p.T) + kBKV - 1) / kBKV);
  hipLaunchKernelGGL(attn_bwd_kernel, dim3(nkt, static_cast<unsigned>(bh)), dim3(256), kLdsBytes,
                     stream, p);
  return hk::launch_status();
}
