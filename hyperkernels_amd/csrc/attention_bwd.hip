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
// waves (latency of one hidden behind the other's MFMAs). K and V of the tile are loaded to
// LDS once; query tiles (Q, dO, LSE, D) stream through LDS with the next tile's global loads
// in flight. Per query tile a wave runs, on the fp32 MFMA v_mfma_f32_32x32x2_f32 (exact fp32
// products): S = Q K^T and dP = dO V^T for its 32 x 32 block (accumulators hold one key column
// per lane), P and dS in registers, then its query half's share of dV += P^T dO and
// dK += dS^T Q straight from those accumulators (their register order is the MFMA operand
// order for a contraction over queries). dS goes through LDS once so that dQ = dS K is formed
// per (query block, d block, key half) with lanes along the head dimension; the two key halves
// are summed through LDS and each dQ element receives one atomic add per key tile. The two
// query halves' dK / dV partials are summed through LDS at the end. 128-key tiles mean 8 dQ
// passes per query row at T = 1024 (the reference's 16-key tiles make 64). Workgroups are
// ordered key tile major, so under causal masking the longest ones are dispatched first.
#include <mutex>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kHD = 64;
constexpr int kBKV = 128;                 // keys per workgroup
constexpr int kBQ = 64;                   // queries per inner tile
constexpr int kThreads = 512;             // 8 waves: 4 key groups x 2 query halves
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
// thread t moves vectors t + 512 j. Rows at or beyond T read as zero.
template <int NV>
__device__ __forceinline__ void load_rows(const float* base, int64_t stride, int64_t r0,
                                          int64_t T, float4 (&reg)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int f = threadIdx.x + kThreads * j;
    const int64_t row = r0 + (f >> 4);
    reg[j] = row < T ? *reinterpret_cast<const float4*>(base + row * stride + (f & 15) * 4)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

template <int NV>
__device__ __forceinline__ void store_rows(float* lds, const float4 (&reg)[NV]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int f = threadIdx.x + kThreads * j;
    *reinterpret_cast<float4*>(lds + (f >> 4) * kPitch + (f & 15) * 4) = reg[j];
  }
}

// Wave w owns key group kg = w % 4 (32 keys) and query half qh = w / 4 (32 of the tile's 64
// queries). Per query tile it forms S and dP for its 32 x 32 block (lane (c, hh) holds key
// column c, queries 8 (i/4) + 4 hh + i%4), turns them into P and dS in registers, and adds its
// query half's share of dV = P^T dO and dK = dS^T Q for its keys. dS goes to LDS; dQ = dS K is
// then split as 4 (query block, d block) pairs x 2 key halves over the 8 waves, the two key
// halves are summed through LDS and one atomic add per dQ element and key tile goes to HBM.
// At the end the two query halves' dK / dV partials of each key group are summed through LDS.
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_kernel(hk_attn_bwd_params p, int nbh) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* sK = lds + kOffK;
  float* sV = lds + kOffV;
  float* sQ = lds + kOffQ;
  float* sdO = lds + kOffdO;
  float* sdS = lds + kOffdS;
  float* sL = lds + kOffL;
  float* sD = lds + kOffD;

  const int64_t T = p.T;
  // Linear order: all (batch, head)s of key tile 0 first, then key tile 1, ... Under causal
  // masking the first key tiles meet the most query tiles, so the hardware's in-order dispatch
  // hands out the longest workgroups first (longest-processing-time-first scheduling).
  const int kt = static_cast<int>(blockIdx.x) / nbh;
  const int bh = static_cast<int>(blockIdx.x) - kt * nbh;
  const int b = bh / p.nh, h = bh - b * p.nh;
  const int64_t k0 = static_cast<int64_t>(kt) * kBKV;

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
  const int kg = wave & 3, qh = wave >> 2;
  const int64_t key = k0 + 32 * kg + c;  // this lane's key column in S / dP
  const float sl2 = p.scale * kLog2e;

  // K and V tiles (128 x 64) once
  {
    float4 r[4];
    load_rows<4>(Kb, p.k_strideM, k0, T, r);
    store_rows<4>(sK, r);
    load_rows<4>(Vb, p.v_strideM, k0, T, r);
    store_rows<4>(sV, r);
  }

  // query tiles: causal starts at the tile holding the first key of this workgroup
  const int64_t q_first = p.is_causal ? (k0 / kBQ) * kBQ : 0;
  const int nq = static_cast<int>((T - q_first + kBQ - 1) / kBQ);

  float4 rq[2], rdo[2];
  float rl = 0.f, rd = 0.f;
  auto fetch = [&](int64_t q0) {
    load_rows<2>(Qb, p.q_strideM, q0, T, rq);
    load_rows<2>(dOb, p.do_strideM, q0, T, rdo);
    if (threadIdx.x < kBQ) {
      const int64_t qq = q0 + threadIdx.x;
      rl = qq < T ? Lb[qq] * kLog2e : 0.f;
      rd = qq < T ? Db[qq] : 0.f;
    }
  };
  if (nq > 0) fetch(q_first);

  f32x16_t dv[2] = {f32x16_t{}, f32x16_t{}};  // dV: key 32 kg + 8(i/4) + 4hh + i%4, d 32db + c
  f32x16_t dk[2] = {f32x16_t{}, f32x16_t{}};

  for (int it = 0; it < nq; ++it) {
    const int64_t q0 = q_first + static_cast<int64_t>(it) * kBQ;
    __syncthreads();  // previous tile's LDS reads are done
    store_rows<2>(sQ, rq);
    store_rows<2>(sdO, rdo);
    if (threadIdx.x < kBQ) {
      sL[threadIdx.x] = rl;
      sD[threadIdx.x] = rd;
    }
    __syncthreads();
    if (it + 1 < nq) fetch(q0 + kBQ);

    // S = Q K^T and dP = dO V^T for this wave's 32 queries x 32 keys
    f32x16_t s = f32x16_t{}, dp = f32x16_t{};
    {
      const float* krow = sK + (32 * kg + c) * kPitch + 32 * hh;
      const float* vrow = sV + (32 * kg + c) * kPitch + 32 * hh;
      const float* qrow = sQ + (32 * qh + c) * kPitch + 32 * hh;
      const float* orow = sdO + (32 * qh + c) * kPitch + 32 * hh;
      // operands of step j + 1 are read while step j multiplies (two register stages)
      float4 xa[2], xb[2];
      xa[0] = *reinterpret_cast<const float4*>(qrow);
      xb[0] = *reinterpret_cast<const float4*>(krow);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j + 1 < 8) {
          xa[(j + 1) & 1] = *reinterpret_cast<const float4*>(qrow + 4 * (j + 1));
          xb[(j + 1) & 1] = *reinterpret_cast<const float4*>(krow + 4 * (j + 1));
        } else {
          xa[0] = *reinterpret_cast<const float4*>(orow);
          xb[0] = *reinterpret_cast<const float4*>(vrow);
        }
        const float4 a = xa[j & 1], bb = xb[j & 1];
        s = mfma(a.x, bb.x, s);
        s = mfma(a.y, bb.y, s);
        s = mfma(a.z, bb.z, s);
        s = mfma(a.w, bb.w, s);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j + 1 < 8) {
          xa[(j + 1) & 1] = *reinterpret_cast<const float4*>(orow + 4 * (j + 1));
          xb[(j + 1) & 1] = *reinterpret_cast<const float4*>(vrow + 4 * (j + 1));
        }
        const float4 a = xa[j & 1], bb = xb[j & 1];
        dp = mfma(a.x, bb.x, dp);
        dp = mfma(a.y, bb.y, dp);
        dp = mfma(a.z, bb.z, dp);
        dp = mfma(a.w, bb.w, dp);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // P and dS in place: register i holds query q0 + 32 qh + 8 (i/4) + 4 hh + i%4.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int qloc = 32 * qh + 8 * g + 4 * hh;
      const float4 lv = *reinterpret_cast<const float4*>(sL + qloc);
      const float4 dv4 = *reinterpret_cast<const float4*>(sD + qloc);
      const float la[4] = {lv.x, lv.y, lv.z, lv.w};
      const float da[4] = {dv4.x, dv4.y, dv4.z, dv4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const int64_t qq = q0 + qloc + e;
        const bool valid = qq < T && key < T && (!p.is_causal || key <= qq);
        // exponent <= ~0 (scores minus the row's log-sum-exp); hardware exp2
        const float pv = valid ? __builtin_amdgcn_exp2f(s[i] * sl2 - la[e]) : 0.f;
        s[i] = pv;
        dp[i] = pv * (dp[i] - da[e]);
      }
    }
    // dV += P^T dO, dK += dS^T Q (contraction over this wave's 32 queries). The dO / Q operands
    // of query group g + 1 are read while group g multiplies; scheduling barriers keep the
    // compiler from hoisting all 64 reads (which would spill).
    {
      float og[2][2][4], qg[2][2][4];
      // per-lane bases; every read below is base + a compile-time offset (one LDS immediate)
      const float* obase = sdO + (32 * qh + 4 * hh) * kPitch + c;
      const float* qbase = sQ + (32 * qh + 4 * hh) * kPitch + c;
      auto rd = [&](int g, int buf) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            og[buf][db][e] = obase[(8 * g + e) * kPitch + 32 * db];
            qg[buf][db][e] = qbase[(8 * g + e) * kPitch + 32 * db];
          }
      };
      rd(0, 0);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (g + 1 < 4) rd(g + 1, (g + 1) & 1);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            dv[db] = mfma(s[4 * g + e], og[g & 1][db][e], dv[db]);
            dk[db] = mfma(dp[4 * g + e], qg[g & 1][db][e], dk[db]);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // dS -> LDS as [query][key]
    {
      float* sbase = sdS + (32 * qh + 4 * hh) * kSPitch + 32 * kg + c;
#pragma unroll
      for (int i = 0; i < 16; ++i) sbase[(8 * (i >> 2) + (i & 3)) * kSPitch] = dp[i];
    }
    __syncthreads();
    // dQ block (queries 32 qb.., d 32 db..), key half kh of this wave = dS[q][keys] K[keys][d]
    const int qb = (wave >> 1) & 1, db = wave & 1, kh = wave >> 2;
    f32x16_t dq = f32x16_t{};
    {
      const float* srow = sdS + (32 * qb + c) * kSPitch + 64 * kh + 32 * hh;
      const float* kcol = sK + (64 * kh + 32 * hh) * kPitch + 32 * db + c;
      float4 sf[2];
      float kk[2][4];
      auto rd = [&](int j, int buf) {
        sf[buf] = *reinterpret_cast<const float4*>(srow + 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) kk[buf][e] = kcol[(4 * j + e) * kPitch];
      };
      rd(0, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j + 1 < 8) rd(j + 1, (j + 1) & 1);
        const float4 a = sf[j & 1];
        dq = mfma(a.x, kk[j & 1][0], dq);
        dq = mfma(a.y, kk[j & 1][1], dq);
        dq = mfma(a.z, kk[j & 1][2], dq);
        dq = mfma(a.w, kk[j & 1][3], dq);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // key half 1 parks its partial in the Q tile's LDS (no longer read this tile); key half 0
    // adds it and issues the atomics.
    float* park = sQ + (wave & 3) * (32 * 33);
    float* pbase = park + 4 * hh * 33 + c;
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) pbase[(8 * (i >> 2) + (i & 3)) * 33] = dq[i];
    }
    __syncthreads();
    if (kh == 0) {
      // per-lane row base; the per-register row steps (8 (i/4) + i%4) * stride are uniform
      const int64_t qrow0 = q0 + 32 * qb + 4 * hh;
      float* dqp = dQb + qrow0 * p.dq_strideM + 32 * db + c;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rs = 8 * (i >> 2) + (i & 3);
        if (qrow0 + rs < T)
          unsafeAtomicAdd(dqp + rs * p.dq_strideM, (dq[i] + pbase[rs * 33]) * p.scale);
      }
    }
  }

  // Sum the two query halves' dK / dV partials of each key group through LDS (the K/V tiles
  // are no longer needed), then store dK (scaled) and dV rows of this wave's keys.
  __syncthreads();
  float* pk = lds + kg * (2 * 32 * 65);  // [2 (dk, dv)][32 keys][65]
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
  hipLaunchKernelGGL(attn_bwd_kernel, dim3(static_cast<unsigned>(nkt * bh)), dim3(kThreads),
                     kLdsBytes, stream, p, static_cast<int>(bh));
  return hk::launch_status();
}
