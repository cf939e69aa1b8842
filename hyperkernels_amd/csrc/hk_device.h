// hk_device.h - device-side helpers shared by the gfx950 kernels of this library.
//
// Wavefronts are 64 lanes wide on CDNA4; every reduction helper here assumes it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hk.h"

#define HK_WAVE 64

namespace hk {

// ---- bf16 <-> fp32 -------------------------------------------------------------------------
// bf16 is the upper half of an fp32 bit pattern. fp32 -> bf16 is gfx950's v_cvt_pk_bf16_f32:
// round to nearest even (denormals kept), NaN stays NaN, matching __float2bfloat16_rn on every
// non-NaN value; one instruction converts two values.
typedef float hk_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 hk_bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Two fp32 -> packed bf16x2 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector(hk_f32x2_t{lo, hi}, hk_bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// ---- fp16 <-> fp32 -------------------------------------------------------------------------
// IEEE binary16 through the hardware conversions: v_cvt_f32_f16 is exact and v_cvt_f16_f32
// rounds to nearest even (the default mode), overflowing to inf, like __float2half_rn.
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// ---- streaming (non-temporal) 16-byte accesses ---------------------------------------------
// HIP's float4 / uint4 are structs; the non-temporal builtins need native vector types.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_nt(const float4* p) {
  const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4* p, float4 v) {
  const f32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<f32x4_t*>(p));
}
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(uint4* p, uint4 v) {
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// ---- storage formats ----------------------------------------------------------------------
// Tags for the element types a kernel can read and write; arithmetic is always fp32. `unpack`
// and `pack` convert one 16-byte vector (kPerVec elements) to and from fp32 values.
struct F32 {
  using storage = float;
  static constexpr int kPerVec = 4;
  __device__ static float load(const float* p, int64_t i) { return p[i]; }
  __device__ static void store(float* p, int64_t i, float v) { p[i] = v; }
  __device__ static void unpack(const uint4& r, float* f) {
    f[0] = __uint_as_float(r.x); f[1] = __uint_as_float(r.y);
    f[2] = __uint_as_float(r.z); f[3] = __uint_as_float(r.w);
  }
  __device__ static uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                      __float_as_uint(f[3]));
  }
};

// 16-bit formats: element 2k of a vector is the low half of 32-bit word k.
template <float (*ToF32)(uint16_t), uint16_t (*FromF32)(float)>
struct Half16 {
  using storage = uint16_t;
  static constexpr int kPerVec = 8;
  __device__ static float load(const uint16_t* p, int64_t i) { return ToF32(p[i]); }
  __device__ static void store(uint16_t* p, int64_t i, float v) { p[i] = FromF32(v); }
  __device__ static void unpack(const uint4& r, float* f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = ToF32(static_cast<uint16_t>(w[k]));
      f[2 * k + 1] = ToF32(static_cast<uint16_t>(w[k] >> 16));
    }
  }
  __device__ static uint32_t pack2(float lo, float hi) {
    if constexpr (FromF32 == f32_to_bf16) {
      return pack_bf16x2(lo, hi);  // one v_cvt_pk_bf16_f32 for the pair
    } else {
      return static_cast<uint32_t>(FromF32(lo)) | (static_cast<uint32_t>(FromF32(hi)) << 16);
    }
  }
  __device__ static uint4 pack(const float* f) {
    return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
  }
};
using BF16 = Half16<bf16_to_f32, f32_to_bf16>;
using F16 = Half16<f16_to_f32, f32_to_f16>;

// Pairwise sum of an fp32 array of length P (a power of two): ((f0 + f1) + (f2 + f3)) + ...
template <int P>
__device__ __forceinline__ float tree_sum(const float* f) {
  if constexpr (P == 1) {
    return f[0];
  } else {
    return tree_sum<P / 2>(f) + tree_sum<P / 2>(f + P / 2);
  }
}

// ---- wave reductions (64 lanes, butterfly: every lane ends with the result) ----------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, HK_WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, HK_WAVE));
  return v;
}

// ---- (max, sum-of-exp) pair used by the streaming softmax ----------------------------------
// Merges two partial states (m, s) with s = sum exp(x - m). An empty state has m = -inf, s = 0.
__device__ __forceinline__ void softmax_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
  m = mn;
}
__device__ __forceinline__ void wave_softmax_merge(float& m, float& s) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, HK_WAVE);
    const float s2 = __shfl_xor(s, off, HK_WAVE);
    softmax_merge(m, s, m2, s2);
  }
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

}  // namespace hk
