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

// ---- wave reductions (every lane ends with the result) --------------------------------------
// A butterfly held in registers: within each row of 16 lanes the partner values come through
// DPP (quad_perm [1,0,3,2] and [2,3,0,1], i.e. lane ^ 1 and lane ^ 2, then row_half_mirror,
// lane i <-> 7 - i, and row_mirror, lane i <-> 15 - i), and the four rows are combined with
// gfx950's v_permlane16_swap and v_permlane32_swap, which called with (v, v) return the even
// and the odd row (then the lower and the upper 32 lanes) side by side. Every step pairs
// lanes symmetrically, so with a commutative `op` all lanes end with the same bits; nothing
// goes through LDS (a ds_bpermute butterfly costs six LDS round trips).
namespace detail {
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
}  // namespace detail

// op over the 16 lanes of each row (lanes 16r .. 16r + 15)
template <typename Op>
__device__ __forceinline__ float row16_reduce(float v, Op op) {
  v = op(v, detail::dpp<detail::kDppXor1>(v));
  v = op(v, detail::dpp<detail::kDppXor2>(v));
  v = op(v, detail::dpp<detail::kDppHalfMirror>(v));
  return op(v, detail::dpp<detail::kDppMirror>(v));
}
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = row16_reduce(v, op);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return op(__uint_as_float(h[0]), __uint_as_float(h[1]));
}
struct AddOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, AddOp{}); }
__device__ __forceinline__ float wave_max(float v) { return wave_reduce(v, MaxOp{}); }
__device__ __forceinline__ float row16_sum(float v) { return row16_reduce(v, AddOp{}); }
// op of lane l's value with lane l ^ 32's (one v_permlane32_swap)
template <typename Op>
__device__ __forceinline__ float half32_reduce(float v, Op op) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return op(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

// ---- (max, sum-of-exp) pair used by the streaming softmax ----------------------------------
// Merges two partial states (m, s) with s = sum exp(x - m). An empty state has m = -inf, s = 0.
__device__ __forceinline__ void softmax_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
  m = mn;
}
// The same register butterfly as wave_reduce over (m, s) pairs; softmax_merge is symmetric in
// its two states, so every lane ends with the same pair.
__device__ __forceinline__ void wave_softmax_merge(float& m, float& s) {
  auto step = [&](float m2, float s2) { softmax_merge(m, s, m2, s2); };
  step(detail::dpp<detail::kDppXor1>(m), detail::dpp<detail::kDppXor1>(s));
  step(detail::dpp<detail::kDppXor2>(m), detail::dpp<detail::kDppXor2>(s));
  step(detail::dpp<detail::kDppHalfMirror>(m), detail::dpp<detail::kDppHalfMirror>(s));
  step(detail::dpp<detail::kDppMirror>(m), detail::dpp<detail::kDppMirror>(s));
  auto swap_step = [&](auto sw) {
    const auto pm = sw(__float_as_uint(m)), ps = sw(__float_as_uint(s));
    m = __uint_as_float(pm[0]);
    s = __uint_as_float(ps[0]);
    softmax_merge(m, s, __uint_as_float(pm[1]), __uint_as_float(ps[1]));
  };
  swap_step([](uint32_t v) { return __builtin_amdgcn_permlane16_swap(v, v, false, false); });
  swap_step([](uint32_t v) { return __builtin_amdgcn_permlane32_swap(v, v, false, false); });
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

}  // namespace hk
