// gelu.hip - tanh-approximation GELU forward/backward, fp32 math, fp32, bf16 or fp16 I/O.
//
// Reference behaviour: kernels/gelu/gelu_forward_sm89_kernel.cu:19-22 (forward formula) and
// kernels/gelu/gelu_backward_sm89_kernel.cu:24-30 (analytic derivative). The reference uses the
// PTX tanh.approx instruction; this file never forms tanh itself: the formula only needs
// 1 + tanh(u) and 1 - tanh(u)^2, which are evaluated through the logistic function
// (1 + tanh(u)) / 2 = 1 / (1 + exp(-2u)) with relative error of a few ulp everywhere.
//
// The three storage types are the reference's instantiations (gelu_forward_sm89_kernel.cu:78-80;
// gelu_backward_sm89_kernel.cu:88-90); 16-bit results are rounded to nearest even.
//
// HBM layout: flat contiguous tensors. Each lane moves 16 bytes per access (8 bf16 / fp16 or
// 4 fp32), one vector per lane, so every wave issues fully coalesced 1 KiB transactions. One
// vector per lane measured fastest on MI355X at the GPT-2 shape (25.2 M bf16: 22 us forward,
// 28.5 us backward, against 30 / 33 us with four): many short workgroups ramp the device up
// and drain it faster. Workgroup sizes from a sweep of plain streams at this size: the
// 1-read / 1-write forward is fastest with 64 lanes (17.1 us against 17.9 us at 256), the
// 2-read / 1-write backward with 512 (24.9 against 25.2 us); in the kernels, fp16 forward
// 18.1 -> 17.3 us and backward 25.7 -> 25.5 us.
#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;        // scalar kernels
constexpr int kFwdVecThreads = 64;   // vector forward: 1 read, 1 write per vector
constexpr int kBwdVecThreads = 512;  // vector backward: 2 reads, 1 write
constexpr int kUnroll = 1;

// With u = c (x + a x^3) (c = sqrt(2/pi), a = 0.044715, the Hendrycks & Gimpel tanh fit):
// (1 + tanh(u)) / 2 = sigmoid(2u) = 1 / (1 + 2^(-2 log2(e) u)): no cancellation for u << 0,
// where 1 + tanh(u) formed from a rounded tanh loses most of its digits. The exponent is
// -2 log2(e) u = x (k1 + k2 x^2) with the constants folded (float64-rounded once):
//   k1 = -2 log2(e) c, k2 = k1 a.
// 2^t overflow (x << 0) gives s = 0 and underflow (x >> 0) gives s = 1, the correct limits.
// v_exp_f32 is the hardware 2^t (about 1 ulp) and v_rcp_f32 the hardware reciprocal (1 ulp):
// s carries a few ulp of relative error everywhere.
constexpr float kK1 = -2.302208198144325f;   // -2 log2(e) sqrt(2/pi)
constexpr float kK2 = -0.1029432395800235f;  // kK1 * 0.044715
constexpr float kC = 0.7978845608028654f;    // sqrt(2/pi)
constexpr float kC3a = 0.10703222440890f;    // 3 * 0.044715 * sqrt(2/pi)

__device__ __forceinline__ float sigmoid_2u(float x, float x2) {
  const float t = x * __builtin_fmaf(kK2, x2, kK1);
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// GELU(x) = 0.5 x (1 + tanh(u)) = x s
__device__ __forceinline__ float gelu_fwd(float x) { return x * sigmoid_2u(x, x * x); }

// GELU'(x) = 0.5 (1 + th) + 0.5 x (1 - th^2) du = s + 2 x du s (1 - s), with s as above,
// 1 - th^2 = (1 - th)(1 + th) = 4 s (1 - s) and du = c (1 + 3 a x^2).
__device__ __forceinline__ float gelu_grad(float x) {
  const float x2 = x * x;
  const float s = sigmoid_2u(x, x2);
  const float two_x_du = 2.0f * x * __builtin_fmaf(kC3a, x2, kC);
  return __builtin_fmaf(two_x_du, __builtin_fmaf(-s, s, s), s);
}

// Vector body: nvec 16-byte vectors, all pointers 16-byte aligned.
template <typename T, int BS>
__global__ __launch_bounds__(BS) void gelu_fwd_vec(const uint4* __restrict__ in,
                                                   uint4* __restrict__ out, int64_t nvec) {
  constexpr int P = T::kPerVec;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * BS * kUnroll + threadIdx.x;
  uint4 r[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * BS;
    if (i < nvec) r[u] = hk::ld_nt(in + i);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * BS;
    if (i < nvec) {
      float f[P];
      T::unpack(r[u], f);
#pragma unroll
      for (int k = 0; k < P; ++k) f[k] = gelu_fwd(f[k]);
      hk::st_nt(out + i, T::pack(f));
    }
  }
}

template <typename T, int BS>
__global__ __launch_bounds__(BS) void gelu_bwd_vec(const uint4* __restrict__ grad,
                                                   const uint4* __restrict__ in,
                                                   uint4* __restrict__ grad_in, int64_t nvec) {
  constexpr int P = T::kPerVec;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * BS * kUnroll + threadIdx.x;
  uint4 rg[kUnroll], rx[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * BS;
    if (i < nvec) {
      rg[u] = hk::ld_nt(grad + i);
      rx[u] = hk::ld_nt(in + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * BS;
    if (i < nvec) {
      float g[P], x[P];
      T::unpack(rg[u], g);
      T::unpack(rx[u], x);
#pragma unroll
      for (int k = 0; k < P; ++k) g[k] = g[k] * gelu_grad(x[k]);
      hk::st_nt(grad_in + i, T::pack(g));
    }
  }
}

// Scalar path: tails and unaligned tensors.
template <typename T, typename S = typename T::storage>
__global__ __launch_bounds__(kThreads) void gelu_fwd_scalar(const S* __restrict__ in,
                                                            S* __restrict__ out, int64_t begin,
                                                            int64_t end) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end;
       i += stride)
    T::store(out, i, gelu_fwd(T::load(in, i)));
}

template <typename T, typename S = typename T::storage>
__global__ __launch_bounds__(kThreads) void gelu_bwd_scalar(const S* __restrict__ grad,
                                                            const S* __restrict__ in,
                                                            S* __restrict__ grad_in,
                                                            int64_t begin, int64_t end) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end;
       i += stride)
    T::store(grad_in, i, T::load(grad, i) * gelu_grad(T::load(in, i)));
}

int scalar_grid(int64_t n) {
  const int64_t blocks = hk::ceil_div(n, kThreads);
  const int64_t cap = static_cast<int64_t>(hk::device_cu_count()) * 8;
  return static_cast<int>(blocks < cap ? (blocks < 1 ? 1 : blocks) : cap);
}

template <typename T, typename S = typename T::storage>
hipError_t launch_fwd(const S* in, S* out, int64_t numel, hipStream_t stream) {
  HK_CHECK_ARG(numel >= 0);
  if (numel == 0) return hipSuccess;
  HK_CHECK_ARG(in != nullptr && out != nullptr);
  constexpr int P = T::kPerVec;
  int64_t done = 0;
  if (hk::aligned16(in) && hk::aligned16(out)) {
    const int64_t nvec = numel / P;
    if (nvec > 0) {
      const int64_t blocks = hk::ceil_div(nvec, int64_t(kFwdVecThreads) * kUnroll);
      HK_CHECK_ARG(blocks <= INT32_MAX);
      hipLaunchKernelGGL((gelu_fwd_vec<T, kFwdVecThreads>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kFwdVecThreads), 0,
                         stream, reinterpret_cast<const uint4*>(in),
                         reinterpret_cast<uint4*>(out), nvec);
      HK_RETURN_IF_ERROR(hk::launch_status());
    }
    done = nvec * P;
  }
  if (done < numel) {
    hipLaunchKernelGGL(gelu_fwd_scalar<T>, dim3(scalar_grid(numel - done)), dim3(kThreads), 0,
                       stream, in, out, done, numel);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  return hipSuccess;
}

template <typename T, typename S = typename T::storage>
hipError_t launch_bwd(const S* grad, const S* in, S* grad_in, int64_t numel,
                      hipStream_t stream) {
  HK_CHECK_ARG(numel >= 0);
  if (numel == 0) return hipSuccess;
  HK_CHECK_ARG(grad != nullptr && in != nullptr && grad_in != nullptr);
  constexpr int P = T::kPerVec;
  int64_t done = 0;
  if (hk::aligned16(grad) && hk::aligned16(in) && hk::aligned16(grad_in)) {
    const int64_t nvec = numel / P;
    if (nvec > 0) {
      const int64_t blocks = hk::ceil_div(nvec, int64_t(kBwdVecThreads) * kUnroll);
      HK_CHECK_ARG(blocks <= INT32_MAX);
      hipLaunchKernelGGL((gelu_bwd_vec<T, kBwdVecThreads>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kBwdVecThreads), 0,
                         stream, reinterpret_cast<const uint4*>(grad),
                         reinterpret_cast<const uint4*>(in), reinterpret_cast<uint4*>(grad_in),
                         nvec);
      HK_RETURN_IF_ERROR(hk::launch_status());
    }
    done = nvec * P;
  }
  if (done < numel) {
    hipLaunchKernelGGL(gelu_bwd_scalar<T>, dim3(scalar_grid(numel - done)), dim3(kThreads), 0,
                       stream, grad, in, grad_in, done, numel);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  return hipSuccess;
}

}  // namespace

extern "C" hipError_t hk_gelu_forward_f32(const float* in, float* out, int64_t numel,
                                          hipStream_t stream) {
  return launch_fwd<hk::F32>(in, out, numel, stream);
}
extern "C" hipError_t hk_gelu_forward_bf16(const hk_bf16* in, hk_bf16* out, int64_t numel,
                                           hipStream_t stream) {
  return launch_fwd<hk::BF16>(in, out, numel, stream);
}
extern "C" hipError_t hk_gelu_forward_f16(const hk_f16* in, hk_f16* out, int64_t numel,
                                          hipStream_t stream) {
  return launch_fwd<hk::F16>(in, out, numel, stream);
}
extern "C" hipError_t hk_gelu_backward_f32(const float* grad, const float* in, float* grad_in,
                                           int64_t numel, hipStream_t stream) {
  return launch_bwd<hk::F32>(grad, in, grad_in, numel, stream);
}
extern "C" hipError_t hk_gelu_backward_bf16(const hk_bf16* grad, const hk_bf16* in,
                                            hk_bf16* grad_in, int64_t numel,
                                            hipStream_t stream) {
  return launch_bwd<hk::BF16>(grad, in, grad_in, numel, stream);
}
extern "C" hipError_t hk_gelu_backward_f16(const hk_f16* grad, const hk_f16* in,
                                           hk_f16* grad_in, int64_t numel, hipStream_t stream) {
  return launch_bwd<hk::F16>(grad, in, grad_in, numel, stream);
}
