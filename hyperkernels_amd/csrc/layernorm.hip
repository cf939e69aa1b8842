// layernorm.hip - LayerNorm forward / backward over rows [rows, cols] of fp32, bf16 or fp16
// (statistics, gamma/beta gradients and all arithmetic in fp32).
//
// Reference behaviour:
//   forward            kernels/layernorm/layer_norm_forward_sm89_kernel.cu:27-209
//                      mean, rstd = 1/sqrt(var + eps) (biased var), y = (x - mean) * rstd * g + b
//   backward (input)   kernels/layernorm/ln_backward_input_sm89_kernel.cu:33-105
//                      dx = rstd * (dy g - (s1 + xhat s2) / cols), s1 = sum dy g,
//                      s2 = sum dy g xhat
//   backward (g, b)    kernels/layernorm/ln_backward_gamma_beta_sm89_kernel.cu:15-49
//                      dgamma += sum_r dy xhat, dbeta += sum_r dy
//
// Design (gfx950): one 64-lane wave owns one row; when a row is a whole number of 16-byte
// vectors (cols % 4 == 0 for fp32, % 8 for 16-bit) of at most 16 per lane (cols <= 4096 fp32,
// 8192 16-bit) the row is held in VGPRs in its storage format, so x is read from HBM once
// and mean/variance are computed in two exact passes over registers (no Welford merge). The
// gamma/beta gradient is accumulated per lane in registers across the rows a wave visits,
// reduced across the workgroup's waves in LDS, written as one partial per workgroup, and summed over the
// workgroups in a fixed order by a second small kernel: the result is deterministic, unlike
// the reference's atomics. Shapes outside the register path use a workgroup-per-row fallback.
#include <initializer_list>
#include <mutex>
#include <type_traits>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / HK_WAVE;

// Storage type of a format tag, in a form that template argument deduction does not look at.
template <typename T>
using St = typename T::storage;

__device__ __forceinline__ uint4 u4_zero() { return make_uint4(0u, 0u, 0u, 0u); }

// One 16-byte vector of gamma (or beta) as fp32, or `dflt` everywhere when the pointer is NULL.
template <typename T>
__device__ __forceinline__ void affine(const uint4* p, int c, float dflt, float* f) {
  if (p) {
    T::unpack(p[c], f);
  } else {
#pragma unroll
    for (int k = 0; k < T::kPerVec; ++k) f[k] = dflt;
  }
}

// ------------------------------------------------------------------------------------------
// Forward, register-resident rows: VPL 16-byte vectors per lane, nvec vectors per row.
// ------------------------------------------------------------------------------------------
template <typename T, int VPL>
__global__ __launch_bounds__(kThreads) void ln_fwd_reg(const uint4* __restrict__ x,
                                                       const uint4* __restrict__ gamma,
                                                       const uint4* __restrict__ beta,
                                                       uint4* __restrict__ y,
                                                       float* __restrict__ mean_out,
                                                       float* __restrict__ rstd_out, int rows,
                                                       int nvec, float inv_cols, float eps) {
  constexpr int P = T::kPerVec;
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint4* xr = x + static_cast<int64_t>(row) * nvec;
  uint4 v[VPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    v[i] = (c < nvec) ? hk::ld_nt(xr + c) : u4_zero();
    float f[P];
    T::unpack(v[i], f);
    s += hk::tree_sum<P>(f);
  }
  const float mu = hk::wave_sum(s) * inv_cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    if (c < nvec) {
      float f[P];
      T::unpack(v[i], f);
#pragma unroll
      for (int k = 0; k < P; ++k) f[k] = (f[k] - mu) * (f[k] - mu);
      q += hk::tree_sum<P>(f);
    }
  }
  const float var = hk::wave_sum(q) * inv_cols;
  const float rs = 1.0f / sqrtf(var + eps);
  if (lane == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = rs;
  }
  uint4* yr = y + static_cast<int64_t>(row) * nvec;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    if (c < nvec) {
      float f[P], g[P], b[P];
      T::unpack(v[i], f);
      affine<T>(gamma, c, 1.f, g);
      affine<T>(beta, c, 0.f, b);
#pragma unroll
      for (int k = 0; k < P; ++k) f[k] = (f[k] - mu) * rs * g[k] + b[k];
      hk::st_nt(yr + c, T::pack(f));
    }
  }
}

// Waves per workgroup of the backward kernels that accumulate gamma/beta: 8 when the flat
// LDS reduction of 8 waves fits 64 KiB (cols <= 1024), else 4. The grid is one workgroup
// per CU (8 waves) or two (4 waves), so each CU holds 8 waves and writes one or two partials
// for the finalize to read back. Measured at 4096 x 768 on MI355X against 4 waves and two
// workgroups per CU (512 partials): 12.2 against 12.9 us per fused backward (fp32), 9.8
// against 10.7 us (bf16); a tree reduction over the waves instead of the flat one was slower.
constexpr int gb_waves(int cols) { return cols <= 1024 ? 8 : 4; }

// One row per wave: when every row fits one round of 16-wave workgroups, one per CU
// (rows <= CUs x 16, cols <= kOneRowMaxCols<T>, so the flat reduction's 16 x 2 x cols floats fit
// 128 KiB), the gamma/beta backward runs the ONE_ROW form of ln_bwd_reg: no prefetch registers
// (108 VGPRs at 768 fp32 columns, 4 waves per SIMD), each wave's row in flight at once, still
// one partial per CU. fp32 rows of 4 vectors per lane (769-1024 columns) would spill at the
// 128-VGPR limit of 4 waves per SIMD and keep the prefetching form.
// 4096 x 768 fp32 fused backward on MI355X, one buffer set: 11.87 -> 11.27 us per call (the
// kernel alone 8.90 -> 8.37 us); eight such waves with two workgroups per CU made the kernel
// 8.02 us but its 512 partials cost the finalize more than that.
constexpr int kOneRowWaves = 16;
template <typename T>
constexpr int kOneRowMaxCols = T::kPerVec == 4 ? 768 : 1024;

// ------------------------------------------------------------------------------------------
// Backward, register-resident rows. WRITE_DX: produce grad_x. DO_GB: accumulate the
// per-workgroup gamma/beta partials into part[blockIdx.x][2 * cols] (gamma then beta).
// Each wave walks its rows with the next row's dy / x already in flight (software prefetch),
// so the two wave reductions of one row overlap the loads of the next; ONE_ROW drops the
// prefetch (each row is loaded at the top of its iteration) for grids where each wave has one
// row. dy, x and gamma stay in registers in their storage format and are widened to fp32
// where they are used.
// ------------------------------------------------------------------------------------------
template <typename T, int VPL, bool WRITE_DX, bool DO_GB, int WAVES, bool ONE_ROW = false>
__global__ __launch_bounds__(WAVES * HK_WAVE, ONE_ROW ? 4 : 1) void ln_bwd_reg(
    const uint4* __restrict__ dy, const uint4* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const uint4* __restrict__ gamma, uint4* __restrict__ dx,
    float* __restrict__ part, int rows, int nvec, float inv_cols) {
  // Every product below is rounded on its own (as the reference formula is written), so a
  // row whose terms cancel exactly (cols == 1) gives exactly zero.
#pragma clang fp contract(off)
  constexpr int P = T::kPerVec;
  extern __shared__ float4 lds4[];  // [WAVES][2][cols] floats when DO_GB
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int wave = threadIdx.x >> 6;
  uint4 graw[VPL];
  float acc_g[VPL][P], acc_b[VPL][P];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    graw[i] = (gamma && c < nvec) ? gamma[c] : u4_zero();
#pragma unroll
    for (int k = 0; k < P; ++k) acc_g[i][k] = acc_b[i][k] = 0.f;
  }
  const int stride = gridDim.x * WAVES;
  int row = blockIdx.x * WAVES + wave;
  uint4 dn[VPL], xn[VPL];
  float mn = 0.f, rn = 0.f;
  auto fetch = [&](int r) {
    const uint4* dyr = dy + static_cast<int64_t>(r) * nvec;
    const uint4* xr = x + static_cast<int64_t>(r) * nvec;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + i * HK_WAVE;
      dn[i] = (c < nvec) ? hk::ld_nt(dyr + c) : u4_zero();
      xn[i] = (c < nvec) ? hk::ld_nt(xr + c) : u4_zero();
    }
    mn = mean[r];
    rn = rstd[r];
  };
  // dy, x-hat and dy * gamma of vector i of the current row (x-hat is zero past the row end).
  auto widen = [&](const uint4& draw, const uint4& xraw, int i, float m, float rs, float* d,
                   float* n, float* a) {
    const bool in = lane + i * HK_WAVE < nvec;
    float g[P];
    T::unpack(draw, d);
    T::unpack(xraw, n);
    if (gamma) {
      T::unpack(graw[i], g);
    } else {
#pragma unroll
      for (int k = 0; k < P; ++k) g[k] = 1.f;
    }
#pragma unroll
    for (int k = 0; k < P; ++k) {
      n[k] = in ? (n[k] - m) * rs : 0.f;
      a[k] = d[k] * g[k];
    }
  };
  if (!ONE_ROW && row < rows) fetch(row);
  for (; row < rows; row += stride) {
    if (ONE_ROW) fetch(row);
    uint4 dcur[VPL], xcur[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      dcur[i] = dn[i];
      xcur[i] = xn[i];
    }
    const float m = mn, rs = rn;
    if (!ONE_ROW && row + stride < rows) fetch(row + stride);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float d[P], n[P], a[P];
      widen(dcur[i], xcur[i], i, m, rs, d, n, a);
      if (DO_GB) {
#pragma unroll
        for (int k = 0; k < P; ++k) {
          acc_g[i][k] += d[k] * n[k];
          acc_b[i][k] += d[k];
        }
      }
      if (WRITE_DX) {
        s1 += hk::tree_sum<P>(a);
#pragma unroll
        for (int k = 0; k < P; ++k) n[k] = a[k] * n[k];
        s2 += hk::tree_sum<P>(n);
      }
    }
    if (WRITE_DX) {
      const float t1 = hk::wave_sum(s1), t2 = hk::wave_sum(s2);
      uint4* dxr = dx + static_cast<int64_t>(row) * nvec;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = lane + i * HK_WAVE;
        if (c < nvec) {
          float d[P], n[P], a[P], o[P];
          widen(dcur[i], xcur[i], i, m, rs, d, n, a);
#pragma unroll
          for (int k = 0; k < P; ++k) o[k] = rs * (a[k] - (t1 + n[k] * t2) * inv_cols);
          hk::st_nt(dxr + c, T::pack(o));
        }
      }
    }
  }
  if (DO_GB) {
    // LDS holds [wave][gamma | beta][cols] floats; vector c covers columns c*P .. c*P+P-1.
    constexpr int Q = P / 4;  // float4s per vector
    const int cols4 = nvec * Q;
    float4* my = lds4 + static_cast<int64_t>(wave) * 2 * cols4;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + i * HK_WAVE;
      if (c < nvec) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          my[c * Q + q] = make_float4(acc_g[i][4 * q], acc_g[i][4 * q + 1], acc_g[i][4 * q + 2],
                                      acc_g[i][4 * q + 3]);
          my[cols4 + c * Q + q] = make_float4(acc_b[i][4 * q], acc_b[i][4 * q + 1],
                                              acc_b[i][4 * q + 2], acc_b[i][4 * q + 3]);
        }
      }
    }
    __syncthreads();
    float4* out = reinterpret_cast<float4*>(part) + static_cast<int64_t>(blockIdx.x) * 2 * cols4;
    for (int c = threadIdx.x; c < 2 * cols4; c += WAVES * HK_WAVE) {
      float4 s = lds4[c];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) {
        const float4 t = lds4[static_cast<int64_t>(w) * 2 * cols4 + c];
        s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
      }
      out[c] = s;
    }
  }
}

// Sums nparts partials [nparts][2 * cols] in a fixed order and adds them into grad_gamma /
// grad_beta. A workgroup owns kFinCols columns and spreads the partials over kFinGroups lane
// groups: group g sums partials g, g + kFinGroups, ... (eight loads in flight per lane, one
// round for up to 256 partials), then the group sums are added in group order in LDS. Narrow
// column slices spread the read of the partials over 2 x cols / 16 workgroups.
constexpr int kFinCols = 16;
constexpr int kFinGroups = 32;
__global__ __launch_bounds__(kFinCols * kFinGroups) void ln_gb_finalize(
    const float* __restrict__ part, int nparts, int cols, float* __restrict__ grad_gamma,
    float* __restrict__ grad_beta) {
  __shared__ float red[kFinGroups][kFinCols];
  const int col = threadIdx.x % kFinCols;
  const int grp = threadIdx.x / kFinCols;
  const int c = blockIdx.x * kFinCols + col;
  const int width = 2 * cols;
  // The value this thread adds into is loaded before the partials, so its latency overlaps
  // theirs instead of following the reduction (4096 x 768 fp32 fused backward on MI355X:
  // 12.15 -> 11.84 us per call, same bits).
  float* dst = nullptr;
  if (grp == 0 && c < width) dst = c < cols ? (grad_gamma ? grad_gamma + c : nullptr)
                                            : (grad_beta ? grad_beta + (c - cols) : nullptr);
  const float prev = dst ? *dst : 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < width) {
    int p = grp;
    for (; p + 7 * kFinGroups < nparts; p += 8 * kFinGroups) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        acc[u] += part[static_cast<int64_t>(p + u * kFinGroups) * width + c];
    }
    for (; p < nparts; p += kFinGroups) acc[0] += part[static_cast<int64_t>(p) * width + c];
  }
  red[grp][col] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (grp == 0 && c < width) {
    float s = red[0][col];
#pragma unroll
    for (int g = 1; g < kFinGroups; ++g) s += red[g][col];
    if (dst) *dst = prev + s;
  }
}

// ------------------------------------------------------------------------------------------
// Fallback kernels (any cols, any alignment): one workgroup per row, row re-read from cache.
// ------------------------------------------------------------------------------------------
__device__ float block_sum(float v, float* red) {
  v = hk::wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) t += red[w];
  return t;
}

template <typename T, typename S = typename T::storage>
__global__ __launch_bounds__(kThreads) void ln_fwd_rowblock(const S* __restrict__ x,
                                                            const S* __restrict__ gamma,
                                                            const S* __restrict__ beta,
                                                            S* __restrict__ y,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ rstd_out,
                                                            int cols, float eps) {
  __shared__ float red[kWavesPerBlock];
  const int64_t row = blockIdx.x;
  const S* xr = x + row * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) s += T::load(xr, c);
  const float mu = block_sum(s, red) / static_cast<float>(cols);
  float q = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float d = T::load(xr, c) - mu;
    q += d * d;
  }
  const float var = block_sum(q, red) / static_cast<float>(cols);
  const float rs = 1.0f / sqrtf(var + eps);
  if (threadIdx.x == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = rs;
  }
  S* yr = y + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float g = gamma ? T::load(gamma, c) : 1.f, b = beta ? T::load(beta, c) : 0.f;
    T::store(yr, c, (T::load(xr, c) - mu) * rs * g + b);
  }
}

template <typename T, typename S = typename T::storage>
__global__ __launch_bounds__(kThreads) void ln_bwd_input_rowblock(
    const S* __restrict__ dy, const S* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const S* __restrict__ gamma, S* __restrict__ dx, int cols) {
#pragma clang fp contract(off)
  __shared__ float red[kWavesPerBlock];
  const int64_t row = blockIdx.x;
  const float m = mean[row], rs = rstd[row];
  const S* dyr = dy + row * cols;
  const S* xr = x + row * cols;
  float s1 = 0.f, s2 = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float a = T::load(dyr, c) * (gamma ? T::load(gamma, c) : 1.f);
    s1 += a;
    s2 += a * ((T::load(xr, c) - m) * rs);
  }
  const float t1 = block_sum(s1, red);
  const float t2 = block_sum(s2, red);
  const float ic = 1.0f / static_cast<float>(cols);
  S* dxr = dx + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float n = (T::load(xr, c) - m) * rs;
    T::store(dxr, c, rs * (T::load(dyr, c) * (gamma ? T::load(gamma, c) : 1.f) - (t1 + n * t2) * ic));
  }
}

// Column-parallel gamma/beta gradient for the fallback path: one thread per column, rows
// summed in order (deterministic).
template <typename T, typename S = typename T::storage>
__global__ __launch_bounds__(kThreads) void ln_gb_columns(const S* __restrict__ dy,
                                                          const S* __restrict__ x,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd,
                                                          float* __restrict__ grad_gamma,
                                                          float* __restrict__ grad_beta,
                                                          int rows, int cols) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  float sg = 0.f, sb = 0.f;
  for (int r = 0; r < rows; ++r) {
    const int64_t o = static_cast<int64_t>(r) * cols + c;
    const float d = T::load(dy, o);
    sg += d * ((T::load(x, o) - mean[r]) * rstd[r]);
    sb += d;
  }
  if (grad_gamma) grad_gamma[c] += sg;
  if (grad_beta) grad_beta[c] += sb;
}

// ------------------------------------------------------------------------------------------
// Dispatch helpers
// ------------------------------------------------------------------------------------------
int pick_vpl(int cols4) {
  static const int kVpl[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int v : kVpl)
    if (cols4 <= v * HK_WAVE) return v;
  return 0;
}

template <typename F>
hipError_t with_vpl(int vpl, F&& f) {
  switch (vpl) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 12: return f(std::integral_constant<int, 12>{});
    case 16: return f(std::integral_constant<int, 16>{});
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
bool reg_path_ok(int cols, std::initializer_list<const void*> ptrs) {
  constexpr int P = T::kPerVec;
  if (cols % P != 0 || pick_vpl(cols / P) == 0) return false;
  for (const void* p : ptrs)
    if (p && !hk::aligned16(p)) return false;
  return true;
}

constexpr int kMaxGbCols = 2048;
template <typename T>
constexpr int kMaxBwdVpl = 4096 / (HK_WAVE * T::kPerVec);

// Lets a ONE_ROW gamma/beta backward form use its up to 128 KiB of dynamic LDS (set once per
// kernel, before its first launch).
template <typename T, int V, bool WRITE_DX>
hipError_t one_row_lds_limit() {
  static std::once_flag once;
  static hipError_t status = hipSuccess;
  std::call_once(once, [] {
    status = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&ln_bwd_reg<T, V, WRITE_DX, true, kOneRowWaves, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize,
        static_cast<int>(kOneRowWaves * 2 * kOneRowMaxCols<T> * sizeof(float)));
  });
  return status;
}

// Workgroups of a gamma/beta backward: one per `waves` rows, at most 8 / waves per CU.
int bwd_gb_grid(int rows, int waves) {
  const int64_t want = hk::ceil_div(rows, waves);
  const int64_t cap = static_cast<int64_t>(hk::device_cu_count()) * (8 / waves);
  return static_cast<int>(want < cap ? want : cap);
}

template <typename T>
hipError_t launch_fwd(const St<T>* x, const St<T>* gamma, const St<T>* beta, St<T>* y,
                      float* mean_out, float* rstd_out, int rows, int cols, float eps,
                      hipStream_t stream) {
  HK_CHECK_ARG(rows >= 0 && cols >= 0);
  if (rows == 0 || cols == 0) return hipSuccess;
  HK_CHECK_ARG(x && y);
  if (reg_path_ok<T>(cols, {x, gamma, beta, y})) {
    const int nvec = cols / T::kPerVec;
    const unsigned grid = static_cast<unsigned>(hk::ceil_div(rows, kWavesPerBlock));
    const float inv_cols = 1.0f / static_cast<float>(cols);
    return with_vpl(pick_vpl(nvec), [&](auto vpl_c) -> hipError_t {
      constexpr int V = decltype(vpl_c)::value;
      hipLaunchKernelGGL((ln_fwd_reg<T, V>), dim3(grid), dim3(kThreads), 0, stream,
                         reinterpret_cast<const uint4*>(x), reinterpret_cast<const uint4*>(gamma),
                         reinterpret_cast<const uint4*>(beta), reinterpret_cast<uint4*>(y),
                         mean_out, rstd_out, rows, nvec, inv_cols, eps);
      return hk::launch_status();
    });
  }
  hipLaunchKernelGGL(ln_fwd_rowblock<T>, dim3(rows), dim3(kThreads), 0, stream, x, gamma, beta, y,
                     mean_out, rstd_out, cols, eps);
  return hk::launch_status();
}

template <typename T>
hipError_t launch_bwd(const St<T>* dy, const St<T>* x, const float* mean, const float* rstd,
                      const St<T>* gamma, St<T>* dx, float* dgamma, float* dbeta, int rows,
                      int cols, bool write_dx, bool do_gb, hipStream_t stream) {
  HK_CHECK_ARG(rows >= 0 && cols >= 0);
  if (rows == 0 || cols == 0) return hipSuccess;
  HK_CHECK_ARG(dy && x && mean && rstd);
  HK_CHECK_ARG(!write_dx || dx);
  // The gamma/beta partials of one workgroup live in LDS: 8 (cols <= 1024) or 4 waves x 2 x
  // cols floats, kept within 64 KiB (cols <= kMaxGbCols); the one-row form's 16 waves take up
  // to 128 KiB (cols <= kOneRowMaxCols<T>). The backward keeps dy, x and their prefetch in
  // registers; past kMaxBwdVpl vectors per lane (4096 columns for every storage type) it would
  // spill, so wider rows take the workgroup-per-row kernels.
  if (reg_path_ok<T>(cols, {dy, x, gamma, dx}) && pick_vpl(cols / T::kPerVec) <= kMaxBwdVpl<T> &&
      (!do_gb || cols <= kMaxGbCols)) {
    const int nvec = cols / T::kPerVec;
    const bool one_row = do_gb && cols <= kOneRowMaxCols<T> &&
                         rows <= static_cast<int64_t>(hk::device_cu_count()) * kOneRowWaves;
    const int waves = one_row ? kOneRowWaves : do_gb ? gb_waves(cols) : kWavesPerBlock;
    const int grid = one_row ? static_cast<int>(hk::ceil_div(rows, kOneRowWaves))
                     : do_gb ? bwd_gb_grid(rows, waves)
                             : static_cast<int>(hk::ceil_div(rows, kWavesPerBlock));
    float* part = nullptr;
    if (do_gb) {
      void* ws = nullptr;
      HK_RETURN_IF_ERROR(
          hk::device_workspace(static_cast<size_t>(grid) * 2 * cols * sizeof(float), stream, &ws));
      part = static_cast<float*>(ws);
    }
    const size_t lds = do_gb ? static_cast<size_t>(waves) * 2 * cols * sizeof(float) : 0;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    HK_RETURN_IF_ERROR(with_vpl(pick_vpl(nvec), [&](auto vpl_c) -> hipError_t {
      constexpr int V = decltype(vpl_c)::value;
      // only the forms the conditions above can select are instantiated
      if constexpr (V > kMaxBwdVpl<T>) {
        return hipErrorInvalidValue;
      } else {
        constexpr int kCols = V * HK_WAVE * T::kPerVec;  // the widest row of this VPL
        constexpr bool kGb = kCols <= kMaxGbCols;
        using Kernel = void (*)(const uint4*, const uint4*, const float*, const float*,
                                const uint4*, uint4*, float*, int, int, float);
        Kernel k = ln_bwd_reg<T, V, true, false, kWavesPerBlock>;
        // pick_vpl takes the smallest VPL that holds the row, so cols <= 1024 exactly when
        // kCols <= 1024: the wave count of the gamma/beta forms is fixed by V
        constexpr int kW = gb_waves(kCols);
        if constexpr (kGb) {
          if (do_gb && one_row) {
            if constexpr (kCols <= kOneRowMaxCols<T>) {
              const hipError_t attr = write_dx ? one_row_lds_limit<T, V, true>()
                                               : one_row_lds_limit<T, V, false>();
              HK_RETURN_IF_ERROR(attr);
              k = write_dx ? ln_bwd_reg<T, V, true, true, kOneRowWaves, true>
                           : ln_bwd_reg<T, V, false, true, kOneRowWaves, true>;
            } else {
              return hipErrorInvalidValue;  // the smallest VPL holding cols has kCols <= the cap
            }
          } else if (do_gb) {
            if (waves != kW) return hipErrorInvalidValue;
            k = write_dx ? ln_bwd_reg<T, V, true, true, kW> : ln_bwd_reg<T, V, false, true, kW>;
          }
        }
        if (do_gb && !kGb) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k, dim3(grid), dim3(waves * HK_WAVE), lds, stream,
                           reinterpret_cast<const uint4*>(dy), reinterpret_cast<const uint4*>(x),
                           mean, rstd, reinterpret_cast<const uint4*>(gamma),
                           reinterpret_cast<uint4*>(dx), part, rows, nvec, inv_cols);
        return hk::launch_status();
      }
    }));
    if (do_gb) {
      hipLaunchKernelGGL(ln_gb_finalize,
                         dim3(static_cast<unsigned>(hk::ceil_div(2 * cols, kFinCols))),
                         dim3(kFinCols * kFinGroups), 0, stream, part, grid, cols, dgamma, dbeta);
      HK_RETURN_IF_ERROR(hk::launch_status());
    }
    return hipSuccess;
  }
  if (write_dx) {
    hipLaunchKernelGGL(ln_bwd_input_rowblock<T>, dim3(rows), dim3(kThreads), 0, stream, dy, x,
                       mean, rstd, gamma, dx, cols);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  if (do_gb) {
    hipLaunchKernelGGL(ln_gb_columns<T>, dim3(static_cast<unsigned>(hk::ceil_div(cols, kThreads))),
                       dim3(kThreads), 0, stream, dy, x, mean, rstd, dgamma, dbeta, rows, cols);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  return hipSuccess;
}

}  // namespace

// One set of four entry points per storage type: fp32 (the float kernels), and the
// reference's __half / __nv_bfloat16 instantiations (layer_norm_forward_sm89_kernel.cu:205-210;
// ln_backward_input_sm89_kernel.cu:107-113; ln_backward_gamma_beta_sm89_kernel.cu:51-56).
#define HK_LN_ENTRY_POINTS(SUFFIX, TAG, S)                                                       \
  extern "C" hipError_t hk_layer_norm_forward_##SUFFIX(const S* x, const S* gamma,              \
                                                       const S* beta, S* y, float* mean_out,    \
                                                       float* rstd_out, int rows, int cols,     \
                                                       float eps, hipStream_t stream) {         \
    return launch_fwd<TAG>(x, gamma, beta, y, mean_out, rstd_out, rows, cols, eps, stream);     \
  }                                                                                             \
  extern "C" hipError_t hk_ln_backward_input_##SUFFIX(const S* grad_y, const S* x,              \
                                                      const float* mean, const float* rstd,     \
                                                      const S* gamma, S* grad_x, int rows,      \
                                                      int cols, hipStream_t stream) {           \
    return launch_bwd<TAG>(grad_y, x, mean, rstd, gamma, grad_x, nullptr, nullptr, rows, cols,  \
                           true, false, stream);                                                \
  }                                                                                             \
  extern "C" hipError_t hk_ln_backward_gamma_beta_##SUFFIX(                                     \
      const S* grad_y, const S* x, const float* mean, const float* rstd, float* grad_gamma,     \
      float* grad_beta, int rows, int cols, hipStream_t stream) {                               \
    HK_CHECK_ARG(grad_gamma || grad_beta || rows == 0 || cols == 0);                            \
    return launch_bwd<TAG>(grad_y, x, mean, rstd, nullptr, nullptr, grad_gamma, grad_beta, rows, \
                           cols, false, true, stream);                                          \
  }                                                                                             \
  extern "C" hipError_t hk_layer_norm_backward_##SUFFIX(                                        \
      const S* grad_y, const S* x, const float* mean, const float* rstd, const S* gamma,        \
      S* grad_x, float* grad_gamma, float* grad_beta, int rows, int cols, hipStream_t stream) { \
    return launch_bwd<TAG>(grad_y, x, mean, rstd, gamma, grad_x, grad_gamma, grad_beta, rows,   \
                           cols, true, grad_gamma || grad_beta, stream);                        \
  }

HK_LN_ENTRY_POINTS(f32, hk::F32, float)
HK_LN_ENTRY_POINTS(bf16, hk::BF16, hk_bf16)
HK_LN_ENTRY_POINTS(f16, hk::F16, hk_f16)
