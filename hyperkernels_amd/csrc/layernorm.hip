// layernorm.hip - LayerNorm forward / backward over fp32 rows [rows, cols].
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
// Design (gfx950): one 64-lane wave owns one row; for cols % 4 == 0 and cols <= 4096 the row is
// held in VGPRs (VPL float4 per lane), so x is read from HBM exactly once and mean/variance
// are computed in two exact passes over registers (no Welford merge needed). The gamma/beta
// gradient is accumulated per lane in registers across the rows a wave visits, reduced across
// the workgroup's waves in LDS, written as one partial per workgroup, and summed over the
// workgroups in a fixed order by a second small kernel: the result is deterministic, unlike
// the reference's atomics. Shapes outside the register path use a workgroup-per-row fallback.
#include <initializer_list>
#include <type_traits>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / HK_WAVE;

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
__device__ __forceinline__ float f4_sum(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// ------------------------------------------------------------------------------------------
// Forward, register-resident rows.
// ------------------------------------------------------------------------------------------
template <int VPL>
__global__ __launch_bounds__(kThreads) void ln_fwd_reg(const float4* __restrict__ x,
                                                       const float4* __restrict__ gamma,
                                                       const float4* __restrict__ beta,
                                                       float4* __restrict__ y,
                                                       float* __restrict__ mean_out,
                                                       float* __restrict__ rstd_out, int rows,
                                                       int cols4, float inv_cols, float eps) {
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4* xr = x + static_cast<int64_t>(row) * cols4;
  float4 v[VPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    v[i] = (c < cols4) ? hk::ld_nt(xr + c) : f4_zero();
    s += f4_sum(v[i]);
  }
  const float mu = hk::wave_sum(s) * inv_cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    if (c < cols4) {
      const float a = v[i].x - mu, b = v[i].y - mu, cc = v[i].z - mu, d = v[i].w - mu;
      q += (a * a + b * b) + (cc * cc + d * d);
    }
  }
  const float var = hk::wave_sum(q) * inv_cols;
  const float rs = 1.0f / sqrtf(var + eps);
  if (lane == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = rs;
  }
  float4* yr = y + static_cast<int64_t>(row) * cols4;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    if (c < cols4) {
      const float4 g = gamma ? gamma[c] : make_float4(1.f, 1.f, 1.f, 1.f);
      const float4 b = beta ? beta[c] : f4_zero();
      float4 o;
      o.x = (v[i].x - mu) * rs * g.x + b.x;
      o.y = (v[i].y - mu) * rs * g.y + b.y;
      o.z = (v[i].z - mu) * rs * g.z + b.z;
      o.w = (v[i].w - mu) * rs * g.w + b.w;
      hk::st_nt(yr + c, o);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Backward, register-resident rows. WRITE_DX: produce grad_x. DO_GB: accumulate the
// per-workgroup gamma/beta partials into part[blockIdx.x][2 * cols] (gamma then beta).
// Each wave walks its rows with the next row's dy / x already in flight (software prefetch),
// so the two wave reductions of one row overlap the loads of the next.
// ------------------------------------------------------------------------------------------
template <int VPL, bool WRITE_DX, bool DO_GB>
__global__ __launch_bounds__(kThreads) void ln_bwd_reg(
    const float4* __restrict__ dy, const float4* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float4* __restrict__ gamma, float4* __restrict__ dx,
    float* __restrict__ part, int rows, int cols4, float inv_cols) {
  // Every product below is rounded on its own (as the reference formula is written), so a
  // row whose terms cancel exactly (cols == 1) gives exactly zero.
#pragma clang fp contract(off)
  extern __shared__ float4 lds4[];  // [kWavesPerBlock][2][cols4] when DO_GB
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int wave = threadIdx.x >> 6;
  float4 g[VPL];
  float4 acc_g[VPL], acc_b[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + i * HK_WAVE;
    g[i] = (gamma && c < cols4) ? gamma[c] : make_float4(1.f, 1.f, 1.f, 1.f);
    acc_g[i] = f4_zero();
    acc_b[i] = f4_zero();
  }
  const int stride = gridDim.x * kWavesPerBlock;
  int row = blockIdx.x * kWavesPerBlock + wave;
  float4 dn[VPL], xn[VPL];
  float mn = 0.f, rn = 0.f;
  auto fetch = [&](int r) {
    const float4* dyr = dy + static_cast<int64_t>(r) * cols4;
    const float4* xr = x + static_cast<int64_t>(r) * cols4;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + i * HK_WAVE;
      dn[i] = (c < cols4) ? hk::ld_nt(dyr + c) : f4_zero();
      xn[i] = (c < cols4) ? hk::ld_nt(xr + c) : f4_zero();
    }
    mn = mean[r];
    rn = rstd[r];
  };
  if (row < rows) fetch(row);
  for (; row < rows; row += stride) {
    float4 d[VPL], n[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      d[i] = dn[i];
      n[i] = xn[i];
    }
    const float m = mn, rs = rn;
    if (row + stride < rows) fetch(row + stride);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const bool in = lane + i * HK_WAVE < cols4;
      n[i].x = in ? (n[i].x - m) * rs : 0.f; n[i].y = in ? (n[i].y - m) * rs : 0.f;
      n[i].z = in ? (n[i].z - m) * rs : 0.f; n[i].w = in ? (n[i].w - m) * rs : 0.f;
      if (DO_GB) {
        acc_g[i].x += d[i].x * n[i].x; acc_g[i].y += d[i].y * n[i].y;
        acc_g[i].z += d[i].z * n[i].z; acc_g[i].w += d[i].w * n[i].w;
        acc_b[i].x += d[i].x; acc_b[i].y += d[i].y; acc_b[i].z += d[i].z; acc_b[i].w += d[i].w;
      }
      if (WRITE_DX) {
        const float a0 = d[i].x * g[i].x, a1 = d[i].y * g[i].y;
        const float a2 = d[i].z * g[i].z, a3 = d[i].w * g[i].w;
        s1 += (a0 + a1) + (a2 + a3);
        s2 += (a0 * n[i].x + a1 * n[i].y) + (a2 * n[i].z + a3 * n[i].w);
      }
    }
    if (WRITE_DX) {
      const float t1 = hk::wave_sum(s1), t2 = hk::wave_sum(s2);
      float4* dxr = dx + static_cast<int64_t>(row) * cols4;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = lane + i * HK_WAVE;
        if (c < cols4) {
          float4 o;
          o.x = rs * (d[i].x * g[i].x - (t1 + n[i].x * t2) * inv_cols);
          o.y = rs * (d[i].y * g[i].y - (t1 + n[i].y * t2) * inv_cols);
          o.z = rs * (d[i].z * g[i].z - (t1 + n[i].z * t2) * inv_cols);
          o.w = rs * (d[i].w * g[i].w - (t1 + n[i].w * t2) * inv_cols);
          hk::st_nt(dxr + c, o);
        }
      }
    }
  }
  if (DO_GB) {
    float4* my = lds4 + static_cast<int64_t>(wave) * 2 * cols4;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + i * HK_WAVE;
      if (c < cols4) {
        my[c] = acc_g[i];
        my[cols4 + c] = acc_b[i];
      }
    }
    __syncthreads();
    float4* out = reinterpret_cast<float4*>(part) + static_cast<int64_t>(blockIdx.x) * 2 * cols4;
    for (int c = threadIdx.x; c < 2 * cols4; c += kThreads) {
      float4 s = lds4[c];
#pragma unroll
      for (int w = 1; w < kWavesPerBlock; ++w) {
        const float4 t = lds4[static_cast<int64_t>(w) * 2 * cols4 + c];
        s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
      }
      out[c] = s;
    }
  }
}

// Sums nparts partials [nparts][2 * cols] in a fixed order and adds them into grad_gamma /
// grad_beta. A workgroup of 16 waves owns 64 columns: wave w sums partials w, w + 16, ...
// (eight loads in flight per lane), then the 16 wave sums are added in wave order in LDS.
constexpr int kFinWaves = 16;
__global__ __launch_bounds__(kFinWaves * HK_WAVE) void ln_gb_finalize(
    const float* __restrict__ part, int nparts, int cols, float* __restrict__ grad_gamma,
    float* __restrict__ grad_beta) {
  __shared__ float red[kFinWaves][HK_WAVE];
  const int lane = threadIdx.x & (HK_WAVE - 1);
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.x * HK_WAVE + lane;
  const int width = 2 * cols;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < width) {
    int p = wave;
    for (; p + 7 * kFinWaves < nparts; p += 8 * kFinWaves) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += part[static_cast<int64_t>(p + u * kFinWaves) * width + c];
    }
    for (; p < nparts; p += kFinWaves) acc[0] += part[static_cast<int64_t>(p) * width + c];
  }
  red[wave][lane] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (wave == 0 && c < width) {
    float s = red[0][lane];
#pragma unroll
    for (int w = 1; w < kFinWaves; ++w) s += red[w][lane];
    if (c < cols) {
      if (grad_gamma) grad_gamma[c] += s;
    } else {
      if (grad_beta) grad_beta[c - cols] += s;
    }
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

__global__ __launch_bounds__(kThreads) void ln_fwd_rowblock(const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            float* __restrict__ y,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ rstd_out,
                                                            int cols, float eps) {
  __shared__ float red[kWavesPerBlock];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) s += xr[c];
  const float mu = block_sum(s, red) / static_cast<float>(cols);
  float q = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float d = xr[c] - mu;
    q += d * d;
  }
  const float var = block_sum(q, red) / static_cast<float>(cols);
  const float rs = 1.0f / sqrtf(var + eps);
  if (threadIdx.x == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = rs;
  }
  float* yr = y + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float g = gamma ? gamma[c] : 1.f, b = beta ? beta[c] : 0.f;
    yr[c] = (xr[c] - mu) * rs * g + b;
  }
}

__global__ __launch_bounds__(kThreads) void ln_bwd_input_rowblock(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma, float* __restrict__ dx,
    int cols) {
#pragma clang fp contract(off)
  __shared__ float red[kWavesPerBlock];
  const int64_t row = blockIdx.x;
  const float m = mean[row], rs = rstd[row];
  const float* dyr = dy + row * cols;
  const float* xr = x + row * cols;
  float s1 = 0.f, s2 = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float a = dyr[c] * (gamma ? gamma[c] : 1.f);
    s1 += a;
    s2 += a * ((xr[c] - m) * rs);
  }
  const float t1 = block_sum(s1, red);
  const float t2 = block_sum(s2, red);
  const float ic = 1.0f / static_cast<float>(cols);
  float* dxr = dx + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float n = (xr[c] - m) * rs;
    dxr[c] = rs * (dyr[c] * (gamma ? gamma[c] : 1.f) - (t1 + n * t2) * ic);
  }
}

// Column-parallel gamma/beta gradient for the fallback path: one thread per column, rows
// summed in order (deterministic).
__global__ __launch_bounds__(kThreads) void ln_gb_columns(const float* __restrict__ dy,
                                                          const float* __restrict__ x,
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
    const float d = dy[o];
    sg += d * ((x[o] - mean[r]) * rstd[r]);
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

bool reg_path_ok(int cols, std::initializer_list<const void*> ptrs) {
  if (cols % 4 != 0 || pick_vpl(cols / 4) == 0) return false;
  for (const void* p : ptrs)
    if (p && !hk::aligned16(p)) return false;
  return true;
}

int bwd_grid(int rows) {
  const int64_t want = hk::ceil_div(rows, kWavesPerBlock);
  const int64_t cap = static_cast<int64_t>(hk::device_cu_count()) * 2;
  return static_cast<int>(want < cap ? want : cap);
}

hipError_t launch_bwd(const float* dy, const float* x, const float* mean, const float* rstd,
                      const float* gamma, float* dx, float* dgamma, float* dbeta, int rows,
                      int cols, bool write_dx, bool do_gb, hipStream_t stream) {
  HK_CHECK_ARG(rows >= 0 && cols >= 0);
  if (rows == 0 || cols == 0) return hipSuccess;
  HK_CHECK_ARG(dy && x && mean && rstd);
  HK_CHECK_ARG(!write_dx || dx);
  // The gamma/beta partials of one workgroup live in LDS: 4 waves x 2 x cols floats, kept
  // within 64 KiB.
  if (reg_path_ok(cols, {dy, x, gamma, dx}) && (!do_gb || cols <= 2048)) {
    const int cols4 = cols / 4;
    const int grid = write_dx && !do_gb ? static_cast<int>(hk::ceil_div(rows, kWavesPerBlock))
                                        : bwd_grid(rows);
    float* part = nullptr;
    if (do_gb) {
      void* ws = nullptr;
      HK_RETURN_IF_ERROR(
          hk::device_workspace(static_cast<size_t>(grid) * 2 * cols * sizeof(float), stream, &ws));
      part = static_cast<float*>(ws);
    }
    const size_t lds = do_gb ? static_cast<size_t>(kWavesPerBlock) * 2 * cols * sizeof(float) : 0;
    const float inv_cols = 1.0f / static_cast<float>(cols);
    HK_RETURN_IF_ERROR(with_vpl(pick_vpl(cols4), [&](auto vpl_c) -> hipError_t {
      constexpr int V = decltype(vpl_c)::value;
      auto* k = write_dx ? (do_gb ? ln_bwd_reg<V, true, true> : ln_bwd_reg<V, true, false>)
                         : ln_bwd_reg<V, false, true>;
      hipLaunchKernelGGL(k, dim3(grid), dim3(kThreads), lds, stream,
                         reinterpret_cast<const float4*>(dy), reinterpret_cast<const float4*>(x),
                         mean, rstd, reinterpret_cast<const float4*>(gamma),
                         reinterpret_cast<float4*>(dx), part, rows, cols4, inv_cols);
      return hk::launch_status();
    }));
    if (do_gb) {
      hipLaunchKernelGGL(ln_gb_finalize, dim3(static_cast<unsigned>(hk::ceil_div(2 * cols, HK_WAVE))),
                         dim3(kFinWaves * HK_WAVE), 0, stream, part, grid, cols, dgamma, dbeta);
      HK_RETURN_IF_ERROR(hk::launch_status());
    }
    return hipSuccess;
  }
  if (write_dx) {
    hipLaunchKernelGGL(ln_bwd_input_rowblock, dim3(rows), dim3(kThreads), 0, stream, dy, x, mean,
                       rstd, gamma, dx, cols);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  if (do_gb) {
    hipLaunchKernelGGL(ln_gb_columns, dim3(static_cast<unsigned>(hk::ceil_div(cols, kThreads))),
                       dim3(kThreads), 0, stream, dy, x, mean, rstd, dgamma, dbeta, rows, cols);
    HK_RETURN_IF_ERROR(hk::launch_status());
  }
  return hipSuccess;
}

}  // namespace

extern "C" hipError_t hk_layer_norm_forward_f32(const float* x, const float* gamma,
                                                const float* beta, float* y, float* mean_out,
                                                float* rstd_out, int rows, int cols, float eps,
                                                hipStream_t stream) {
  HK_CHECK_ARG(rows >= 0 && cols >= 0);
  if (rows == 0 || cols == 0) return hipSuccess;
  HK_CHECK_ARG(x && y);
  if (reg_path_ok(cols, {x, gamma, beta, y})) {
    const int cols4 = cols / 4;
    const unsigned grid = static_cast<unsigned>(hk::ceil_div(rows, kWavesPerBlock));
    const float inv_cols = 1.0f / static_cast<float>(cols);
    return with_vpl(pick_vpl(cols4), [&](auto vpl_c) -> hipError_t {
      constexpr int V = decltype(vpl_c)::value;
      hipLaunchKernelGGL(ln_fwd_reg<V>, dim3(grid), dim3(kThreads), 0, stream,
                         reinterpret_cast<const float4*>(x),
                         reinterpret_cast<const float4*>(gamma),
                         reinterpret_cast<const float4*>(beta), reinterpret_cast<float4*>(y),
                         mean_out, rstd_out, rows, cols4, inv_cols, eps);
      return hk::launch_status();
    });
  }
  hipLaunchKernelGGL(ln_fwd_rowblock, dim3(rows), dim3(kThreads), 0, stream, x, gamma, beta, y,
                     mean_out, rstd_out, cols, eps);
  return hk::launch_status();
}

extern "C" hipError_t hk_ln_backward_input_f32(const float* grad_y, const float* x,
                                               const float* mean, const float* rstd,
                                               const float* gamma, float* grad_x, int rows,
                                               int cols, hipStream_t stream) {
  return launch_bwd(grad_y, x, mean, rstd, gamma, grad_x, nullptr, nullptr, rows, cols, true,
                    false, stream);
}

extern "C" hipError_t hk_ln_backward_gamma_beta_f32(const float* grad_y, const float* x,
                                                    const float* mean, const float* rstd,
                                                    float* grad_gamma, float* grad_beta,
                                                    int rows, int cols, hipStream_t stream) {
  HK_CHECK_ARG(grad_gamma || grad_beta || rows == 0 || cols == 0);
  return launch_bwd(grad_y, x, mean, rstd, nullptr, nullptr, grad_gamma, grad_beta, rows, cols,
                    false, true, stream);
}

extern "C" hipError_t hk_layer_norm_backward_f32(const float* grad_y, const float* x,
                                                 const float* mean, const float* rstd,
                                                 const float* gamma, float* grad_x,
                                                 float* grad_gamma, float* grad_beta, int rows,
                                                 int cols, hipStream_t stream) {
  return launch_bwd(grad_y, x, mean, rstd, gamma, grad_x, grad_gamma, grad_beta, rows, cols,
                    true, grad_gamma || grad_beta, stream);
}
