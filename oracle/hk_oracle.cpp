// hk_oracle.cpp - CPU restatement of BlubridgeAI/HyperKernels' reference math.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels of this repository:
// only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
// product library (hyperkernels_amd/libhk_amd.so) never calls it and has no CPU fallback.
//
// Every function restates a CPU reference of the reference repository's own harnesses (the
// file:line cited at each one), written from the formulas: same precision choices (double
// accumulation where the harness uses double, fp32 where it uses fp32), same operation order
// where the order fixes the rounding (AdamW). The GEMM references restate the device "naive
// reference" kernels of the BLAS harnesses on the CPU. The random generators reproduce the
// harnesses' input streams (std::mt19937_64 + uniform_real_distribution<float> in
// kernels_test.cu, splitmix64 in sgemm_test.cu / bgemm_test.cu).
//
// Build: see oracle/Makefile (g++ -O2 -ffp-contract=off -fopenmp). Contraction is off so the
// compiler never fuses a multiply-add the reference wrote as two roundings.
#include <omp.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#define ORACLE_API extern "C" __attribute__((visibility("default")))

namespace {

inline float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline uint64_t splitmix64(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}

// tanh-GELU exactly as the harness lambda (kernels_test.cu:251-254).
inline float tanh_gelu(float x) {
  const float c = 0.7978845608028654f, k = 0.044715f;
  return 0.5f * x * (1.0f + std::tanh(c * (x + k * x * x * x)));
}

// Analytic GELU derivative in fp32 (gelu_backward_sm89_kernel.cu:24-30), with std::tanh.
inline float tanh_gelu_grad(float x) {
  const float c = 0.7978845608028654f, k = 0.044715f;
  const float x2 = x * x;
  const float u = c * (x + k * x2 * x);
  const float du = c * (1.0f + 3.0f * k * x2);
  const float th = std::tanh(u);
  return 0.5f * (1.0f + th) + 0.5f * x * (1.0f - th * th) * du;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Library control and conversions
// ---------------------------------------------------------------------------------------------
ORACLE_API void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
ORACLE_API int oracle_max_threads(void) { return omp_get_max_threads(); }
ORACLE_API int oracle_hardware_concurrency(void) {
  return static_cast<int>(std::thread::hardware_concurrency());
}

ORACLE_API void oracle_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}
ORACLE_API void oracle_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]);
}

// ---------------------------------------------------------------------------------------------
// Input generators
// ---------------------------------------------------------------------------------------------
// kernels_test.cu:48-54 (rand_vec): std::mt19937_64(seed), uniform_real_distribution<float>.
ORACLE_API void oracle_rand_uniform(float* out, int64_t n, uint64_t seed, float lo, float hi) {
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<float> d(lo, hi);
  for (int64_t i = 0; i < n; ++i) out[i] = d(rng);
}

// sgemm_test.cu:151-162 / bgemm_test.cu:161-172 (fill_random_kernel), element i from seed + i.
ORACLE_API void oracle_splitmix_uniform(float* out, int64_t n, uint64_t seed, float lo,
                                        float hi) {
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t x = splitmix64(seed + static_cast<uint64_t>(i));
    const float u = static_cast<float>(x >> 40) * (1.0f / 16777216.0f);
    out[i] = u * (hi - lo) + lo;
  }
}

// Normal variates for the BASELINE configurations: splitmix64 stream -> two uniforms ->
// Box-Muller (no counterpart in the reference, which only draws uniforms).
ORACLE_API void oracle_normal(float* out, int64_t n, uint64_t seed, float mean, float stddev) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t a = splitmix64(seed * 0x9e3779b97f4a7c15ULL + 2 * static_cast<uint64_t>(i));
    const uint64_t b = splitmix64(seed * 0x9e3779b97f4a7c15ULL + 2 * static_cast<uint64_t>(i) + 1);
    const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740993.0);
    const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    out[i] = static_cast<float>(mean + stddev * z);
  }
}

// ---------------------------------------------------------------------------------------------
// GELU (kernels_test.cu:251-279; gelu_backward_sm89_kernel.cu:24-30)
// ---------------------------------------------------------------------------------------------
ORACLE_API void oracle_gelu_forward_f32(const float* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = tanh_gelu(x[i]);
}

ORACLE_API void oracle_gelu_backward_f32(const float* g, const float* x, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = g[i] * tanh_gelu_grad(x[i]);
}

// The harness's own check of the backward: a central difference of the forward with h = 1e-3
// (kernels_test.cu:271-272).
ORACLE_API void oracle_gelu_backward_fd_f32(const float* g, const float* x, float* out,
                                            int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float h = 1e-3f;
    out[i] = g[i] * ((tanh_gelu(x[i] + h) - tanh_gelu(x[i] - h)) / (2 * h));
  }
}

// bf16 I/O: inputs decoded from bf16, math in fp32, result left unrounded (fp32); the caller
// rounds to bf16 to form the comparison target.
ORACLE_API void oracle_gelu_forward_bf16(const uint16_t* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = tanh_gelu(bf16_to_f32(x[i]));
}
ORACLE_API void oracle_gelu_backward_bf16(const uint16_t* g, const uint16_t* x, float* out,
                                          int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(g[i]) * tanh_gelu_grad(bf16_to_f32(x[i]));
}

// ---------------------------------------------------------------------------------------------
// LayerNorm (kernels_test.cu:283-363)
// ---------------------------------------------------------------------------------------------
// Forward, double accumulation (kernels_test.cu:288-293). mean/rstd as floats (:314).
ORACLE_API void oracle_layer_norm_forward(const float* x, const float* gamma, const float* beta,
                                          float* y, float* mean, float* rstd, int64_t rows,
                                          int64_t cols, float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double m = 0;
    for (int64_t c = 0; c < cols; ++c) m += xr[c];
    m /= cols;
    double var = 0;
    for (int64_t c = 0; c < cols; ++c) {
      const double d = xr[c] - m;
      var += d * d;
    }
    var /= cols;
    const double rs = 1.0 / std::sqrt(var + eps);
    for (int64_t c = 0; c < cols; ++c) {
      const double g = gamma ? gamma[c] : 1.0, b = beta ? beta[c] : 0.0;
      y[r * cols + c] = static_cast<float>(((xr[c] - m) * rs) * g + b);
    }
    if (mean) mean[r] = static_cast<float>(m);
    if (rstd) rstd[r] = static_cast<float>(rs);
  }
}

// Backward w.r.t. the input (kernels_test.cu:317-323), from float mean/rstd. As in the harness,
// xhat and dy * gamma are float products; the sums and the final expression are double.
ORACLE_API void oracle_ln_backward_input(const float* dy, const float* x, const float* mean,
                                         const float* rstd, const float* gamma, float* dx,
                                         int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    double s1 = 0, s2 = 0;
    for (int64_t c = 0; c < cols; ++c) {
      const double nx = (x[r * cols + c] - mean[r]) * rstd[r];
      const double a = dy[r * cols + c] * (gamma ? gamma[c] : 1.0f);
      s1 += a;
      s2 += a * nx;
    }
    const double ic = 1.0 / cols;
    for (int64_t c = 0; c < cols; ++c) {
      const double nx = (x[r * cols + c] - mean[r]) * rstd[r];
      dx[r * cols + c] = static_cast<float>(
          rstd[r] * (dy[r * cols + c] * (gamma ? gamma[c] : 1.0f) - (s1 + nx * s2) * ic));
    }
  }
}

// grad_gamma = sum_r dy * xhat, grad_beta = sum_r dy (kernels_test.cu:346-349); written, not
// accumulated.
ORACLE_API void oracle_ln_backward_gamma_beta(const float* dy, const float* x, const float* mean,
                                              const float* rstd, float* dgamma, float* dbeta,
                                              int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < cols; ++c) {
    double dg = 0, db = 0;
    for (int64_t r = 0; r < rows; ++r) {
      const double nx = (x[r * cols + c] - mean[r]) * rstd[r];
      dg += dy[r * cols + c] * nx;
      db += dy[r * cols + c];
    }
    dgamma[c] = static_cast<float>(dg);
    dbeta[c] = static_cast<float>(db);
  }
}

// ---------------------------------------------------------------------------------------------
// Sparse cross-entropy (kernels_test.cu:374-396)
// ---------------------------------------------------------------------------------------------
ORACLE_API void oracle_sparse_ce_forward(const float* logits, const int32_t* targets,
                                         float* loss, float* out_max, float* out_sum,
                                         int64_t rows, int64_t vocab) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* l = logits + r * vocab;
    float mx = -1e38f;
    for (int64_t c = 0; c < vocab; ++c) mx = std::max(mx, l[c]);
    double sum = 0;
    for (int64_t c = 0; c < vocab; ++c) sum += std::exp(l[c] - mx);
    out_max[r] = mx;
    out_sum[r] = static_cast<float>(sum);
    const int64_t t = targets[r];
    const float xt = (t >= 0 && t < vocab) ? l[t] : NAN;
    loss[r] = static_cast<float>(std::log(sum) - (xt - mx));
  }
}

// grad = (softmax - onehot) * scale, scale = grad_output * host_scale (kernels_test.cu:393-396;
// sparseCENormalize_from_stats.cu:30 for the scale).
ORACLE_API void oracle_sparse_ce_backward(const float* logits, const int32_t* targets,
                                          const float* in_max, const float* in_sum, float* grad,
                                          int64_t rows, int64_t vocab, float scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const double inv = 1.0 / in_sum[r];
    const int64_t t = targets[r];
    for (int64_t c = 0; c < vocab; ++c) {
      const float sm = static_cast<float>(std::exp(logits[r * vocab + c] - in_max[r]) * inv);
      grad[r * vocab + c] = (sm - (c == t ? 1.0f : 0.0f)) * scale;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// AdamW (kernels_test.cu:436-437; multi_tensor_adam_sm89_kernel.cu:56-63): exact op order.
// ---------------------------------------------------------------------------------------------
ORACLE_API void oracle_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr,
                             float b1, float b2, float eps, float wd, float bc1, float bc2) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float mn = std::fma(b1, m[i], (1 - b1) * g[i]);
    const float vn = std::fma(b2, v[i], (1 - b2) * g[i] * g[i]);
    const float denom = std::sqrt(vn / bc2) + eps;
    p[i] = p[i] - lr * ((mn / bc1) / denom + wd * p[i]);
    m[i] = mn;
    v[i] = vn;
  }
}

// ---------------------------------------------------------------------------------------------
// Unified reduce (unified_reduce_standalone.cu:816-835): sums in double (the harness sums in
// float; double is the tighter reference for random inputs and identical for its exact inputs).
// ---------------------------------------------------------------------------------------------
ORACLE_API void oracle_reduce_inner(const float* src, float* dst, int64_t nout, int64_t len,
                                    int64_t row_stride) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < nout; ++o) {
    double s = 0;
    for (int64_t k = 0; k < len; ++k) s += src[o * row_stride + k];
    dst[o] = static_cast<float>(s);
  }
}

ORACLE_API void oracle_reduce_outer(const float* src, float* dst, int64_t nout, int64_t inner,
                                    int64_t outer_stride, int64_t row_stride, int64_t len) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < nout; ++o) {
    const float* base = src + (o / inner) * outer_stride + (o % inner);
    double s = 0;
    for (int64_t k = 0; k < len; ++k) s += base[k * row_stride];
    dst[o] = static_cast<float>(s);
  }
}

// The reference input (unified_reduce_standalone.cu:821): ((i % 17) - 8) * 0.25, exact in fp32.
ORACLE_API void oracle_reduce_selftest_input(float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = static_cast<float>((i % 17) - 8) * 0.25f;
}

// ---------------------------------------------------------------------------------------------
// Attention (kernels_test.cu:68-139, 459-481). [B,H,T,Hd] contiguous; LSE/D [B,H,T].
// ---------------------------------------------------------------------------------------------
// With `mask` (a [B*H, T, T] fp32 dropout mask, or NULL) each exp term is multiplied by
// mask[(bh*T + i)*T + j] and the row sum is taken after that product, so O is normalised by the
// post-dropout sum and LSE = m + log(l) is -inf for a row with nothing kept: the reference
// kernel's dropout path (fused_attn_forward_kernel_tc_sm89.cu:316-334, 421-425).
ORACLE_API void oracle_attn_forward(const float* Q, const float* K, const float* V, int B, int H,
                                    int T, int Hd, float scale, int causal, const float* mask,
                                    float* O, float* LSE) {
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int bh = 0; bh < B * H; ++bh) {
    for (int i = 0; i < T; ++i) {
      const int64_t base = static_cast<int64_t>(bh) * T * Hd;
      const int64_t lbase = static_cast<int64_t>(bh) * T;
      const float* qi = Q + base + static_cast<int64_t>(i) * Hd;
      const int jmax = causal ? i : (T - 1);
      float m = -1e30f;
      for (int j = 0; j <= jmax; ++j) {
        const float* kj = K + base + static_cast<int64_t>(j) * Hd;
        double d = 0;
        for (int k = 0; k < Hd; ++k) d += static_cast<double>(qi[k]) * kj[k];
        const float s = static_cast<float>(d * scale);
        if (s > m) m = s;
      }
      double l = 0;
      std::vector<double> oacc(Hd, 0.0);
      for (int j = 0; j <= jmax; ++j) {
        const float* kj = K + base + static_cast<int64_t>(j) * Hd;
        const float* vj = V + base + static_cast<int64_t>(j) * Hd;
        double d = 0;
        for (int k = 0; k < Hd; ++k) d += static_cast<double>(qi[k]) * kj[k];
        float e = std::exp(static_cast<float>(d * scale) - m);
        if (mask) e *= mask[(static_cast<int64_t>(bh) * T + i) * T + j];
        l += e;
        for (int k = 0; k < Hd; ++k) oacc[k] += static_cast<double>(e) * vj[k];
      }
      const double inv = (l > 0) ? 1.0 / l : 0.0;
      for (int k = 0; k < Hd; ++k) O[base + static_cast<int64_t>(i) * Hd + k] = static_cast<float>(oacc[k] * inv);
      LSE[lbase + i] = (l > 0) ? static_cast<float>(m + std::log(l)) : -INFINITY;
    }
  }
}

// D = rowsum(dO * O) (kernels_test.cu:465).
ORACLE_API void oracle_attn_precompute_D(const float* dO, const float* O, float* D, int64_t rows,
                                         int Hd) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    double s = 0;
    for (int k = 0; k < Hd; ++k) s += dO[r * Hd + k] * O[r * Hd + k];
    D[r] = static_cast<float>(s);
  }
}

// Backward (kernels_test.cu:101-139): fills D, dQ, dK, dV (zeroed first). Parallel over (b, h);
// within one head the loop order is the harness's.
ORACLE_API void oracle_attn_backward(const float* Q, const float* K, const float* V,
                                     const float* O, const float* dO, const float* LSE, int B,
                                     int H, int T, int Hd, float scale, int causal, float* D,
                                     float* dQ, float* dK, float* dV) {
#pragma omp parallel for schedule(dynamic)
  for (int bh = 0; bh < B * H; ++bh) {
    const int64_t base = static_cast<int64_t>(bh) * T * Hd;
    const int64_t lbase = static_cast<int64_t>(bh) * T;
    std::fill(dQ + base, dQ + base + static_cast<int64_t>(T) * Hd, 0.f);
    std::fill(dK + base, dK + base + static_cast<int64_t>(T) * Hd, 0.f);
    std::fill(dV + base, dV + base + static_cast<int64_t>(T) * Hd, 0.f);
    for (int i = 0; i < T; ++i) {
      const float* qi = Q + base + static_cast<int64_t>(i) * Hd;
      const float* doi = dO + base + static_cast<int64_t>(i) * Hd;
      const float* oi = O + base + static_cast<int64_t>(i) * Hd;
      double Di = 0;
      for (int k = 0; k < Hd; ++k) Di += static_cast<double>(doi[k]) * oi[k];
      D[lbase + i] = static_cast<float>(Di);
      const float Li = LSE[lbase + i];
      const int jmax = causal ? i : (T - 1);
      float* dqi = dQ + base + static_cast<int64_t>(i) * Hd;
      for (int j = 0; j <= jmax; ++j) {
        const float* kj = K + base + static_cast<int64_t>(j) * Hd;
        const float* vj = V + base + static_cast<int64_t>(j) * Hd;
        float* dkj = dK + base + static_cast<int64_t>(j) * Hd;
        float* dvj = dV + base + static_cast<int64_t>(j) * Hd;
        double sd = 0, dp = 0;
        for (int k = 0; k < Hd; ++k) {
          sd += static_cast<double>(qi[k]) * kj[k];
          dp += static_cast<double>(doi[k]) * vj[k];
        }
        const float p = std::exp(static_cast<float>(sd * scale) - Li);
        const float ds = static_cast<float>(p * (dp - Di) * scale);
        for (int k = 0; k < Hd; ++k) {
          dqi[k] += ds * kj[k];
          dkj[k] += ds * qi[k];
          dvj[k] += p * doi[k];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// GEMM references. Row-major. transA: A stored [K, M]; transB: B stored [N, K]. fp32
// accumulation in k order, as the BLAS harnesses' device reference kernels
// (sgemm_test.cu:176-185, bgemm_test.cu:186-197).
// ---------------------------------------------------------------------------------------------
// C[M,N] = alpha * op(A) op(B) + beta * C0 + bias[col] (bias added once; NULL bias and NULL C0
// allowed).
ORACLE_API void oracle_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                             const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                             const float* C0, int64_t ldc0, const float* bias, float* C,
                             int64_t ldc) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < M; ++r) {
    for (int64_t c = 0; c < N; ++c) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float a = transA ? A[k * lda + r] : A[r * lda + k];
        const float b = transB ? B[c * ldb + k] : B[k * ldb + c];
        acc += a * b;
      }
      float out = alpha * acc + (C0 ? beta * C0[r * ldc0 + c] : 0.0f);
      if (bias) out += bias[c];
      C[r * ldc + c] = out;
    }
  }
}

// bf16 inputs decoded to fp32; out = alpha * acc + beta * C0 (+ beta * bias), fp32 result.
ORACLE_API void oracle_bgemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                             const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb,
                             float beta, const uint16_t* C0, int64_t ldc0, const uint16_t* bias,
                             int64_t bias_numel, float* C, int64_t ldc) {
  // bias (bgemm_addmm_sm89_kernel.cu:214-300; bgemm_core_template.cu:270-289): element
  // (r, c) uses bias[c] when bias_numel == N, else bias[r] when == M, else bias[0] when == 1,
  // else bias[r * N + c] (M * N); the result adds beta * bias.
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < M; ++r) {
    for (int64_t c = 0; c < N; ++c) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float a = bf16_to_f32(transA ? A[k * lda + r] : A[r * lda + k]);
        const float b = bf16_to_f32(transB ? B[c * ldb + k] : B[k * ldb + c]);
        acc += a * b;
      }
      float out = alpha * acc + (C0 ? beta * bf16_to_f32(C0[r * ldc0 + c]) : 0.0f);
      if (bias) {
        const int64_t i =
            bias_numel == N ? c : bias_numel == M ? r : bias_numel == 1 ? 0 : r * N + c;
        out += beta * bf16_to_f32(bias[i]);
      }
      C[r * ldc + c] = out;
    }
  }
}
