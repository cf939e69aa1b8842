// cross_entropy.hip - sparse softmax cross-entropy over fp32 logits [rows, vocab].
//
// Reference behaviour:
//   forward   kernels/loss/sparse_ce_forward_kernel_vec_save_stats.cu:14-106
//             per row: max, sum = sum_j exp(x_j - max) (streaming online softmax),
//             loss = log(sum) + max - x[target]; saves max and sum for the backward.
//   backward  kernels/loss/sparseCENormalize_from_stats.cu:7-49
//             grad_j = (exp(x_j - max) / sum - [j == target]) * (*grad_output * host_scale)
//   target index types int32, int64 and uint16, as the reference instantiates both kernels
//             (sparse_ce_forward_kernel_vec_save_stats.cu:108-113;
//             sparseCENormalize_from_stats.cu:52-60). The index is widened to int64 before use.
//
// Design (gfx950): one 1024-lane workgroup streams one row in the forward. A row of fp32 logits starts at
// row * vocab * 4 bytes, which is only 4-byte aligned when vocab is odd (the GPT-2 vocabulary
// 50257 is), so each row is split into a scalar head up to the next 16-byte boundary, a body
// of 16-byte loads (each lane keeps 2 of them in flight), and a scalar tail. This is what lets
// any vocab size work; the reference assumes vocab % 4 == 0. Each lane keeps an online
// (max, sum) state, updated once per 4 values; lanes merge with 64-wide butterflies and the
// four waves merge through LDS.
#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void absorb1(float& m, float& s, float v) {
  if (v > m) {
    s = s * __expf(m - v) + 1.0f;
    m = v;
  } else {
    s += __expf(v - m);
  }
}

__device__ __forceinline__ void absorb4(float& m, float& s, float4 v) {
  const float mx = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
  if (mx > m) {
    s *= __expf(m - mx);
    m = mx;
  }
  s += (__expf(v.x - m) + __expf(v.y - m)) + (__expf(v.z - m) + __expf(v.w - m));
}

// Splits [0, n) of a row that starts at p into head [0, h), body [h, h + 4 nb), tail.
__device__ __forceinline__ void split_row(const void* p, int64_t n, int64_t& h, int64_t& nb) {
  const int64_t mis = (reinterpret_cast<uintptr_t>(p) >> 2) & 3;
  h = (4 - mis) & 3;
  if (h > n) h = n;
  nb = (n - h) >> 2;
}

// Forward workgroup: 1024 lanes per row with two 16-byte loads each in flight. A row is
// ~200 KB, so a workgroup's life is a dozen dependent load rounds; wide workgroups shorten
// that chain (measured on MI355X: 6.85 TB/s at 1024 lanes against 6.3 TB/s at 256).
constexpr int kFwdThreads = 1024;
constexpr int kFwdWaves = kFwdThreads / HK_WAVE;
constexpr int kFwdUnroll = 2;

template <typename TIdx>
__global__ __launch_bounds__(kFwdThreads) void ce_forward(const float* __restrict__ logits,
                                                          const TIdx* __restrict__ targets,
                                                          float* __restrict__ losses,
                                                          float* __restrict__ saved_max,
                                                          float* __restrict__ saved_sum,
                                                          int64_t vocab) {
  __shared__ float red_m[kFwdWaves], red_s[kFwdWaves];
  const int64_t row = blockIdx.x;
  const float* x = logits + row * vocab;
  const int tid = threadIdx.x;
  float m = -INFINITY, s = 0.f;

  int64_t h, nb;
  split_row(x, vocab, h, nb);
  if (tid < h) absorb1(m, s, x[tid]);
  const float4* body = reinterpret_cast<const float4*>(x + h);
  int64_t i = tid;
  for (; i + (kFwdUnroll - 1) * kFwdThreads < nb; i += kFwdUnroll * kFwdThreads) {
    float4 v[kFwdUnroll];
#pragma unroll
    for (int u = 0; u < kFwdUnroll; ++u) v[u] = hk::ld_nt(body + i + u * kFwdThreads);
#pragma unroll
    for (int u = 0; u < kFwdUnroll; ++u) absorb4(m, s, v[u]);
  }
  {  // remainder of the body: the same loads in flight, predicated
    float4 v[kFwdUnroll];
    bool ok[kFwdUnroll];
#pragma unroll
    for (int u = 0; u < kFwdUnroll; ++u) {
      ok[u] = i + u * kFwdThreads < nb;
      if (ok[u]) v[u] = hk::ld_nt(body + i + u * kFwdThreads);
    }
#pragma unroll
    for (int u = 0; u < kFwdUnroll; ++u)
      if (ok[u]) absorb4(m, s, v[u]);
  }
  for (int64_t j = h + 4 * nb + tid; j < vocab; j += kFwdThreads) absorb1(m, s, x[j]);

  hk::wave_softmax_merge(m, s);
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float fm = red_m[0], fs = red_s[0];
#pragma unroll
    for (int w = 1; w < kFwdWaves; ++w) hk::softmax_merge(fm, fs, red_m[w], red_s[w]);
    saved_max[row] = fm;
    saved_sum[row] = fs;
    const int64_t t = static_cast<int64_t>(targets[row]);
    const float xt = (t >= 0 && t < vocab) ? x[t] : __builtin_nanf("");
    losses[row] = logf(fs) + fm - xt;
  }
}

__device__ __forceinline__ float ce_grad1(float v, float mx, float inv_sum, float scale,
                                          bool hit) {
  return (__expf(v - mx) * inv_sum - (hit ? 1.0f : 0.0f)) * scale;
}

// Row-chunk path (vocab < 4 * kFlatThreads; larger vocabularies take ce_backward_flat below):
// logits and grad share the same 16-byte phase on every row. The row's body is cut
// into chunks of kBwdThreads 16-byte vectors, one workgroup each (grid = rows x chunks), one
// vector per lane: many short-lived workgroups keep more bytes in flight across the device
// than a few long ones (measured on MI355X at 8192 x 50257: ~6.2 TB/s with 512-vector
// chunks against ~5.7 TB/s with 1024-vector chunks of four vectors per lane). Chunk 0 also
// writes the row's head, the last chunk its tail.
constexpr int kBwdThreads = 512;
constexpr int kChunkVec = kBwdThreads;

template <typename TIdx>
__global__ __launch_bounds__(kBwdThreads) void ce_backward(
    const float* __restrict__ logits, const TIdx* __restrict__ targets,
    float* __restrict__ grad, const float* __restrict__ saved_max,
    const float* __restrict__ saved_sum, int64_t vocab, int nchunks,
    const float* __restrict__ grad_output, float host_scale) {
  const int64_t row = blockIdx.x / nchunks;
  const int chunk = blockIdx.x - static_cast<int>(row) * nchunks;
  const float* x = logits + row * vocab;
  float* g = grad + row * vocab;
  const int tid = threadIdx.x;
  int64_t h, nb;
  split_row(x, vocab, h, nb);
  const float4* xb = reinterpret_cast<const float4*>(x + h);
  float4* gb = reinterpret_cast<float4*>(g + h);
  const int64_t i = static_cast<int64_t>(chunk) * kChunkVec + tid;
  float4 v;
  if (i < nb) v = hk::ld_nt(xb + i);  // issued before the row statistics are needed
  const float mx = saved_max[row];
  const float inv_sum = 1.0f / saved_sum[row];
  const float scale = (grad_output ? grad_output[0] : 1.0f) * host_scale;
  const int64_t t = static_cast<int64_t>(targets[row]);
  if (chunk == 0 && tid < h) g[tid] = ce_grad1(x[tid], mx, inv_sum, scale, tid == t);
  if (chunk == nchunks - 1) {
    const int64_t j = h + 4 * nb + tid;
    if (j < vocab) g[j] = ce_grad1(x[j], mx, inv_sum, scale, j == t);
  }
  if (i < nb) {
    const int64_t j = h + 4 * i;
    float4 o;
    o.x = ce_grad1(v.x, mx, inv_sum, scale, j + 0 == t);
    o.y = ce_grad1(v.y, mx, inv_sum, scale, j + 1 == t);
    o.z = ce_grad1(v.z, mx, inv_sum, scale, j + 2 == t);
    o.w = ce_grad1(v.w, mx, inv_sum, scale, j + 3 == t);
    hk::st_nt(gb + i, o);
  }
}

// Flat path (vocab >= 4 * kFlatThreads): the [rows, vocab] logits as one stream of 16-byte
// vectors from the first 16-byte boundary of the buffer, kFlatThreads vectors per workgroup,
// one per lane. A workgroup's 4 * kFlatThreads elements then span at most two rows, whose
// statistics it reads once; every element picks its row's by comparing its flat index with the
// row boundary. With no row-aligned chunks there are no part-empty tail chunks and no per-row
// head/tail work: 522 us against 541 us for the row chunks above at 8192 x 50257 on MI355X
// (a plain 1-read/1-write copy of the same bytes: 500-511 us). Results are the same bits: the
// per-element formula is ce_grad1 in both. The buffer's own head (before the first 16-byte
// boundary, in row 0) and tail (after the last whole vector, in the last row) go to the first
// and last workgroups' lanes.
constexpr int kFlatThreads = 512;

template <typename TIdx>
__global__ __launch_bounds__(kFlatThreads) void ce_backward_flat(
    const float* __restrict__ logits, const TIdx* __restrict__ targets,
    float* __restrict__ grad, const float* __restrict__ saved_max,
    const float* __restrict__ saved_sum, int64_t rows, int64_t vocab, int64_t head,
    int64_t nvec, const float* __restrict__ grad_output, float host_scale) {
  const int tid = threadIdx.x;
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kFlatThreads + tid;
  const float4* xb = reinterpret_cast<const float4*>(logits + head);
  float4 x;
  if (v < nvec) x = hk::ld_nt(xb + v);  // issued before the row statistics are needed
  const int64_t e0 = head + static_cast<int64_t>(blockIdx.x) * kFlatThreads * 4;
  const int64_t r0 = e0 / vocab;
  const int64_t r1 = min(r0 + 1, rows - 1);
  const int64_t start1 = (r0 + 1) * vocab;  // flat index of row r0 + 1's first element
  const float mx0 = saved_max[r0], inv0 = 1.0f / saved_sum[r0];
  const float mx1 = saved_max[r1], inv1 = 1.0f / saved_sum[r1];
  const int64_t t0 = static_cast<int64_t>(targets[r0]), t1 = static_cast<int64_t>(targets[r1]);
  const float scale = (grad_output ? grad_output[0] : 1.0f) * host_scale;
  if (blockIdx.x == 0 && tid < head)  // buffer head: row 0
    grad[tid] = ce_grad1(logits[tid], mx0, inv0, scale, tid == t0);
  if (blockIdx.x == gridDim.x - 1) {  // buffer tail: the last row
    const int64_t j = head + 4 * nvec + tid;
    if (j < rows * vocab) {
      const int64_t rl = rows - 1;
      grad[j] = ce_grad1(logits[j], saved_max[rl], 1.0f / saved_sum[rl], scale,
                         j - rl * vocab == static_cast<int64_t>(targets[rl]));
    }
  }
  if (v < nvec) {
    const int64_t e = head + 4 * v;
    const float xs[4] = {x.x, x.y, x.z, x.w};
    float os[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool second = e + c >= start1;
      const int64_t col = e + c - (second ? start1 : start1 - vocab);
      os[c] = ce_grad1(xs[c], second ? mx1 : mx0, second ? inv1 : inv0, scale,
                       col == (second ? t1 : t0));
    }
    hk::st_nt(reinterpret_cast<float4*>(grad + head) + v, make_float4(os[0], os[1], os[2], os[3]));
  }
}

// Scalar path for a grad buffer whose 16-byte phase differs from the logits buffer's.
template <typename TIdx>
__global__ __launch_bounds__(kThreads) void ce_backward_scalar(
    const float* __restrict__ logits, const TIdx* __restrict__ targets,
    float* __restrict__ grad, const float* __restrict__ saved_max,
    const float* __restrict__ saved_sum, int64_t vocab, const float* __restrict__ grad_output,
    float host_scale) {
  const int64_t row = blockIdx.x;
  const float* x = logits + row * vocab;
  float* g = grad + row * vocab;
  const float mx = saved_max[row];
  const float inv_sum = 1.0f / saved_sum[row];
  const float scale = (grad_output ? grad_output[0] : 1.0f) * host_scale;
  const int64_t t = static_cast<int64_t>(targets[row]);
  for (int64_t j = threadIdx.x; j < vocab; j += kThreads)
    g[j] = ce_grad1(x[j], mx, inv_sum, scale, j == t);
}

template <typename TIdx>
hipError_t ce_forward_launch(const float* logits, const TIdx* targets, float* losses,
                             float* saved_max, float* saved_sum, int64_t batch_size,
                             int64_t vocab_size, hipStream_t stream) {
  HK_CHECK_ARG(batch_size >= 0 && vocab_size >= 1 && batch_size <= INT32_MAX);
  if (batch_size == 0) return hipSuccess;
  HK_CHECK_ARG(logits && targets && losses && saved_max && saved_sum);
  hipLaunchKernelGGL(ce_forward<TIdx>, dim3(static_cast<unsigned>(batch_size)), dim3(kFwdThreads),
                     0, stream, logits, targets, losses, saved_max, saved_sum, vocab_size);
  return hk::launch_status();
}

template <typename TIdx>
hipError_t ce_backward_launch(const float* logits, const TIdx* targets, float* grad,
                              const float* saved_max, const float* saved_sum, int64_t batch_size,
                              int64_t vocab_size, const float* grad_output, float host_scale,
                              hipStream_t stream) {
  HK_CHECK_ARG(batch_size >= 0 && vocab_size >= 1 && batch_size <= INT32_MAX);
  if (batch_size == 0) return hipSuccess;
  HK_CHECK_ARG(logits && targets && grad && saved_max && saved_sum);
  const bool same_phase = ((reinterpret_cast<uintptr_t>(logits) ^
                            reinterpret_cast<uintptr_t>(grad)) & 15u) == 0;
  if (!same_phase) {
    hipLaunchKernelGGL(ce_backward_scalar<TIdx>, dim3(static_cast<unsigned>(batch_size)),
                       dim3(kThreads), 0, stream, logits, targets, grad, saved_max, saved_sum,
                       vocab_size, grad_output, host_scale);
    return hk::launch_status();
  }
  if (vocab_size >= 4 * kFlatThreads) {
    const int64_t total = batch_size * vocab_size;
    const int64_t head = (4 - ((reinterpret_cast<uintptr_t>(logits) >> 2) & 3)) & 3;
    const int64_t nvec = (total - head) / 4;
    const int64_t blocks = hk::ceil_div(nvec, int64_t{kFlatThreads});
    HK_CHECK_ARG(blocks <= INT32_MAX);
    hipLaunchKernelGGL(ce_backward_flat<TIdx>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kFlatThreads), 0, stream, logits, targets, grad, saved_max, saved_sum,
                       batch_size, vocab_size, head, nvec, grad_output, host_scale);
    return hk::launch_status();
  }
  // body vectors per row are at most vocab / 4; at least one chunk per row (head/tail only)
  const int64_t nchunks = hk::ceil_div(vocab_size / 4 + 1, kChunkVec);
  HK_CHECK_ARG(nchunks <= INT32_MAX && batch_size * nchunks <= INT32_MAX);
  hipLaunchKernelGGL(ce_backward<TIdx>, dim3(static_cast<unsigned>(batch_size * nchunks)),
                     dim3(kBwdThreads), 0, stream, logits, targets, grad, saved_max, saved_sum,
                     vocab_size, static_cast<int>(nchunks), grad_output, host_scale);
  return hk::launch_status();
}

}  // namespace

#define HK_CE_ENTRY_POINTS(SUFFIX, TIdx)                                                          \
  extern "C" hipError_t hk_sparse_ce_forward_f32_##SUFFIX(                                       \
      const float* logits, const TIdx* targets, float* losses, float* saved_max,                 \
      float* saved_sum, int64_t batch_size, int64_t vocab_size, hipStream_t stream) {            \
    return ce_forward_launch<TIdx>(logits, targets, losses, saved_max, saved_sum, batch_size,    \
                                   vocab_size, stream);                                          \
  }                                                                                              \
  extern "C" hipError_t hk_sparse_ce_backward_f32_##SUFFIX(                                      \
      const float* logits, const TIdx* targets, float* grad, const float* saved_max,             \
      const float* saved_sum, int64_t batch_size, int64_t vocab_size, const float* grad_output,  \
      float host_scale, hipStream_t stream) {                                                    \
    return ce_backward_launch<TIdx>(logits, targets, grad, saved_max, saved_sum, batch_size,     \
                                    vocab_size, grad_output, host_scale, stream);                \
  }

HK_CE_ENTRY_POINTS(i32, int32_t)
HK_CE_ENTRY_POINTS(i64, int64_t)
HK_CE_ENTRY_POINTS(u16, uint16_t)
