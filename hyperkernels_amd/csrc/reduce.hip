// reduce.hip - unified fp32 sum reduction over an inner, outer or generic strided axis.
//
// Reference behaviour: kernels/reduction/unified_reduce_standalone.cu. ReductionLayout
// (:46-56) names the three paths; the kernel index maps are at :389-445 (inner rows read
// base = o * reduced_count; outer columns read base = (o / inner) * outer_stride + o % inner
// with a row stride; generic paths add an output offset and an input offset from two
// OffsetCalculators, :224-249); the host solver build_reduce_config (:151-221) picks block
// shape and a multi-CTA split; launch_reduce_kernel (:702-804) allocates staging with
// cudaMalloc on every call.
//
// Design (gfx950): the host picks one of three launch shapes below and, when one output's
// work is too small a share of the 256 CUs, splits the reduced axis over several workgroups.
// The split writes partials [split][num_outputs] to the library's per-device workspace and a
// second kernel sums them in slice order, so results are deterministic and nothing is
// allocated per call (the reference stages through freshly allocated memory and semaphores).
//   inner:   a workgroup (512 lanes) per output row slice, 16-byte loads after a head peel
//            when the row is long; a 64-lane wave per output when rows are short.
//   outer:   a lane per output (consecutive lanes read consecutive columns), 8 rows in
//            flight per lane, the reduced axis split over blockIdx.y.
//   generic: a wave per output; each lane walks the reduced index space with the strided
//            offset map.
#include <algorithm>
#include <mutex>
#include <vector>

#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / HK_WAVE;

// ---- inner, long rows: workgroup per (output, slice) ----------------------------------------
// 512 lanes with four 16-byte loads each in flight, the body's remainder included: a row
// slice is a short chain of dependent load rounds, so lanes per row and loads per round set
// the rate (measured on MI355X at 16384 x 50304: ~7.0 TB/s, against 5.6 TB/s for 256 lanes
// with a one-load remainder loop).
constexpr int kBlockThreads = 512;
constexpr int kBlockWaves = kBlockThreads / HK_WAVE;
constexpr int kBlockUnroll = 4;

__global__ __launch_bounds__(kBlockThreads) void reduce_inner_block(const float* __restrict__ src,
                                                                    float* __restrict__ dst,
                                                                    int64_t row_stride,
                                                                    int64_t len,
                                                                    int64_t slice_len,
                                                                    int64_t nout) {
  __shared__ float red[kBlockWaves];
  const int64_t o = blockIdx.x;
  const int64_t s0 = static_cast<int64_t>(blockIdx.y) * slice_len;
  int64_t s1 = s0 + slice_len;
  if (s1 > len) s1 = len;
  const float* row = src + o * row_stride;
  const int tid = threadIdx.x;
  float acc[kBlockUnroll] = {};
  if (s0 < s1) {
    const float* x = row + s0;
    const int64_t n = s1 - s0;
    int64_t h = (4 - ((reinterpret_cast<uintptr_t>(x) >> 2) & 3)) & 3;
    if (h > n) h = n;
    const int64_t nb = (n - h) >> 2;
    if (tid < h) acc[0] += x[tid];
    const float4* b = reinterpret_cast<const float4*>(x + h);
    int64_t i = tid;
    for (; i + (kBlockUnroll - 1) * kBlockThreads < nb; i += kBlockUnroll * kBlockThreads) {
      float4 v[kBlockUnroll];
#pragma unroll
      for (int u = 0; u < kBlockUnroll; ++u) v[u] = hk::ld_nt(b + i + u * kBlockThreads);
#pragma unroll
      for (int u = 0; u < kBlockUnroll; ++u) acc[u] += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    {  // remainder of the body, the same loads in flight, predicated
      float4 v[kBlockUnroll];
      bool ok[kBlockUnroll];
#pragma unroll
      for (int u = 0; u < kBlockUnroll; ++u) {
        ok[u] = i + u * kBlockThreads < nb;
        if (ok[u]) v[u] = hk::ld_nt(b + i + u * kBlockThreads);
      }
#pragma unroll
      for (int u = 0; u < kBlockUnroll; ++u)
        if (ok[u]) acc[u] += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (int64_t j = h + 4 * nb + tid; j < n; j += kBlockThreads) acc[1] += x[j];
  }
  float v = hk::wave_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kBlockWaves; ++w) t += red[w];
    dst[static_cast<int64_t>(blockIdx.y) * nout + o] = t;
  }
}

// ---- inner, short rows: wave per output --------------------------------------------------------
__global__ __launch_bounds__(kThreads) void reduce_inner_wave(const float* __restrict__ src,
                                                              float* __restrict__ dst,
                                                              int64_t row_stride, int64_t len,
                                                              int64_t nout) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (o >= nout) return;
  const int lane = threadIdx.x & 63;
  const float* row = src + o * row_stride;
  float a0 = 0.f, a1 = 0.f;
  int64_t k = lane;
  for (; k + HK_WAVE < len; k += 2 * HK_WAVE) {
    a0 += row[k];
    a1 += row[k + HK_WAVE];
  }
  if (k < len) a0 += row[k];
  const float t = hk::wave_sum(a0 + a1);
  if (lane == 0) dst[o] = t;
}

// ---- outer: lane per output, reduced axis split over blockIdx.y --------------------------------
__global__ __launch_bounds__(kThreads) void reduce_outer(const float* __restrict__ src,
                                                         float* __restrict__ dst, int64_t nout,
                                                         int64_t inner, int64_t outer_stride,
                                                         int64_t row_stride, int64_t len,
                                                         int64_t slice_len) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (o >= nout) return;
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * slice_len;
  int64_t k1 = k0 + slice_len;
  if (k1 > len) k1 = len;
  const float* base = src + (o / inner) * outer_stride + (o % inner);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t k = k0;
  for (; k + 7 < k1; k += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += base[(k + u) * row_stride];
  }
  for (; k < k1; ++k) acc[0] += base[k * row_stride];
  dst[static_cast<int64_t>(blockIdx.y) * nout + o] =
      ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// ---- generic: wave per output ---------------------------------------------------------------
struct StridedMap {
  int ndim;
  int64_t sizes[HK_REDUCE_MAX_DIMS];
  int64_t strides[HK_REDUCE_MAX_DIMS];
};

__device__ __forceinline__ int64_t map_offset(const StridedMap& m, int64_t linear) {
  int64_t off = 0;
  for (int d = m.ndim - 1; d >= 0; --d) {
    const int64_t c = linear % m.sizes[d];
    linear /= m.sizes[d];
    off += c * m.strides[d];
  }
  return off;
}

__global__ __launch_bounds__(kThreads) void reduce_generic(const float* __restrict__ src,
                                                           float* __restrict__ dst,
                                                           StridedMap out_map, StridedMap red_map,
                                                           int64_t nout, int64_t len) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (o >= nout) return;
  const int lane = threadIdx.x & 63;
  const float* base = src + map_offset(out_map, o);
  float a = 0.f;
  for (int64_t k = lane; k < len; k += HK_WAVE) a += base[map_offset(red_map, k)];
  const float t = hk::wave_sum(a);
  if (lane == 0) dst[o] = t;
}

// ---- split finalize: dst[o] = sum_s part[s][o] in slice order ---------------------------------
__global__ __launch_bounds__(kThreads) void reduce_finalize(const float* __restrict__ part,
                                                            float* __restrict__ dst, int64_t nout,
                                                            int split) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (o >= nout) return;
  float s = 0.f;
  for (int i = 0; i < split; ++i) s += part[static_cast<int64_t>(i) * nout + o];
  dst[o] = s;
}

hipError_t finalize(const float* part, float* dst, int64_t nout, int split, hipStream_t stream) {
  hipLaunchKernelGGL(reduce_finalize, dim3(static_cast<unsigned>(hk::ceil_div(nout, kThreads))),
                     dim3(kThreads), 0, stream, part, dst, nout, split);
  return hk::launch_status();
}

// Workgroups wanted in flight to cover the device: 2 per CU.
int64_t target_groups() { return static_cast<int64_t>(hk::device_cu_count()) * 2; }

// Where a split reduction keeps its partials [split][num_outputs]: the library's grow-only
// workspace of the stream (scratch == nullptr), or a fixed scratch array of `scratch_bytes`
// (the entry point that allocates nothing), which a plan needing more bytes is refused.
struct PartialSource {
  float* scratch = nullptr;
  size_t scratch_bytes = 0;

  hipError_t get(size_t bytes, hipStream_t stream, float** out) const {
    if (scratch) {
      if (bytes > scratch_bytes) return hipErrorInvalidValue;
      *out = scratch;
      return hipSuccess;
    }
    void* ws = nullptr;
    HK_RETURN_IF_ERROR(hk::device_workspace(bytes, stream, &ws));
    *out = static_cast<float*>(ws);
    return hipSuccess;
  }
};

hipError_t reduce_inner(const float* src, float* dst, int64_t nout, int64_t len,
                        int64_t row_stride, const PartialSource& ps, hipStream_t stream) {
  if (len < 1024) {
    hipLaunchKernelGGL(reduce_inner_wave, dim3(static_cast<unsigned>(hk::ceil_div(nout, kWaves))),
                       dim3(kThreads), 0, stream, src, dst, row_stride, len, nout);
    return hk::launch_status();
  }
  // Split a row over several workgroups when there are too few rows to cover the device; each
  // slice keeps at least 16 KiB of work.
  int64_t split = 1;
  if (nout < target_groups()) {
    split = std::min<int64_t>(hk::ceil_div(target_groups(), nout), hk::ceil_div(len, 4096));
    split = std::max<int64_t>(split, 1);
  }
  HK_CHECK_ARG(nout <= INT32_MAX && split <= 65535);
  const int64_t slice_len = hk::ceil_div(hk::ceil_div(len, split), 4) * 4;
  split = hk::ceil_div(len, slice_len);
  float* out = dst;
  if (split > 1)
    HK_RETURN_IF_ERROR(ps.get(static_cast<size_t>(split * nout) * sizeof(float), stream, &out));
  hipLaunchKernelGGL(reduce_inner_block, dim3(static_cast<unsigned>(nout), static_cast<unsigned>(split)),
                     dim3(kBlockThreads), 0, stream, src, out, row_stride, len, slice_len, nout);
  HK_RETURN_IF_ERROR(hk::launch_status());
  if (split > 1) return finalize(out, dst, nout, static_cast<int>(split), stream);
  return hipSuccess;
}

hipError_t reduce_outer_launch(const float* src, float* dst, int64_t nout, int64_t inner,
                               int64_t outer_stride, int64_t row_stride, int64_t len,
                               const PartialSource& ps, hipStream_t stream) {
  const int64_t gx = hk::ceil_div(nout, kThreads);
  int64_t split = 1;
  if (gx < target_groups() * 2) {
    split = std::min<int64_t>(hk::ceil_div(target_groups() * 2, gx), hk::ceil_div(len, 64));
    split = std::max<int64_t>(split, 1);
  }
  HK_CHECK_ARG(gx <= INT32_MAX && split <= 65535);
  const int64_t slice_len = hk::ceil_div(len, split);
  split = hk::ceil_div(len, slice_len);
  float* out = dst;
  if (split > 1)
    HK_RETURN_IF_ERROR(ps.get(static_cast<size_t>(split * nout) * sizeof(float), stream, &out));
  hipLaunchKernelGGL(reduce_outer, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(split)),
                     dim3(kThreads), 0, stream, src, out, nout, inner, outer_stride, row_stride,
                     len, slice_len);
  HK_RETURN_IF_ERROR(hk::launch_status());
  if (split > 1) return finalize(out, dst, nout, static_cast<int>(split), stream);
  return hipSuccess;
}

__global__ void fill_zero(float* __restrict__ dst, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) dst[i] = 0.f;
}

hipError_t zero_outputs(float* dst, int64_t nout, hipStream_t stream) {
  hipLaunchKernelGGL(fill_zero, dim3(static_cast<unsigned>(hk::ceil_div(nout, kThreads))),
                     dim3(kThreads), 0, stream, dst, nout);
  return hk::launch_status();
}

// Scratch of the entry point that allocates nothing (hk_unified_reduce_sum_f32_noalloc): the
// split partials [split][num_outputs] of one call, at most kScratchBytes. Each device holds
// its own copy for the life of the process. Every slot a call uses is written by that call's
// first kernel before its finalize reads it, so nothing needs clearing; calls that overlap on
// one device share the array and race.
constexpr size_t kScratchBytes = HK_REDUCE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device address of `scratch` on the current device, looked up once per device with that
// device current (the host-side name is only a stand-in for the symbol, not an address).
hipError_t scratch_address(float** out) {
  static std::mutex mu;
  static std::vector<float*> addr;
  int dev = 0;
  HK_RETURN_IF_ERROR(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(mu);
  if (static_cast<int>(addr.size()) <= dev) addr.resize(dev + 1, nullptr);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    HK_RETURN_IF_ERROR(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    addr[dev] = static_cast<float*>(p);
  }
  *out = addr[dev];
  return hipSuccess;
}

hipError_t unified_reduce(const hk_reduction_layout* layout, const float* src, float* dst,
                          const PartialSource& ps, hipStream_t stream) {
  HK_CHECK_ARG(layout != nullptr);
  const hk_reduction_layout& L = *layout;
  HK_CHECK_ARG(L.num_outputs >= 0 && L.reduced_count >= 0);
  if (L.num_outputs == 0) return hipSuccess;
  HK_CHECK_ARG(dst != nullptr);
  if (L.reduced_count == 0) return zero_outputs(dst, L.num_outputs, stream);
  HK_CHECK_ARG(src != nullptr);
  switch (L.path) {
    case HK_REDUCE_INNER: {
      const int64_t row_stride = L.input_outer_stride > 0 ? L.input_outer_stride : L.reduced_count;
      return reduce_inner(src, dst, L.num_outputs, L.reduced_count, row_stride, ps, stream);
    }
    case HK_REDUCE_OUTER: {
      const int64_t inner = L.inner_count > 0 ? L.inner_count : L.num_outputs;
      HK_CHECK_ARG(L.input_row_stride > 0);
      return reduce_outer_launch(src, dst, L.num_outputs, inner, L.input_outer_stride,
                                 L.input_row_stride, L.reduced_count, ps, stream);
    }
    case HK_REDUCE_GENERIC: {
      // A layout-only generic request describes contiguous rows (the reference self-test's
      // generic case, unified_reduce_standalone.cu:871-881).
      const int64_t row_stride = L.input_outer_stride > 0 ? L.input_outer_stride : L.reduced_count;
      const int64_t out_sizes[1] = {L.num_outputs}, out_strides[1] = {row_stride};
      const int64_t red_sizes[1] = {L.reduced_count}, red_strides[1] = {1};
      return hk_reduce_generic_f32(src, dst, 1, out_sizes, out_strides, 1, red_sizes, red_strides,
                                   stream);
    }
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

extern "C" hipError_t hk_unified_reduce_sum_f32(const hk_reduction_layout* layout,
                                                const float* src, float* dst,
                                                hipStream_t stream) {
  return unified_reduce(layout, src, dst, PartialSource{}, stream);
}

extern "C" hipError_t hk_unified_reduce_sum_f32_noalloc(const hk_reduction_layout* layout,
                                                        const float* src, float* dst,
                                                        hipStream_t stream) {
  PartialSource ps;
  HK_RETURN_IF_ERROR(scratch_address(&ps.scratch));
  ps.scratch_bytes = kScratchBytes;
  return unified_reduce(layout, src, dst, ps, stream);
}

extern "C" hipError_t hk_reduce_generic_f32(const float* src, float* dst, int out_ndim,
                                            const int64_t* out_sizes, const int64_t* out_strides,
                                            int red_ndim, const int64_t* red_sizes,
                                            const int64_t* red_strides, hipStream_t stream) {
  HK_CHECK_ARG(out_ndim >= 0 && out_ndim <= HK_REDUCE_MAX_DIMS);
  HK_CHECK_ARG(red_ndim >= 0 && red_ndim <= HK_REDUCE_MAX_DIMS);
  StridedMap om{}, rm{};
  int64_t nout = 1, len = 1;
  om.ndim = out_ndim;
  rm.ndim = red_ndim;
  for (int d = 0; d < out_ndim; ++d) {
    HK_CHECK_ARG(out_sizes && out_strides && out_sizes[d] >= 0);
    om.sizes[d] = out_sizes[d];
    om.strides[d] = out_strides[d];
    nout *= out_sizes[d];
  }
  for (int d = 0; d < red_ndim; ++d) {
    HK_CHECK_ARG(red_sizes && red_strides && red_sizes[d] >= 0);
    rm.sizes[d] = red_sizes[d];
    rm.strides[d] = red_strides[d];
    len *= red_sizes[d];
  }
  if (nout == 0) return hipSuccess;
  HK_CHECK_ARG(dst != nullptr);
  if (len == 0) return zero_outputs(dst, nout, stream);
  HK_CHECK_ARG(src != nullptr);
  hipLaunchKernelGGL(reduce_generic, dim3(static_cast<unsigned>(hk::ceil_div(nout, kWaves))),
                     dim3(kThreads), 0, stream, src, dst, om, rm, nout, len);
  return hk::launch_status();
}
