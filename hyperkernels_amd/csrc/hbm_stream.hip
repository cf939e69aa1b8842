// hbm_stream.hip - a measurement kernel with no counterpart in the reference: it streams n_in
// fp32 arrays from HBM and n_out fp32 arrays to HBM (out_j = sum of the inputs + j), with the
// same access pattern as this library's memory-bound kernels: 16-byte non-temporal accesses,
// 256 lanes per workgroup, `unroll` consecutive 4 KiB spans per workgroup and stream. Timing it
// at a kernel's read/write mix and size gives the HBM rate that mix can reach on the device:
// the ceiling a memory-bound kernel of the path is judged against (AdamW is 4 reads and 3
// writes per element, LayerNorm backward 2 and 1, LayerNorm forward and GELU forward 1 and 1).
#include "hk_device.h"
#include "hk_host.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxIn = 4;
constexpr int kMaxOut = 3;

struct StreamPtrs {
  const float4* in[kMaxIn];
  float4* out[kMaxOut];
};

template <int NIN, int NOUT, int U>
__global__ __launch_bounds__(kThreads) void hbm_stream(StreamPtrs p, int64_t nvec,
                                                       float* __restrict__ sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * U + threadIdx.x;
  float4 acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + static_cast<int64_t>(u) * kThreads;
    acc[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < nvec) {
#pragma unroll
      for (int s = 0; s < NIN; ++s) {
        const float4 v = hk::ld_nt(p.in[s] + i);
        acc[u].x += v.x; acc[u].y += v.y; acc[u].z += v.z; acc[u].w += v.w;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + static_cast<int64_t>(u) * kThreads;
    if (i >= nvec) continue;
#pragma unroll
    for (int s = 0; s < NOUT; ++s) {
      const float j = static_cast<float>(s);
      hk::st_nt(p.out[s] + i, make_float4(acc[u].x + j, acc[u].y + j, acc[u].z + j, acc[u].w + j));
    }
    if constexpr (NOUT == 0) {
      // a data-dependent store that random inputs never take keeps every load live
      const float t = (acc[u].x + acc[u].y) + (acc[u].z + acc[u].w);
      if (t == 1234.5f) sink[blockIdx.x] = t;
    }
  }
}

template <int NIN, int NOUT>
hipError_t launch(const StreamPtrs& p, int64_t nvec, int unroll, float* sink, hipStream_t stream) {
  const int64_t per = static_cast<int64_t>(kThreads) * unroll;
  const unsigned grid = static_cast<unsigned>(hk::ceil_div(nvec, per));
  switch (unroll) {
    case 1: hipLaunchKernelGGL((hbm_stream<NIN, NOUT, 1>), dim3(grid), dim3(kThreads), 0, stream, p, nvec, sink); break;
    case 2: hipLaunchKernelGGL((hbm_stream<NIN, NOUT, 2>), dim3(grid), dim3(kThreads), 0, stream, p, nvec, sink); break;
    case 4: hipLaunchKernelGGL((hbm_stream<NIN, NOUT, 4>), dim3(grid), dim3(kThreads), 0, stream, p, nvec, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hk::launch_status();
}

template <int NIN, int NOUT = 0>
hipError_t dispatch(int n_out, const StreamPtrs& p, int64_t nvec, int unroll, float* sink,
                    hipStream_t stream) {
  if constexpr (NOUT > kMaxOut) {
    return hipErrorInvalidValue;
  } else {
    if (n_out == NOUT) return launch<NIN, NOUT>(p, nvec, unroll, sink, stream);
    return dispatch<NIN, NOUT + 1>(n_out, p, nvec, unroll, sink, stream);
  }
}

}  // namespace

extern "C" HK_API hipError_t hk_hbm_stream(const float* const* in, int n_in, float* const* out,
                                          int n_out, int64_t n, int unroll, float* sink,
                                          hipStream_t stream) {
  HK_CHECK_ARG(n_in >= 0 && n_in <= kMaxIn && n_out >= 0 && n_out <= kMaxOut);
  HK_CHECK_ARG(n_in + n_out > 0 && n >= 0 && n % 4 == 0);
  HK_CHECK_ARG(unroll == 1 || unroll == 2 || unroll == 4);
  HK_CHECK_ARG(n_out > 0 || sink);
  if (n == 0) return hipSuccess;
  StreamPtrs p{};
  for (int s = 0; s < n_in; ++s) {
    HK_CHECK_ARG(in && in[s] && hk::aligned16(in[s]));
    p.in[s] = reinterpret_cast<const float4*>(in[s]);
  }
  for (int s = 0; s < n_out; ++s) {
    HK_CHECK_ARG(out && out[s] && hk::aligned16(out[s]));
    p.out[s] = reinterpret_cast<float4*>(out[s]);
  }
  const int64_t nvec = n / 4;
  switch (n_in) {
    case 0: return dispatch<0>(n_out, p, nvec, unroll, sink, stream);
    case 1: return dispatch<1>(n_out, p, nvec, unroll, sink, stream);
    case 2: return dispatch<2>(n_out, p, nvec, unroll, sink, stream);
    case 3: return dispatch<3>(n_out, p, nvec, unroll, sink, stream);
    default: return dispatch<4>(n_out, p, nvec, unroll, sink, stream);
  }
}
