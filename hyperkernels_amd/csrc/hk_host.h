// hk_host.h - host-side helpers shared by the launchers (validation, device facts, workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hk.h"

#define HK_CHECK_ARG(cond)                 \
  do {                                     \
    if (!(cond)) return hipErrorInvalidValue; \
  } while (0)

#define HK_RETURN_IF_ERROR(expr)           \
  do {                                     \
    hipError_t hk_e_ = (expr);             \
    if (hk_e_ != hipSuccess) return hk_e_; \
  } while (0)

namespace hk {

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Scratch device memory for the launchers' multi-workgroup partials (split-K, reduce, the
// LayerNorm gamma/beta partials): one grow-only buffer per (device, stream), held until the
// process ends. Work on one stream runs in order, so consecutive calls on that stream reuse
// the buffer safely; calls on different streams get different buffers. The pointer is valid
// until the next call on the same (device, stream) asks for more bytes, so a launcher fetches
// it once per call; growing it first waits for the work queued on that stream.
hipError_t device_workspace(size_t bytes, hipStream_t stream, void** out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Status of the launch just issued on this thread.
inline hipError_t launch_status() { return hipGetLastError(); }

}  // namespace hk
