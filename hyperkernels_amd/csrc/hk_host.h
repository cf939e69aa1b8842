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

// Device scratch owned by the library: one grow-only buffer per device, kept until the
// process ends. The returned pointer is valid until the next call on the same device asks for
// more bytes, so a launcher must fetch it once per call. Calls on one device that overlap in
// time on different streams must not share it; the launchers here synchronise on nothing, so
// the workspace is only handed to work on the caller's stream, and growing it waits for the
// device first.
hipError_t device_workspace(size_t bytes, void** out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Status of the launch just issued on this thread.
inline hipError_t launch_status() { return hipGetLastError(); }

}  // namespace hk
