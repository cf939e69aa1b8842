// runtime.hip - library-level state: ABI version, per-device facts and the workspaces.
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "hk_host.h"

extern "C" int hk_abi_version(void) { return HK_ABI_VERSION; }

extern "C" const char* hk_error_string(hipError_t status) { return hipGetErrorString(status); }

namespace hk {

namespace {
struct DeviceState {
  int cu_count = 0;
};
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_mu;
std::vector<DeviceState> g_devices;
// One grow-only workspace per (device, stream): work on one stream is ordered, so a call may
// reuse the buffer the previous call on that stream used; calls on different streams never
// share one.
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

DeviceState* state_for_current(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (static_cast<int>(g_devices.size()) <= dev) g_devices.resize(dev + 1);
  return &g_devices[dev];
}
}  // namespace

int device_cu_count() {
  std::lock_guard<std::mutex> lk(g_mu);
  hipError_t e;
  DeviceState* s = state_for_current(&e);
  if (!s) return 256;
  if (s->cu_count == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
      s->cu_count = cus;
    else
      s->cu_count = 256;
  }
  return s->cu_count;
}

hipError_t device_workspace(size_t bytes, hipStream_t stream, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  int dev = 0;
  HK_RETURN_IF_ERROR(hipGetDevice(&dev));
  Workspace& w = g_ws[std::make_pair(dev, stream)];
  if (bytes > w.bytes) {
    if (w.ptr) {
      // Work already queued on this stream may still read the old buffer.
      HK_RETURN_IF_ERROR(hipStreamSynchronize(stream));
      HK_RETURN_IF_ERROR(hipFree(w.ptr));
      w.ptr = nullptr;
      w.bytes = 0;
    }
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    HK_RETURN_IF_ERROR(hipMalloc(&w.ptr, want));
    w.bytes = want;
  }
  *out = w.ptr;
  return hipSuccess;
}

}  // namespace hk
