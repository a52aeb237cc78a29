// Library-level entry points (version, error strings) and the per-device workspace.
#include "tlx_common.h"

#include <mutex>

extern "C" int tlx_version(void) { return 1; }

extern "C" const char* tlx_strerror(int code) {
  switch (code) {
    case TLX_OK: return "ok";
    case TLX_E_ARG: return "argument out of range (M, sizes or layout)";
    case TLX_E_ALIGN: return "pointer or row stride misaligned for this layout";
    case TLX_E_NODEV: return "no usable gfx950 device";
    case TLX_E_NOMEM: return "the library workspace could not be allocated";
    case TLX_E_TRUNC: return "the GGUF image ends inside the header";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown tlx error";
  }
}

// One workspace of kWsBytes per device, allocated on the first call that needs it.
int tlx_workspace(void** ws) {
  static std::mutex mu;
  static void* cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TLX_E_NODEV;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == nullptr) {
    // zeroed once: the arrival counters of the tiled-record GEMV start (and end every call) at 0
    if (hipMalloc(&cache[dev], kWsBytes) != hipSuccess || hipMemset(cache[dev], 0, kWsBytes) != hipSuccess) {
      if (cache[dev] != nullptr) (void)hipFree(cache[dev]);
      cache[dev] = nullptr;
      return TLX_E_NOMEM;
    }
  }
  *ws = cache[dev];
  return TLX_OK;
}

// The prefill GEMM's stream-K workspace, allocated and zeroed on first use per device.
int tlx_workspace_gemm(void** ws) {
  static std::mutex mu;
  static void* cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TLX_E_NODEV;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == nullptr) {
    if (hipMalloc(&cache[dev], kPfWsBytes) != hipSuccess || hipMemset(cache[dev], 0, kPfWsBytes) != hipSuccess) {
      if (cache[dev] != nullptr) (void)hipFree(cache[dev]);
      cache[dev] = nullptr;
      return TLX_E_NOMEM;
    }
  }
  *ws = cache[dev];
  return TLX_OK;
}
