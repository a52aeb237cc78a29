// Library-level entry points (version, error strings) and the caller-attached per-device workspaces.
#include "tlx_common.h"

#include <atomic>
#include <mutex>

extern "C" int tlx_version(void) { return 1; }

extern "C" const char* tlx_strerror(int code) {
  switch (code) {
    case TLX_OK: return "ok";
    case TLX_E_ARG: return "argument out of range (M, sizes or layout)";
    case TLX_E_ALIGN: return "pointer or row stride misaligned for this layout";
    case TLX_E_NODEV: return "no usable gfx950 device";
    case TLX_E_NOMEM: return "out of memory";
    case TLX_E_NOWS: return "no workspace attached on this device (tlx_attach_workspace)";
    case TLX_E_TRUNC: return "the GGUF image ends inside the header";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown tlx error";
  }
}

namespace {

// Per-device workspaces the caller attached (tlx_attach_workspace); the library allocates none.
struct DevWs {
  void* gemv = nullptr;
  void* gemm = nullptr;
  size_t gemm_bytes = 0;
};
std::mutex g_ws_mu;
DevWs g_ws[64];

__global__ __launch_bounds__(256) void ws_zero_kernel(uint32_t* p, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0u;
}

}  // namespace

int tlx_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int tlx_ws_clear_counters(void* ws, hipStream_t st) {
  static_assert(kWsKcntOff == kWsCntOff + kWsCntBytes, "the two counter regions are cleared together");
  const int n = (int)((kWsCntBytes + kWsKcntBytes) / 4);
  ws_zero_kernel<<<(n + 255) / 256, 256, 0, st>>>(reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + kWsCntOff), n);
  return tlx_launch_status();
}

extern "C" int tlx_workspace_size(uint64_t* gemv_bytes, uint64_t* gemm_bytes) {
  if (gemv_bytes) *gemv_bytes = kWsBytes;
  if (gemm_bytes) *gemm_bytes = kPfWsBytes;
  return TLX_OK;
}

extern "C" int tlx_attach_workspace(void* gemv_ws, uint64_t gemv_bytes, void* gemm_ws, uint64_t gemm_bytes,
                                    void* stream) {
  TLX_RET_IF(gemv_ws != nullptr && gemv_bytes < kWsBytes, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(gemv_ws, 256) || !tlx_aligned(gemm_ws, 256), TLX_E_ALIGN);
  int dev = 0;
  TLX_RET_IF(hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64, TLX_E_NODEV);
  // the per-process and per-device one-time set-up, here so that later calls do none of it (they
  // may be made under stream capture): kernel attributes, the cached compute-unit count
  (void)tlx_cu_count();
  const int src = tlx_kq_setup();
  TLX_RET_IF(src != TLX_OK, src);
  const int scr = tlx_scratch_init(nullptr);   // tlx_ffn8_noalloc's scratch address on this device
  TLX_RET_IF(scr != TLX_OK, scr);
  if (gemv_ws != nullptr) {   // the arrival counters start at 0 (every complete call leaves them at 0)
    const int rc = tlx_ws_clear_counters(gemv_ws, (hipStream_t)stream);
    TLX_RET_IF(rc != TLX_OK, rc);
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  g_ws[dev].gemv = gemv_ws;
  g_ws[dev].gemm = gemm_ws;
  g_ws[dev].gemm_bytes = gemm_ws != nullptr ? (size_t)gemm_bytes : 0;
  return TLX_OK;
}

int tlx_workspace(void** ws) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TLX_E_NODEV;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  *ws = g_ws[dev].gemv;
  return TLX_OK;
}

int tlx_workspace_gemm(void** ws, size_t* bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TLX_E_NODEV;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  *ws = g_ws[dev].gemm;
  *bytes = g_ws[dev].gemm_bytes;
  return TLX_OK;
}
