// HBM read-stream probe: the measured bandwidth ceiling that the decode GEMVs' fraction of
// peak is stated against beside the 8 TB/s datasheet figure.  The reference measures its card the
// same way, with a read-only stream over a 1 GB buffer (/root/reference/tools/w0_e4_bw.cu; 880 GB/s
// = 94% of the RTX 3090's 936 GB/s, docs/history/W0_E4_BANDWIDTH.md:27).
//
// Each workgroup reads one contiguous 64 KB chunk: 256 threads x 16 loads of 16 B, all issued
// before the first use (a 64-B run per lane quad per load: the coalesced pattern of the vector
// memory path), folds them with XOR and stores one word per workgroup so the loads stay live.
#include "tlx_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kLoads = 16;
constexpr size_t kChunk = size_t(kThreads) * kLoads * 16;   // bytes per workgroup

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u4_t* __restrict__ src, uint32_t* __restrict__ sink) {
  const u4_t* p = src + (size_t)blockIdx.x * (kChunk / 16) + threadIdx.x;
  u4_t v[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) v[i] = __builtin_nontemporal_load(p + i * kThreads);
  u4_t a = v[0];
#pragma unroll
  for (int i = 1; i < kLoads; ++i) a ^= v[i];
  uint32_t x = a.x ^ a.y ^ a.z ^ a.w;
  // one word per workgroup (a wave-level fold keeps the store count negligible)
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

}  // namespace

extern "C" uint64_t tlx_stream_chunk_bytes(void) { return kChunk; }

extern "C" int tlx_stream_read(const void* src, uint64_t nbytes, uint32_t* sink, void* stream) {
  TLX_RET_IF(nbytes == 0 || nbytes % kChunk != 0 || nbytes / kChunk > 0x7fffffffull, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(src, 16) || !tlx_aligned(sink, 4), TLX_E_ALIGN);
  stream_read_kernel<<<(unsigned)(nbytes / kChunk), kThreads, 0, (hipStream_t)stream>>>((const u4_t*)src, sink);
  return tlx_launch_status();
}
