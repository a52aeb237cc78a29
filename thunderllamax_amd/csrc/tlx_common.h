// Shared device/host helpers for the gfx950 quantized-matmul library.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/tlx.h"

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

#define TLX_WAVE 64

// ---------------------------------------------------------------- host-side checks
#define TLX_RET_IF(cond, code) \
  do {                         \
    if (cond) return (code);   \
  } while (0)

static inline int tlx_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TLX_OK : (int)e;
}

static inline bool tlx_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ float tlx_h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint16_t tlx_f2h_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// fp16 pair {s * lo(h2), s * hi(h2)}: v_fma_mix takes the two fp16 halves of h2 as operands and
// rounds each product to fp16 once, from the exact value (measured: 1 + 2^-11 + 2^-40 gives
// 1 + 2^-10, not the 1.0 an intermediate f32 rounding would).  So it is the reference's fp16(f32
// product) bit for bit only where the product is exact in f32 -- a block scale of <= 18
// significant bits (fp16 d times a small integer) times a level of <= 6 -- and is not used for
// a*q - b forms (Q4_K / Q5_K), whose f32 result can round.
__device__ __forceinline__ uint32_t tlx_mix2_f16(float s, uint32_t h2) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
      : "=&v"(r)
      : "v"(s), "v"(h2));
  return r;
}

// An MFMA does not wait for a VALU result in its source registers: 2 wait states must separate the
// write and the read, and the compiler inserts none after inline asm it does not look into (such as
// the v_fma_mix above).  An operand built by tlx_mix2_f16 and read by an MFMA directly passes
// through this guard first: its nops sit after the operand's last write (the asm takes the operand
// as an input) and before the MFMA (which takes it as an output).
__device__ __forceinline__ void tlx_mfma_operand_guard(u4_t& h) { asm volatile("s_nop 2" : "+v"(h)); }

// fp16 pair of bytes {0, 1} (hi = 0) or {2, 3} (hi = 1) of v as the integers byte - bias: v_perm
// puts 0x64 above each byte (the fp16 1024 + byte, exact), a packed fp16 add takes 1024 + bias off
// (exact: small integers).
__device__ __forceinline__ uint32_t tlx_bytes_h2(uint32_t v, int hi, float bias) {
  const uint32_t p = __builtin_amdgcn_perm(0x64646464u, v, hi ? 0x04030402u : 0x04010400u);
  const _Float16 o = (_Float16)(1024.f + bias);
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p) - h2_t{o, o});
}

// Loads through a byte pointer whose alignment is only known to be 2 (raw GGUF blocks).
template <typename T>
__device__ __forceinline__ T tlx_ldu(const uint8_t* p) {
  T v;
  __builtin_memcpy(&v, p, sizeof(T));
  return v;
}

// fp16 SiLU chain of the reference FFN epilogue (/root/reference/engine/ffn8.cu:22-24):
// h * rcp(1 + exp2(h * fp16(-log2 e))) with every step rounded to fp16.  The constant
// -1.4423828125 is fp16(-log2(e)).  exp2 and rcp are the ROCm device-library fp16 routines.
__device__ __forceinline__ __half tlx_hsilu(__half h) {
  const __half t = __hmul(h, __float2half(-1.4423828125f));
  const __half den = __hadd(__float2half(1.0f), hexp2(t));
  return __hmul(h, hrcp(den));
}

// SwiGLU epilogue: gact = silu16(half(g)) * half(u), all in fp16.
__device__ __forceinline__ uint16_t tlx_swiglu_bits(float g, float u) {
  const __half hg = __float2half(g);
  const __half hu = __float2half(u);
  return __builtin_bit_cast(uint16_t, __hmul(tlx_hsilu(hg), hu));
}

// IQ3_XXS sign-folded lookup table of the decode GEMVs, built by the workgroup in LDS from the
// caller's gridf buffer (float[256][4]): entry (nib << 8 | g) = grid[g][j] with the sign of bit j
// of nib, j = 0..3, as four fp16 values (grid magnitudes are exact in fp16).
// Entries (nib << 8 | g) for nib = 4q .. 4q+3 of grid word g (values v).
__device__ __forceinline__ void tlx_iq3_table_entries(u2_t* tbl, float4 v, int g, int q) {
  const h2_t lo = {(_Float16)v.x, (_Float16)v.y};
  const h2_t hi = {(_Float16)v.z, (_Float16)v.w};
  const uint32_t l = __builtin_bit_cast(uint32_t, lo), h = __builtin_bit_cast(uint32_t, hi);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t nib = 4 * q + i;
    const uint32_t ml = ((nib & 1u) << 15) | ((nib & 2u) << 30);
    const uint32_t mh = ((nib & 4u) << 13) | ((nib & 8u) << 28);
    tbl[(nib << 8) | g] = u2_t{l ^ ml, h ^ mh};
  }
}

__device__ __forceinline__ void tlx_iq3_table(u2_t* tbl, const float* __restrict__ gridf) {
  for (int e = threadIdx.x; e < 256 * 4; e += blockDim.x)
    tlx_iq3_table_entries(tbl, reinterpret_cast<const float4*>(gridf)[e & 255], e & 255, e >> 8);
}

// ---------------------------------------------------------------- device properties
// Compute-unit count of the current device (tlx_core.hip; cached per device, one cache for the
// whole library, filled at the latest by tlx_attach_workspace).
int tlx_cu_count();

// ---------------------------------------------------------------- workspace
// Device memory the caller owns and attaches per device (tlx_attach_workspace, tlx_core.hip):
// the IQ3_XXS decode GEMVs' scratch.  Calls that overlap in time on one device must not share it.
//   [0, 1 MB)            partial tiles of the tiled-record GEMV (4 KB per workgroup boundary)
//   [1 MB, +4 KB)        their arrival counters (0 between calls; zeroed by attach)
//   [1 MB + 4 KB, +4 KB) per-tile arrival counters of the k-split form (0 between calls)
//   [1 MB + 64 KB, +2 MB) the tile-ordered activation copy of the packed-row GEMVs (K * 32 B)
//   [3 MB + 64 KB, +4 MB) the k-split form's range partials ([tile][range][64 lanes] f4)
constexpr size_t kWsPartOff = 0;
constexpr size_t kWsCntOff = size_t(1) << 20;
constexpr size_t kWsCntBytes = 4096;
constexpr size_t kWsKcntOff = kWsCntOff + kWsCntBytes;
constexpr size_t kWsKcntBytes = 4096;
constexpr size_t kWsXtOff = (size_t(1) << 20) + (size_t(64) << 10);
constexpr size_t kWsXtBytes = size_t(2) << 20;
constexpr size_t kWsBaseBytes = kWsXtOff + kWsXtBytes;   // what the forms without the k-split use
constexpr size_t kWsKpartOff = kWsBaseBytes;
constexpr size_t kWsKpartBytes = size_t(4) << 20;
constexpr size_t kWsBytes = kWsKpartOff + kWsKpartBytes;
// The attached GEMV workspace of the current device (nullptr when none is attached).
int tlx_workspace(void** ws);
// Zeroes the arrival counters of a GEMV workspace with a fill kernel on `st` (no memset node:
// safe inside stream capture).
int tlx_ws_clear_counters(void* ws, hipStream_t st);
// Device address of tlx_ffn8_noalloc's static scratch on the current device (tlx_iq3.hip).
int tlx_scratch_init(void** ptr);

// RMSNorm producer (tlx_norm.hip): add form (hh = x + a) when add; optionally also writes the
// IQ3_XXS GEMVs' tile-ordered activation copy xt (M <= 16)
int tlx_rms_launch(bool add, const float* x, const uint16_t* a, const float* nw, float* hh, uint16_t* xh,
                   _Float16* xt, int M, int D, hipStream_t st);
int tlx_rms_check(const float* x, const uint16_t* a, const float* nw, const float* hh, const uint16_t* xh, int M, int D);
int tlx_workspace(void** ws);
// The prefill GEMM's split-tile workspace: fp32 parts of 256 x 256 tiles (256 KB each), caller
// owned and attached per device like the GEMV workspace; without one (or when it is too small for
// a split) the GEMM runs whole tiles only.
constexpr int kPfMaxTiles = 65536;
constexpr size_t kPfPartBytes = size_t(512) * 256 * 256 * 4;
constexpr size_t kPfWsBytes = kPfPartBytes;
int tlx_workspace_gemm(void** ws, size_t* bytes);

// Internal entry points shared by the fused attention projections (tlx_attn.hip).  With
// launch == false they validate the arguments only.
//   IQ3_XXS: up to three matrices (packed rows or GGUF blocks) sharing the activations, one
//   launch (tlx_iq3.hip);
int tlx_iq3_segments(const void* const* w, uint16_t* const* out, const int* n, int nseg,
                     const float* gridf, const uint16_t* xh_f16, int M, int K, int layout,
                     bool launch, void* stream);
//   IQ3_XXS tiled records: the balanced GEMV (tlx_iq3s.hip); arguments already validated, x the
//   activations or (xt != 0) their tile-ordered copy; nmat 2 = gate/up pair with epi SwiGLU,
//   epi 0 = fp16 out, 2 = fp32 residual; up to 4 fp16-out matrices (nseg) share one launch
bool tlx_iq3s_stages_x(int nmat, int M, int N, int K, int nseg, bool ws_kparts);
//   ws: the GEMV workspace (required; kWsBytes, or kWsBaseBytes with ws_kparts false: no k-split)
int tlx_iq3s_launch(int nmat, int epi, int nseg, const void* const* w, const void* w1, void* const* out,
                    const int* n, const float* res, const float* gridf, const _Float16* x, int xt, int M, int K,
                    void* ws, bool ws_kparts, bool out_tileord, hipStream_t st);
//   k-quants: fmt 0 = Q6_K raw, 1 = Q6_K padded, 2 = Q4_K, 3 = Q5_K (tlx_kquant.hip).
//   one-time kernel set-up of the k-quant GEMVs (dynamic LDS limit), run by tlx_attach_workspace
int tlx_kq_setup();
int tlx_kq_gemv(int fmt, const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                int K, bool launch, void* stream);
