// RMSNorm activation producers on either side of the decode GEMVs (the reference's k0n{M} /
// k0_norm and hh{M} / k3m_hh, engine/k0n11.cu:88-103, engine/hh11.cu:88-107,
// engine/gdn_block.cu:30-40,258-276):
//   norm form: xh = half((x * r) * nw)
//   add form:  hh = x + float(a), hhx = half((hh * r) * nw)
// with r = rsqrt(sum(v^2) / D + 1e-6) over the row.  One 256-thread workgroup per row, 8
// elements a thread per step; the sum of squares is reduced in a fixed order (thread partials
// -> wave butterfly -> the 4 wave sums in order), so results are deterministic.  hh is the
// reference's exactly; r comes from the hardware reciprocal square root (the reference's is
// CUDA's approximate rsqrtf), so an fp16 output can differ from the reference's by one unit
// in the last place where the float product sits at an fp16 rounding boundary.
//
// Optionally the producer also writes the tile-ordered copy the IQ3_XXS GEMVs read from M = 6
// on (xt[k / 8][col][k % 8] = out[min(col, M - 1)][k], 16 columns): fused into the producer,
// the GEMV needs no copy launch of its own.
#include "tlx_common.h"

namespace {

constexpr float kEps = 1e-6f;   // EPS_N (engine/gdn_block.cu:19)

template <bool kAdd>
__global__ __launch_bounds__(256) void rms_kernel(const float* __restrict__ x, const uint16_t* __restrict__ a,
                                                  const float* __restrict__ nw, float* __restrict__ hh,
                                                  uint16_t* __restrict__ xh, _Float16* __restrict__ xt, int M, int D) {
  __shared__ float wsum[4];
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* xr = x + (size_t)row * D;
  const uint16_t* ar = kAdd ? a + (size_t)row * D : nullptr;
  auto load8 = [&](int c, float* v) {
    const float4 p = *reinterpret_cast<const float4*>(xr + 8 * c);
    const float4 q = *reinterpret_cast<const float4*>(xr + 8 * c + 4);
    v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
    if constexpr (kAdd) {
      const h8_t h = *reinterpret_cast<const h8_t*>(ar + 8 * c);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] += (float)h[j];
    }
  };
  const int nc = D / 8;
  float ss = 0.f;
  for (int c = t; c < nc; c += 256) {
    float v[8];
    load8(c, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(v[j], v[j], ss);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  const float tot = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float r = rsqrtf(tot / (float)D + kEps);
  for (int c = t; c < nc; c += 256) {
    float v[8];
    load8(c, v);
    if constexpr (kAdd) {
      float4* ho = reinterpret_cast<float4*>(hh + (size_t)row * D + 8 * c);
      ho[0] = float4{v[0], v[1], v[2], v[3]};
      ho[1] = float4{v[4], v[5], v[6], v[7]};
    }
    const float4 w0 = *reinterpret_cast<const float4*>(nw + 8 * c);
    const float4 w1 = *reinterpret_cast<const float4*>(nw + 8 * c + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    h8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (_Float16)((v[j] * r) * wv[j]);
    *reinterpret_cast<h8_t*>(xh + (size_t)row * D + 8 * c) = o;
    if (xt != nullptr && row < 16) {
      // this row's column, and on the last row the padding columns M..15
      const int c1 = row == M - 1 ? 16 : row + 1;
      for (int col = row; col < c1; ++col) *reinterpret_cast<h8_t*>(xt + ((size_t)c * 16 + col) * 8) = o;
    }
  }
}

}  // namespace

// shared with the GEMV entry points that fuse the producer (tlx_ffn8_hh)
int tlx_rms_launch(bool add, const float* x, const uint16_t* a, const float* nw, float* hh, uint16_t* xh,
                   _Float16* xt, int M, int D, hipStream_t st) {
  if (add)
    rms_kernel<true><<<M, 256, 0, st>>>(x, a, nw, hh, xh, xt, M, D);
  else
    rms_kernel<false><<<M, 256, 0, st>>>(x, nullptr, nw, nullptr, xh, xt, M, D);
  return tlx_launch_status();
}

int tlx_rms_check(const float* x, const uint16_t* a, const float* nw, const float* hh, const uint16_t* xh, int M, int D) {
  if (M < 1 || D < 8 || (D % 8)) return TLX_E_ARG;
  if (!tlx_aligned(x, 16) || !tlx_aligned(nw, 16) || !tlx_aligned(xh, 16)) return TLX_E_ALIGN;
  if ((a != nullptr && !tlx_aligned(a, 16)) || (hh != nullptr && !tlx_aligned(hh, 16))) return TLX_E_ALIGN;
  return TLX_OK;
}

extern "C" int tlx_rms_f16(const float* x, const float* nw, uint16_t* xh, int M, int D, void* stream) {
  const int rc = tlx_rms_check(x, nullptr, nw, nullptr, xh, M, D);
  TLX_RET_IF(rc != TLX_OK, rc);
  return tlx_rms_launch(false, x, nullptr, nw, nullptr, xh, nullptr, M, D, (hipStream_t)stream);
}

extern "C" int tlx_add_rms_f16(const float* x, const uint16_t* a, const float* nw, float* hh, uint16_t* hhx, int M,
                               int D, void* stream) {
  TLX_RET_IF(a == nullptr || hh == nullptr, TLX_E_ARG);
  const int rc = tlx_rms_check(x, a, nw, hh, hhx, M, D);
  TLX_RET_IF(rc != TLX_OK, rc);
  return tlx_rms_launch(true, x, a, nw, hh, hhx, nullptr, M, D, (hipStream_t)stream);
}
