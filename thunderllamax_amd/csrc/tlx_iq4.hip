// IQ4_XS kernels for gfx950: bit-exact dequantization of raw 136-byte blocks
// [d f16][scales_h u16][scales_l u8[4]][qs u8[128]] (llama.cpp dequantize_row_iq4_xs, as
// restated in engine/mm/MM_P0_d2_repack.py:78-93).
#include "tlx_common.h"

namespace {

constexpr int kIq4Bytes = 136;

// One thread per (block, group ib, j in 0..15): outputs 32ib+j (low nibble) and 32ib+16+j.
__global__ __launch_bounds__(256) void iq4_dequant_kernel(const uint8_t* __restrict__ w,
                                                          const float* __restrict__ kv,
                                                          float* __restrict__ out, int64_t nblk) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nblk * 128) return;
  const int64_t blkid = t >> 7;
  const int ib = (int)((t >> 4) & 7), j = (int)(t & 15);
  const uint8_t* blk = w + blkid * kIq4Bytes;
  const float d = tlx_h2f(tlx_ldu<uint16_t>(blk));
  const uint32_t sh = tlx_ldu<uint16_t>(blk + 2);
  const uint32_t sl = blk[4 + (ib >> 1)];
  const int ls = (int)(((sl >> (4 * (ib & 1))) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4));
  const float dl = d * (float)(ls - 32);
  const uint32_t qb = blk[8 + 16 * ib + j];
  float* o = out + blkid * 256 + 32 * ib + j;
  o[0] = dl * kv[qb & 0xFu];
  o[16] = dl * kv[qb >> 4];
}

}  // namespace

extern "C" int tlx_iq4xs_dequant(const void* w, const float* iq4nl, float* out, int64_t rows,
                                 int64_t kdim, void* stream) {
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 2) || !tlx_aligned(out, 4), TLX_E_ALIGN);
  const int64_t nblk = rows * (kdim >> 8);
  const int64_t grid = (nblk * 128 + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  iq4_dequant_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)w, iq4nl, out,
                                                                       nblk);
  return tlx_launch_status();
}
