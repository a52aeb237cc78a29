// Q6_K kernels for gfx950: bit-exact dequantization (raw 210-B and padded 212-B blocks) and
// the fp32-activation GEMV (the h6k2048 contract, engine/mm/MM_P34_h6k2048.cu:8-52).
//
// GEMV design (fp32 x, fp32 y -- a VALU kernel; fp32 activations do not fit the fp16 MFMA
// operand without rounding them):
//   * a workgroup of 4 waves owns 4 consecutive rows; every wave covers all 4 rows (one per
//     16-lane quarter) and the waves split the K blocks (block b -> wave b % 4); a wave issues
//     the loads of all its blocks of a round (up to 8) before the first use, so a round costs one
//     memory round trip;
//   * x is staged in LDS once per workgroup (DMA), and beside it 32 x the sum of every 4
//     consecutive x a lane multiplies, so sum x (q - 32) = sum x q - 32 sum x needs no per-weight
//     subtraction;
//   * within a quarter, lane i owns half h = i >> 3 and the l-quad p = i & 7 of a block,
//     i.e. the 16 weights k = 128h + 32g + 4p + j (g, j = 0..3): one dword each of
//     ql[64h+4p], ql[64h+32+4p], qh[32h+4p] decodes all 16 with byte-parallel masks into
//     bytes 0..63, each converted to fp32 by one byte-select conversion and multiplied in one fma;
//   * per (lane, g) the 4-term sum is weighted by sc[g], the block's sum by d;
//   * a 16-lane butterfly then a fixed-order LDS sum over the 4 waves finish the row.
#include "tlx_common.h"

#include <algorithm>
#include <mutex>

namespace {

constexpr int kQ6Raw = 210;
constexpr int kQ6Pad = 212;

struct Q6Off {  // byte offsets of the fields inside one block
  int ql, qh, sc, d;
};

__device__ __forceinline__ Q6Off q6_offsets(int layout) {
  return layout == TLX_LAYOUT_RAW ? Q6Off{0, 128, 192, 208} : Q6Off{20, 148, 4, 2};
}

// ------------------------------------------------------------------ dequantization
// One thread per (row, block, l in 0..31, h in 0..1): 4 outputs k = 128h + 32g + l.
__global__ __launch_bounds__(256) void q6k_dequant_kernel(const uint8_t* __restrict__ w,
                                                          void* __restrict__ out, int64_t nblk,
                                                          int layout, int out_f16) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nblk * 64) return;
  const int64_t blkid = t >> 6;
  const int l = (int)(t & 31), h = (int)((t >> 5) & 1);
  const int bs = layout == TLX_LAYOUT_RAW ? kQ6Raw : kQ6Pad;
  const Q6Off o = q6_offsets(layout);
  const uint8_t* blk = w + blkid * bs;
  const float d = tlx_h2f(tlx_ldu<uint16_t>(blk + o.d));
  const int qa = blk[o.ql + 64 * h + l], qb = blk[o.ql + 64 * h + l + 32];
  const int hb = blk[o.qh + 32 * h + l];
  const int q[4] = {(qa & 0xF) | ((hb & 3) << 4), (qb & 0xF) | (((hb >> 2) & 3) << 4),
                    (qa >> 4) | (((hb >> 4) & 3) << 4), (qb >> 4) | (((hb >> 6) & 3) << 4)};
  const int64_t k0 = blkid * 256 + 128 * h + l;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float sc = (float)(int8_t)blk[o.sc + 8 * h + (l >> 4) + 2 * g];
    const float v = (d * sc) * (float)(q[g] - 32);
    if (out_f16)
      reinterpret_cast<uint16_t*>(out)[k0 + 32 * g] = tlx_f2h_bits(v);
    else
      reinterpret_cast<float*>(out)[k0 + 32 * g] = v;
  }
}

// ------------------------------------------------------------------ fp32 GEMV
constexpr int kQ6Waves = 4;     // waves per row group (they split the K blocks)
#ifndef Q6_RG
#define Q6_RG 1
#endif
constexpr int kQ6Rg = Q6_RG;    // row groups (of 4 rows) per workgroup: x is staged once for all
constexpr int kQ6MaxU = 8;      // blocks per wave per round (all their loads in flight together)
constexpr int kQ6MaxK = 15360;  // x and its group sums staged in LDS: 1.25 K floats (75 KB at most)

// Buffer resource over the workgroup's rows: per-lane field offsets stay in fixed VGPRs, the
// block offset is a wave-uniform SGPR, so the loads need no per-block vector address math.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t q6_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

template <int U>
__global__ __launch_bounds__(kQ6Rg * kQ6Waves * 64) void q6k_gemv_f32_kernel(const uint8_t* __restrict__ w,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int rows,
                                                                    int K, int layout) {
  // xs: x (K floats); xg: 32 * (sum of x over each lane's 4 consecutive k), K / 4 floats, in
  // (block, h, p, g) order so a lane reads its 4 groups of a block as one float4
  extern __shared__ __align__(16) float xs[];
  float* xg = xs + K;
  __shared__ float red[kQ6Rg][kQ6Waves][4];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rg = wave / kQ6Waves, wk = wave % kQ6Waves;
  const int quarter = lane >> 4, i = lane & 15;
  const int h = i >> 3, p = i & 7;
  const int nb = K >> 8;
  const int bs = layout == TLX_LAYOUT_RAW ? kQ6Raw : kQ6Pad;
  const Q6Off o = q6_offsets(layout);
  const int row0 = ((int)blockIdx.x * kQ6Rg + rg) * 4;
  const int rbase = min(row0, rows - 1), row = min(row0 + quarter, rows - 1);
  const uint32_t rowb = (uint32_t)bs * nb;
  const __amdgpu_buffer_rsrc_t rs = q6_rsrc(w + (size_t)rbase * rowb, 4 * rowb);
  const int vr = (row - rbase) * (int)rowb;
  const int vql = vr + o.ql + 64 * h + 4 * p, vqh = vr + o.qh + 32 * h + 4 * p;
  const int vsc = vr + o.sc + 8 * h, vd = vr + o.d;

  // x into LDS by DMA (1 KB a wave instruction), issued ahead of the first round's weight loads.
  // Written out as assembly: the compiler cannot count a loop of DMA loads, so before the first LDS
  // read of x it would drain every load in flight, the round's weights included; the explicit wait
  // before the staging barrier below is the one these loads need.
  for (int q = wave; q < nb; q += kQ6Rg * kQ6Waves) {
    const float* src = x + 256 * q + 4 * lane;
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(xs + 256 * q));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(dst) : "memory", "m0");
  }
  float acc = 0.f;
  int b0 = wk;
  do {   // every wave runs the first round (it holds the staging barriers)
    // the round's blocks b0 + 4 j (past the end: the last block, loaded and weighted 0)
    uint32_t qla[U], qlb[U], qhv[U];
    uint64_t sc8[U];
    uint16_t dh[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      __builtin_amdgcn_sched_barrier(0);   // block by block, in order: the waits below count them
      const int so = min(b0 + kQ6Waves * j, nb - 1) * bs;
      qla[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, vql, so, 0);
      qlb[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, vql + 32, so, 0);
      qhv[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, vqh, so, 0);
      sc8[j] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rs, vsc, so, 0));
      dh[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, vd, so, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (b0 == wk) {
      // this wave's DMA pieces have landed; the round's 5U weight loads issued after them need not
      // have (the barrier is written out without the fence __syncthreads carries, which would drain
      // them): each block's arithmetic then waits only for that block's loads
      constexpr int N = 5 * U;
      static_assert(N <= 63, "vmcnt range");
      __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
      asm volatile("s_barrier" ::: "memory");
      // group sums: entry e = (b, h, p, g) covers x[256 b + 128 h + 32 g + 4 p .. + 3]
      for (int e = threadIdx.x; e < (K >> 2); e += kQ6Rg * kQ6Waves * 64) {
        const int k = 256 * (e >> 6) + 128 * ((e >> 5) & 1) + 32 * (e & 3) + 4 * ((e >> 2) & 7);
        const float4 v = *reinterpret_cast<const float4*>(xs + k);
        xg[e] = 32.f * ((v.x + v.y) + (v.z + v.w));
      }
      __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));   // lgkmcnt(0)
      asm volatile("s_barrier" ::: "memory");
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int b = b0 + kQ6Waves * j;
      const int bc = min(b, nb - 1);
      const float d = b < nb ? tlx_h2f(dh[j]) : 0.f;
      const float* xb = xs + 256 * bc + 128 * h + 4 * p;
      const float4 sg = *reinterpret_cast<const float4*>(xg + 64 * bc + 32 * h + 4 * p);
      const uint64_t scs = sc8[j] >> (8 * (p >> 2));   // this lane's scales at bytes 0, 2, 4, 6
      float blk = 0.f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 xv = *reinterpret_cast<const float4*>(xb + 32 * g);
        const uint32_t ql = (g & 1) ? qlb[j] : qla[j];
        const uint32_t lo = ((g >> 1) ? (ql >> 4) : ql) & 0x0F0F0F0Fu;
        const uint32_t q = lo | (((qhv[j] >> (2 * g)) & 0x03030303u) << 4);   // 4 bytes, 0..63
        // sum x (q - 32) = sum x q - 32 sum x, the q exact in fp32
        float s = __builtin_fmaf(xv.x, (float)(q & 0xFFu), -sg[g]);
        s = __builtin_fmaf(xv.y, (float)((q >> 8) & 0xFFu), s);
        s = __builtin_fmaf(xv.z, (float)((q >> 16) & 0xFFu), s);
        s = __builtin_fmaf(xv.w, (float)(q >> 24), s);
        blk = __builtin_fmaf((float)(int8_t)(uint8_t)(scs >> (16 * g)), s, blk);
      }
      acc = __builtin_fmaf(d, blk, acc);
    }
    b0 += kQ6Waves * U;
  } while (b0 < nb);
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (i == 0) red[rg][wk][quarter] = acc;
  __syncthreads();
  if (wk == 0 && i == 0) {
    float sum = red[rg][0][quarter];
#pragma unroll
    for (int v = 1; v < kQ6Waves; ++v) sum += red[rg][v][quarter];
    const int r = row0 + quarter;
    if (r < rows) y[r] = sum;
  }
}

}  // namespace

extern "C" int tlx_q6k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int layout,
                               int out_f16, void* stream) {
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255), TLX_E_ARG);
  TLX_RET_IF(layout != TLX_LAYOUT_RAW && layout != TLX_LAYOUT_PACKED, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 2) || !tlx_aligned(out, 4), TLX_E_ALIGN);
  const int64_t nblk = rows * (kdim >> 8);
  const int64_t grid = (nblk * 64 + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  q6k_dequant_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)w, out, nblk,
                                                                        layout, out_f16);
  return tlx_launch_status();
}

extern "C" int tlx_q6k_gemv(const void* w, const float* x, float* y, int rows, int K, int layout,
                            void* stream) {
  TLX_RET_IF(rows < 1 || K < 256 || (K & 255), TLX_E_ARG);
  TLX_RET_IF(layout != TLX_LAYOUT_RAW && layout != TLX_LAYOUT_PACKED, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 4) || !tlx_aligned(x, 16), TLX_E_ALIGN);
  TLX_RET_IF(K > kQ6MaxK, TLX_E_ARG);
  const int nb = K >> 8, U = std::min(kQ6MaxU, (nb + kQ6Waves - 1) / kQ6Waves);
  const dim3 grid((rows + 4 * kQ6Rg - 1) / (4 * kQ6Rg)), block(kQ6Rg * kQ6Waves * 64);
  const size_t lds = (size_t)K * sizeof(float) * 5 / 4;   // x and its group sums
  if (lds > 65536) {   // above 64 KB of dynamic LDS (only the U = 8 form): set once per process
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
      attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&q6k_gemv_f32_kernel<8>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, kQ6MaxK * 5);
    });
    if (attr != hipSuccess) return (int)attr;
  }
  const uint8_t* wp = (const uint8_t*)w;
  hipStream_t st = (hipStream_t)stream;
  switch (U) {
    case 1: q6k_gemv_f32_kernel<1><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 2: q6k_gemv_f32_kernel<2><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 3: q6k_gemv_f32_kernel<3><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 4: q6k_gemv_f32_kernel<4><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 5: q6k_gemv_f32_kernel<5><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 6: q6k_gemv_f32_kernel<6><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    case 7: q6k_gemv_f32_kernel<7><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
    default: q6k_gemv_f32_kernel<8><<<grid, block, lds, st>>>(wp, x, y, rows, K, layout); break;
  }
  return tlx_launch_status();
}
