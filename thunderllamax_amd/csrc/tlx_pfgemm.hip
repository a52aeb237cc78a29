// IQ3_XXS prefill dequant-GEMM for gfx950 (the pf_gemm3 family with REPACK=1,
// engine/pf_gemm3.cu:313-430): C[m][n] = sum_k X[m][k] * W[n][k], X fp16 [M][K] row-major,
// W in the packed7 unit layout (engine/pack_w7.py:7-21): per 8-row group and 128-k chunk, 32
// 16-byte units, unit r*4+c = everything row r needs for sub-block c of the chunk (8 bytes of
// grid indices, the scale/sign word, d, 2 pad bytes).
// Epilogues: FFN  out16[m][n] = silu16(half(g)) * half(u)   (W = gate rows, W2 = up rows)
//            RES  out32[m][n] = res[m][n] + acc             (no half rounding, as the reference)
//            F16  out16[m][n] = half(acc)
//
// Design:
//   * workgroup tile 256 (m) x 256 (n) x 32 (k) per step; for FFN the 256 n are 128 gate + 128
//     up rows of one n-range, so a lane holds g and u of the same output element;
//   * 8 waves, two per SIMD (256 registers each: while one waits at a dependency the other
//     issues); wave (wm, wn) computes m [64wm, +64) x 128 n (FFN: 64 gate + 64 up columns of one
//     n-range) with v_mfma_f32_16x16x32_f16, 32 MFMAs per step into 128 accumulator registers
//     (measured against 4 waves of 128 x 128: +3-5% FFN, up to +10% down at M=8192);
//   * every global->LDS load is a direct (LDS-DMA) 16-byte load in which each group of 4 lanes
//     reads 64 contiguous bytes: that is what keeps the vector-memory path at full rate (a load
//     whose 4-lane groups span 4 rows runs at a quarter of it);
//   * activations: a 3-deep ring, two steps ahead; a 16-row group is stored row-major (64 B a
//     row), the 16-B piece p of row r at piece p ^ ((r >> 1) & 3), which makes the MFMA operand
//     reads (lane l: row l % 16, piece l / 16) bank-conflict-free;
//   * weights: the tile's 128-k chunk of packed7 units (32 groups x 512 contiguous bytes) is
//     staged in one burst into a 2-deep ring, four steps before its first use; each sub-block
//     is dequantized one step ahead into a double-buffered B tile in fragment order (16-B piece
//     p of row R at ((R / 16) * 64 + p * 16 + R % 16) * 16 bytes, so operand reads are
//     lane-linear), to the reference's fp16 values fp16((+-g*(2s+1)/4) * d) = fp16(db*g) (the
//     first product is exact in fp16, the second rounds once) via the sign-folded grid table
//     the GEMV uses;
//   * one barrier per step; the step's operand loads come first, then the producers of later
//     steps, which the compiler interleaves with the step's MFMAs;
//   * workgroup w runs on XCD w % 8; when M is a multiple of 2048 each XCD sweeps the n-tiles
//     of one m-tile at a time, so its L2 keeps that activation slice.
#include "tlx_common.h"

#include <algorithm>

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kWaves = 8;                 // two per SIMD: one wave's stalls are the other's issue slots
constexpr int kThreads = kWaves * TLX_WAVE;
constexpr int kMI = kBM / (16 * (kWaves / 2));   // 16-row A fragments per wave (waves: kWaves/2 along m, 2 along n)
constexpr int kLdW = 16 / kWaves;                // wave-loads per wave per 16-load burst
constexpr int kTile = kBM * kBK;          // halfs per A or B tile

enum PfEpi { PF_FFN = 0, PF_RES = 1, PF_F16 = 2 };

struct __attribute__((aligned(16))) PfLds {
  uint32_t tbl[4096 * 2];                 // sign-folded grid table, 4 fp16 per entry
  _Float16 a[3][kTile];                   // activation ring: 16-row groups, row-major, swizzled
  _Float16 b[2][kTile];                   // dequantized weights, fragment order
  u4_t w[2][kBN * 4];                     // packed7 units of one 128-k chunk: [group][r*4+c]
};

// B tile: fragment-order offset (halfs) of piece p of tile row R
__device__ __forceinline__ int pf_frag(int R, int p) { return ((R >> 4) * 64 + p * 16 + (R & 15)) * 8; }

__device__ __forceinline__ void pf_build_table(uint32_t* tbl, const float* __restrict__ gridf) {
  for (int e = threadIdx.x; e < 256 * 4; e += blockDim.x) {
    const int g = e & 255, q = e >> 8;
    const float4 v = reinterpret_cast<const float4*>(gridf)[g];
    const h2_t lo = {(_Float16)v.x, (_Float16)v.y};
    const h2_t hi = {(_Float16)v.z, (_Float16)v.w};
    const uint32_t l = __builtin_bit_cast(uint32_t, lo), h = __builtin_bit_cast(uint32_t, hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t nib = 4 * q + i;
      tbl[2 * ((nib << 8) | g)] = l ^ (((nib & 1u) << 15) | ((nib & 2u) << 30));
      tbl[2 * ((nib << 8) | g) + 1] = h ^ (((nib & 4u) << 13) | ((nib & 8u) << 28));
    }
  }
}

// Stage chunk h (128 k) of the tile's 256 weight rows into ring slot `slot`: 32 groups x 512 B,
// 16 wave-loads, wave w doing loads kLdW w .. kLdW w + kLdW - 1; load j moves tile groups 2j, 2j+1 (lane l: group
// 2j + l / 32, unit l % 32).  FFN tiles take gate groups 16nt.. for tile groups 0-15 and the up
// groups for 16-31.
__device__ __forceinline__ void pf_dma_w(PfLds& L, int slot, const u4_t* __restrict__ w1, const u4_t* __restrict__ w2,
                                         bool ffn, int nt, int nch, int h, int wave, int lane) {
#pragma unroll
  for (int jj = 0; jj < kLdW; ++jj) {
    const int j = kLdW * wave + jj;
    const int G = 2 * j + (lane >> 5);
    const u4_t* base;
    int grp;
    if (ffn) { base = G < 16 ? w1 : w2; grp = 16 * nt + (G & 15); }
    else { base = w1; grp = 32 * nt + G; }
    const u4_t* src = base + ((size_t)grp * nch + h) * 32 + (lane & 31);
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(L.w[slot] + 64 * j), 16, 0, 0);
  }
}

// Dequantize sub-block u (32 weights) of tile row r into the B tile: thread tid does row
// tid % 256, pieces c of half tid / 256 (two threads a row).
__device__ __forceinline__ void pf_dequant(const PfLds& L, _Float16* bt, int tid, int u) {
  const int r = tid & (kBN - 1), c0 = (tid >> 8) * (4 * kBN / kThreads);
  const u4_t unit = L.w[(u >> 2) & 1][4 * r + (u & 3)];
  const uint32_t sw = unit.z;
  const _Float16 ks = (_Float16)((float)(2u * (sw >> 28) + 1u) * 0.25f);
  const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)unit.w);
  const h8_t kv = {ks, ks, ks, ks, ks, ks, ks, ks};
  const h8_t dv = {d, d, d, d, d, d, d, d};
#pragma unroll
  for (int cc = 0; cc < 4 * kBN / kThreads; ++cc) {
    const int c = c0 + cc;
    const uint32_t qd = (c >> 1) ? unit.y : unit.x;
    const uint32_t qw = (c & 1) ? (qd >> 16) : (qd & 0xFFFFu);
    const uint32_t sidx = (sw >> (7 * c)) & 0x7Fu;
    const uint32_t par = __builtin_popcount(sidx) & 1u;
    const uint32_t i0 = ((sidx & 0xFu) << 8) | (qw & 0xFFu);
    const uint32_t i1 = (((sidx >> 4) | (par << 3)) << 8) | ((qw >> 8) & 0xFFu);
    const u2_t e0 = *reinterpret_cast<const u2_t*>(L.tbl + 2 * i0);
    const u2_t e1 = *reinterpret_cast<const u2_t*>(L.tbl + 2 * i1);
    h8_t v = __builtin_bit_cast(h8_t, u4_t{e0.x, e0.y, e1.x, e1.y});
    v = (v * kv) * dv;
    *reinterpret_cast<h8_t*>(bt + pf_frag(r, c)) = v;
  }
}

// Activations of k-step `step` (32 k) for the tile's 256 rows: 16 wave-loads, kLdW per wave.  Load g
// moves rows 16g..16g+15 x 64 B: lane l fills LDS piece l % 4 of row 16g + l / 4 with logical
// piece (l % 4) ^ ((l / 8) % 4), the swizzle of row l / 4.
__device__ __forceinline__ void pf_dma_a(_Float16* abuf, const _Float16* __restrict__ x, int m0, int K,
                                         int step, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < kLdW; ++j) {
    const int g = kLdW * wave + j;
    const _Float16* src = x + (size_t)(m0 + 16 * g + (lane >> 2)) * K + kBK * step + 8 * ((lane & 3) ^ ((lane >> 3) & 3));
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(abuf + 512 * g), 16, 0, 0);
  }
}

struct PfFrag {
  h8_t a[kMI], b[8];
};

// Operand loads of one step: A rows (group 8wm + i, row l % 16, piece l / 16 stored at
// (l / 16) ^ ((l % 16 >> 1) & 3)) and B rows (fragment order: lane-linear).
__device__ __forceinline__ void pf_load_frag(PfFrag& f, const _Float16* A, const _Float16* B, const int* bg,
                                             int aoff, int wm, int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) f.b[j] = *reinterpret_cast<const h8_t*>(B + 512 * bg[j] + 8 * lane);
#pragma unroll
  for (int i = 0; i < kMI; ++i) f.a[i] = *reinterpret_cast<const h8_t*>(A + 512 * (kMI * wm + i) + aoff);
}

template <int I0, int I1>
__device__ __forceinline__ void pf_mfma(f4_t (&acc)[kMI][8], const PfFrag& f) {
#pragma unroll
  for (int i = I0; i < I1; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

struct PfArgs {
  const u4_t* w1;
  const u4_t* w2;
  const _Float16* x;
  int K, nch, m0, nt;
  int tlast, hlast;   // last k-step / 128-k chunk of the segment being computed (loads clamp there)
};

// One k-step t: operand loads of step t (written before the last barrier), then the producers
// -- activations of step t+2, on every 4th step the burst staging the next chunk, the dequant
// of sub-block t+1 -- which the scheduler interleaves with the 64 MFMAs of step t, then the
// barrier.
template <bool kFfn>
__device__ __forceinline__ void pf_step(PfLds& L, f4_t (&acc)[kMI][8], const PfArgs& g, const int* bg, int aoff,
                                        int t, int ra, int wave, int wm, int lane) {
  PfFrag f;
  pf_load_frag(f, L.a[ra], L.b[t & 1], bg, aoff, wm, lane);
  // activations of step t+2 into the ring slot read at step t-1 (its reads completed before the
  // previous barrier; past the tail the source step is clamped and the slot is not read again)
  const int ra2 = ra == 0 ? 2 : ra - 1;
  pf_dma_a(L.a[ra2], g.x, g.m0, g.K, min(t + 2, g.tlast), wave, lane);
  // weights: at t = 4h-1 chunk h+1 goes into ring slot (h+1) & 1, whose chunk h-1 was last read
  // at step 4h-2; it is first read at step t+4.  Past the tail the source is clamped.
  const bool wstep = (t & 3) == 3;
  if (wstep) {
    const int h = ((t + 1) >> 2) + 1;
    pf_dma_w(L, h & 1, g.w1, g.w2, kFfn, g.nt, g.nch, min(h, g.hlast), wave, lane);
  }
  // sub-block t+1 into the other B buffer (clamped on the last step: not read again)
  pf_dequant(L, L.b[(t + 1) & 1], threadIdx.x, min(t + 1, g.tlast));
  pf_mfma<0, kMI>(acc, f);
  // step t+1's activations (issued one step earlier) and every earlier chunk burst must have
  // landed; this step's loads (4, or 8 on a burst step) stay in flight.  Then a barrier without
  // a memory fence (a fence would also wait for those).  The scheduling fences keep every MFMA
  // of the step on its side of the barrier (MFMAs touch no memory, so the asm alone would not).
  __builtin_amdgcn_sched_barrier(0);
  static_assert(kLdW == 2, "the wait counts below assume 2 A loads (+2 weight loads) per wave per step");
  if (wstep) asm volatile("s_waitcnt vmcnt(4)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(2)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Schedule: `full` workgroups own one whole tile each (the complete rounds of one workgroup per
// CU); the remaining r tiles are split into p chunk ranges (segments) whose workgroups fill the
// last round(s).  Segments store their fp32 parts; pf_fix_kernel sums each split tile's parts in
// segment order.  (Combining inside the kernel -- last arriver adds -- needs the parts visible
// across the XCDs' L2s: per-access coherent atomics or agent-scope fences on ~1 MB per tile cost
// more than the split saved.)  Tile index tau maps to (m-tile, n-tile) so that, when there are m-tiles for all 8
// XCDs, workgroup tau runs on XCD tau % 8 and each XCD sweeps the n-tiles of its m-tiles, keeping
// that activation slice in its L2.
struct PfSk {
  int full, r, p;      // whole-tile workgroups, split tiles, segments per split tile
  float* part;         // workspace: one 256 KB fp32 slot per segment
};

template <int EPI>
__device__ __forceinline__ void pf_epilogue(const f4_t (&acc)[kMI][8], const int* bg, int m0, int nt, int wm, int kq,
                                            int col, void* __restrict__ out, const float* __restrict__ res, int N) {
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * kMI * wm + 16 * i + 4 * kq + e;
      if constexpr (EPI == PF_FFN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = nt * (kBN / 2) + 16 * bg[j] + col;
          reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] = tlx_swiglu_bits(acc[i][j][e], acc[i][j + 4][e]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = nt * kBN + 16 * bg[j] + col;
          const size_t o = (size_t)m * N + n;
          if constexpr (EPI == PF_RES)
            reinterpret_cast<float*>(out)[o] = res[o] + acc[i][j][e];
          else
            reinterpret_cast<uint16_t*>(out)[o] = tlx_f2h_bits(acc[i][j][e]);
        }
      }
    }
  }
}

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void pf_gemm_kernel(
    const u4_t* __restrict__ w1, const u4_t* __restrict__ w2, const float* __restrict__ gridf,
    const _Float16* __restrict__ x, void* __restrict__ out, const float* __restrict__ res, int M, int N,
    int K, int mtiles, int ntiles, const PfSk sk) {
  __shared__ PfLds L;
  constexpr bool kFfn = EPI == PF_FFN;
  // wave index as a scalar: the per-wave DMA selection branches on SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int nch = K / 128;
  const int bx = (int)blockIdx.x;
  int tau, h0 = 0, h1 = nch, seg = -1;
  if (bx < sk.full) {
    tau = bx;
  } else {
    seg = bx - sk.full;
    const int q = seg % sk.p;
    tau = sk.full + seg / sk.p;
    h0 = q * nch / sk.p;
    h1 = (q + 1) * nch / sk.p;
  }
  int mt, nt;
  if ((mtiles & 7) == 0) {   // XCD x = tau % 8 sweeps the n-tiles of m-tiles x, x+8, ... in turn
    const int l = tau >> 3;
    mt = (tau & 7) + 8 * (l / ntiles);
    nt = l % ntiles;
  } else {
    mt = tau % mtiles;
    nt = tau / mtiles;
  }
  PfArgs g;
  g.w1 = w1; g.w2 = w2; g.x = x; g.K = K; g.nch = nch;
  g.m0 = mt * kBM; g.nt = nt;
  g.tlast = 4 * h1 - 1; g.hlast = h1 - 1;
  const int s0 = 4 * h0;

  // prologue: activation steps s0, s0+1 and weight chunks h0, h0+1 in flight; table; sub-block s0
  pf_dma_a(L.a[0], x, g.m0, K, s0, wave, lane);
  pf_dma_a(L.a[1], x, g.m0, K, min(s0 + 1, g.tlast), wave, lane);
  pf_dma_w(L, h0 & 1, w1, w2, kFfn, nt, nch, h0, wave, lane);
  pf_dma_w(L, (h0 + 1) & 1, w1, w2, kFfn, nt, nch, min(h0 + 1, g.hlast), wave, lane);
  pf_build_table(L.tbl, gridf);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
  __syncthreads();
  pf_dequant(L, L.b[s0 & 1], threadIdx.x, s0);
  __syncthreads();

  // the wave's eight 16-column n-tiles (row groups of the B tile); for FFN tiles 0..3 are gate
  // columns [64wn, +64) and tiles 4..7 the up columns of the same range
  int bg[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) bg[j] = kFfn ? (j < 4 ? 4 * wn + j : 8 + 4 * wn + (j - 4)) : 8 * wn + j;
  const int aoff = 8 * (4 * col + (kq ^ ((col >> 1) & 3)));

  f4_t acc[kMI][8];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  int ra = 0;
  for (int t = s0; t <= g.tlast; ++t) {
    pf_step<kFfn>(L, acc, g, bg, aoff, t, ra, wave, wm, lane);
    ra = ra == 2 ? 0 : ra + 1;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // drain the clamped tail loads before the block exits

  if (seg >= 0) {
    // a segment of a split tile: store the part (the register layout, 16 B a lane, coalesced);
    // pf_fix_kernel, launched next on the stream, adds the parts in order and applies the epilogue
    f4_t* mine = reinterpret_cast<f4_t*>(sk.part) + (size_t)seg * (kBM * kBN / 4);
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) mine[(i * 8 + j) * kThreads + threadIdx.x] = acc[i][j];
    return;
  }
  pf_epilogue<EPI>(acc, bg, g.m0, nt, wm, kq, col, out, res, N);
}

int pf_check(const void* w, const void* x, int M, int N, int K, int layout, int ntile) {
  if (M < kBM || (M % kBM) || N < ntile || (N % ntile) || K < 128 || (K % 128)) return TLX_E_ARG;
  if (layout != TLX_LAYOUT_PACK7) return TLX_E_ARG;
  if (!tlx_aligned(w, 16) || !tlx_aligned(x, 16)) return TLX_E_ALIGN;
  return TLX_OK;
}

// The split tiles' sums: workgroup (st, i) adds the p parts of row group i (16 rows per wave
// row) of split tile st in segment order (fixed: the result does not depend on which segment
// finished first) and applies the epilogue to them.  8 workgroups a tile keep the reads spread.
template <int EPI>
__global__ __launch_bounds__(kThreads) void pf_fix_kernel(const f4_t* __restrict__ part, void* __restrict__ out,
                                                          const float* __restrict__ res, int N, int mtiles,
                                                          int ntiles, int full, int p) {
  constexpr bool kFfn = EPI == PF_FFN;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4, wm = wave >> 1, wn = wave & 1;
  const int st = (int)blockIdx.x / kMI, i = (int)blockIdx.x % kMI, tau = full + st;
  int mt, nt;
  if ((mtiles & 7) == 0) {
    const int l = tau >> 3;
    mt = (tau & 7) + 8 * (l / ntiles);
    nt = l % ntiles;
  } else {
    mt = tau % mtiles;
    nt = tau / mtiles;
  }
  int bg[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) bg[j] = kFfn ? (j < 4 ? 4 * wn + j : 8 + 4 * wn + (j - 4)) : 8 * wn + j;
  f4_t acc[8];
  const f4_t* src = part + (size_t)st * p * (kBM * kBN / 4) + i * 8 * kThreads + threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    f4_t sum = src[j * kThreads];
    for (int q = 1; q < p; ++q) sum += src[(size_t)q * (kBM * kBN / 4) + j * kThreads];
    acc[j] = sum;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = mt * kBM + 16 * kMI * wm + 16 * i + 4 * kq + e;
    if constexpr (EPI == PF_FFN) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = nt * (kBN / 2) + 16 * bg[j] + col;
        reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] = tlx_swiglu_bits(acc[j][e], acc[j + 4][e]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = nt * kBN + 16 * bg[j] + col;
        const size_t o = (size_t)m * N + n;
        if constexpr (EPI == PF_RES)
          reinterpret_cast<float*>(out)[o] = res[o] + acc[j][e];
        else
          reinterpret_cast<uint16_t*>(out)[o] = tlx_f2h_bits(acc[j][e]);
      }
    }
  }
}

// Launch shape: whole tiles for the complete rounds of one workgroup per CU; the r tiles left
// over are split into p segments, p (<= 4) minimizing the chunks the busiest CU computes
// (ties: fewer segments), when that beats one more round of whole tiles.
template <int EPI>
int pf_launch(const u4_t* w1, const u4_t* w2, const float* gridf, const _Float16* x, void* out, const float* res,
              int M, int N, int K, int mtiles, int ntiles, hipStream_t st) {
  const int tiles = mtiles * ntiles, G0 = tlx_cu_count(), nch = K / 128;
  const int R = tiles / G0, r = tiles - R * G0;
  PfSk sk{tiles, 0, 1, nullptr};
  if (r > 0) {
    // the split needs r * p parts of 256 KB in the attached workspace; without room, whole tiles
    void* ws = nullptr;
    size_t wsb = 0;
    const int rc = tlx_workspace_gemm(&ws, &wsb);
    TLX_RET_IF(rc != TLX_OK, rc);
    const size_t cap = ws != nullptr ? std::min(wsb, kPfPartBytes) : 0;
    int best_p = 1;
    long best = (long)(R + 1) * nch;
    for (int p = 2; p <= 4; ++p) {
      if ((size_t)r * p * (kBM * kBN * 4) > cap || r > kPfMaxTiles) break;
      const long span = (long)R * nch + (long)((r * p + G0 - 1) / G0) * ((nch + p - 1) / p);
      if (span < best) { best = span; best_p = p; }
    }
    if (best_p > 1) sk = PfSk{R * G0, r, best_p, static_cast<float*>(ws)};
  }
  pf_gemm_kernel<EPI><<<sk.full + sk.r * sk.p, kThreads, 0, st>>>(w1, w2, gridf, x, out, res, M, N, K, mtiles,
                                                                    ntiles, sk);
  if (sk.p > 1) {
    const int rc = tlx_launch_status();
    TLX_RET_IF(rc != TLX_OK, rc);
    pf_fix_kernel<EPI><<<sk.r * kMI, kThreads, 0, st>>>(reinterpret_cast<const f4_t*>(sk.part), out, res, N, mtiles,
                                                      ntiles, sk.full, sk.p);
  }
  return tlx_launch_status();
}

}  // namespace

extern "C" int tlx_pfg3_ffn(const void* wg, const void* wu, const float* gridf, const uint16_t* x16,
                            uint16_t* out16, int M, int N, int K, int layout, void* stream) {
  int rc = pf_check(wg, x16, M, N, K, layout, kBN / 2);
  if (rc == TLX_OK) rc = pf_check(wu, x16, M, N, K, layout, kBN / 2);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  return pf_launch<PF_FFN>((const u4_t*)wg, (const u4_t*)wu, gridf, (const _Float16*)x16, out16, nullptr, M, N, K,
                           M / kBM, N / (kBN / 2), (hipStream_t)stream);
}

extern "C" int tlx_pfg3_iq3d(const void* w, const float* gridf, const uint16_t* x16, const float* res,
                             float* out32, int M, int N, int K, int layout, void* stream) {
  const int rc = pf_check(w, x16, M, N, K, layout, kBN);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  return pf_launch<PF_RES>((const u4_t*)w, nullptr, gridf, (const _Float16*)x16, out32, res, M, N, K, M / kBM,
                           N / kBN, (hipStream_t)stream);
}

extern "C" int tlx_pfg3_iq3o(const void* w, const float* gridf, const uint16_t* x16, uint16_t* out16,
                             int M, int N, int K, int layout, void* stream) {
  const int rc = pf_check(w, x16, M, N, K, layout, kBN);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  return pf_launch<PF_F16>((const u4_t*)w, nullptr, gridf, (const _Float16*)x16, out16, nullptr, M, N, K, M / kBM,
                           N / kBN, (hipStream_t)stream);
}
