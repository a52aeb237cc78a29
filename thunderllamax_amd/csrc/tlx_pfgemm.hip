// IQ3_XXS prefill dequant-GEMM for gfx950 (the pf_gemm3 family, engine/pf_gemm3.cu:313-430):
//   C[m][n] = sum_k X[m][k] * W[n][k],  X fp16 [M][K] row-major, W packed IQ3_XXS rows.
// Epilogues: FFN  out16[m][n] = silu16(half(g)) * half(u)   (W = gate rows, W2 = up rows)
//            RES  out32[m][n] = res[m][n] + acc             (no half rounding, as the reference)
//            F16  out16[m][n] = half(acc)
//
// Design:
//   * workgroup tile 256 (m) x 256 (n): for FFN the 256 n are 128 gate + 128 up rows of one
//     n-range, so a lane holds g and u of the same output element;
//   * 4 waves (one per SIMD, so each owns 512 registers), wave (wm, wn) computes m [128wm, +128)
//     x 128 n (FFN: 64 gate + 64 up columns of one n-range) with v_mfma_f32_16x16x32_f16,
//     64 MFMAs per K-step; K-step = 32 = one IQ3 sub-block;
//   * activations stream into a 3-deep LDS ring with direct global->LDS 16-B loads issued two
//     steps ahead; each wave waits only for the step it needs (vmcnt), so later loads stay in
//     flight; the next 256-k block of weights is prefetched into registers;
//   * weights are dequantized to the reference's fp16 values, fp16((+-g*(2s+1)/4) * d) =
//     fp16(db*g) (the first product is exact in fp16, the second rounds once), into a
//     double-buffered LDS tile [256 n][32 k]; the sign-folded grid table is the one the GEMV
//     uses;
//   * workgroup w runs on XCD w % 8; the m-tile is taken from w % 8 so every XCD reuses one
//     activation slice from its own L2.
#include "tlx_common.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * TLX_WAVE;

enum PfEpi { PF_FFN = 0, PF_RES = 1, PF_F16 = 2 };

struct __attribute__((aligned(16))) PfLds {
  uint32_t tbl[4096 * 2];                 // sign-folded grid table, 4 fp16 per entry
  _Float16 a[3][kBM * kBK];               // activation ring, [m][32 k]
  _Float16 b[2][kBN * kBK];               // dequantized weights, [n][32 k]
  uint8_t wq[kBN * 64];                   // raw weight block being staged: grid indices
  uint8_t ws[kBN * 32];                   //   scale/sign words
  uint32_t wd[kBN];                       //   the aligned d pair holding d (blocks 2i, 2i+1)
};

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

// One weight row's 256-k block: 64 B of grid indices, the 8 scale/sign words, d.
struct PfW {
  uint32_t q[16];
  u4_t s[2];
  uint32_t d;
};

// Stage block b of the tile's 256 weight rows into LDS with direct loads: 1024 16-B index
// pieces, 512 16-B scale pieces and 256 dwords holding d = 28 wave-loads, 7 per wave.  The d
// words are the dword-aligned pairs (block b & ~1, b | 1) -- rows are dword-aligned since NB
// is even -- because a sub-dword direct load still spaces lanes 4 bytes apart in LDS.
__device__ __forceinline__ void pf_dma_w(PfLds& L, const uint8_t* __restrict__ w1, const uint8_t* __restrict__ w2,
                                         bool ffn, int nt, size_t rowb, int nb, int b, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 7; ++j) {
    const int ins = 7 * wave + j;              // 0..27; 0..15 qs, 16..23 sw, 24..27 d
    int row, off, size;
    __attribute__((address_space(3))) void* dst;
    if (ins < 16) {
      row = 16 * ins + (lane >> 2); off = 64 * b + 16 * (lane & 3); size = 16;
      dst = (__attribute__((address_space(3))) void*)(L.wq + 1024 * ins);
    } else if (ins < 24) {
      row = 32 * (ins - 16) + (lane >> 1); off = 64 * nb + 32 * b + 16 * (lane & 1); size = 16;
      dst = (__attribute__((address_space(3))) void*)(L.ws + 1024 * (ins - 16));
    } else {
      row = 64 * (ins - 24) + lane; off = 96 * nb + 4 * (b >> 1); size = 4;
      dst = (__attribute__((address_space(3))) void*)(L.wd + 64 * (ins - 24));
    }
    const uint8_t* src;
    if (ffn) src = (row < 128 ? w1 : w2) + (size_t)(nt * 128 + (row & 127)) * rowb + off;
    else src = w1 + (size_t)(nt * kBN + row) * rowb + off;
    if (size == 16) __builtin_amdgcn_global_load_lds((const void*)src, dst, 16, 0, 0);
    else __builtin_amdgcn_global_load_lds((const void*)src, dst, 4, 0, 0);
  }
}

__device__ __forceinline__ void pf_read_w(PfW& w, const PfLds& L, int r, int b) {
  const u4_t* q = reinterpret_cast<const u4_t*>(L.wq + 64 * r);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u4_t v = q[i];
    w.q[4 * i] = v.x; w.q[4 * i + 1] = v.y; w.q[4 * i + 2] = v.z; w.q[4 * i + 3] = v.w;
  }
  w.s[0] = *reinterpret_cast<const u4_t*>(L.ws + 32 * r);
  w.s[1] = *reinterpret_cast<const u4_t*>(L.ws + 32 * r + 16);
  w.d = L.wd[r] >> (16 * (b & 1));
}

// Dequantize sub-block S (32 weights) of the thread's row into dst (32 fp16).
template <int S>
__device__ __forceinline__ void pf_dequant(const PfW& w, const uint32_t* tbl, _Float16* dst) {
  const uint32_t sw = w.s[S >> 2][S & 3];
  const _Float16 ks = (_Float16)((float)(2u * (sw >> 28) + 1u) * 0.25f);
  const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)w.d);
  const h8_t kv = {ks, ks, ks, ks, ks, ks, ks, ks};
  const h8_t dv = {d, d, d, d, d, d, d, d};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint32_t qd = w.q[2 * S + (c >> 1)];
    const uint32_t qw = (c & 1) ? (qd >> 16) : (qd & 0xFFFFu);
    const uint32_t sidx = (sw >> (7 * c)) & 0x7Fu;
    const uint32_t par = __builtin_popcount(sidx) & 1u;
    const uint32_t i0 = ((sidx & 0xFu) << 8) | (qw & 0xFFu);
    const uint32_t i1 = (((sidx >> 4) | (par << 3)) << 8) | ((qw >> 8) & 0xFFu);
    const u2_t e0 = *reinterpret_cast<const u2_t*>(tbl + 2 * i0);
    const u2_t e1 = *reinterpret_cast<const u2_t*>(tbl + 2 * i1);
    h8_t v = __builtin_bit_cast(h8_t, u4_t{e0.x, e0.y, e1.x, e1.y});
    v = (v * kv) * dv;
    *reinterpret_cast<h8_t*>(dst + 8 * c) = v;
  }
}

__device__ __forceinline__ void pf_dma_a(_Float16* abuf, const _Float16* __restrict__ x, int m0, int K,
                                         int step, int wave, int lane) {
  // 256 rows x 64 B = 16 x 1 KB; wave w moves rows [64w, 64w+64)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int blk = 4 * wave + j;
    const int row = 16 * blk + (lane >> 2);
    const _Float16* src = x + (size_t)(m0 + row) * K + kBK * step + 8 * (lane & 3);
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(abuf + 512 * blk), 16, 0, 0);
  }
}

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void pf_gemm_kernel(
    const uint8_t* __restrict__ w1, const uint8_t* __restrict__ w2, const float* __restrict__ gridf,
    const _Float16* __restrict__ x, void* __restrict__ out, const float* __restrict__ res, int M, int N,
    int K, int mtiles) {
  __shared__ PfLds L;
  // wave index as a scalar: the per-wave DMA selection below then branches on SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int mt = (int)blockIdx.x % mtiles, nt = (int)blockIdx.x / mtiles;
  const int m0 = mt * kBM;
  const int nb = K >> 8, steps = K / kBK;
  const size_t rowb = (size_t)98 * nb;

  // dequant role of this thread: B-tile row r
  const int r = threadIdx.x;
  constexpr bool kFfn = EPI == PF_FFN;

  // prologue: activation steps 0 and 1 in flight, weight block 0 staged, then block 1
  pf_dma_a(L.a[0], x, m0, K, 0, wave, lane);
  pf_dma_a(L.a[1], x, m0, K, min(1, steps - 1), wave, lane);
  pf_dma_w(L, w1, w2, kFfn, nt, rowb, nb, 0, wave, lane);
  pf_build_table(L.tbl, gridf);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
  __syncthreads();
  PfW wc;
  pf_read_w(wc, L, r, 0);
  pf_dequant<0>(wc, L.tbl, L.b[0] + r * kBK);
  __syncthreads();                      // staging area read by everyone
  pf_dma_w(L, w1, w2, kFfn, nt, rowb, nb, min(1, nb - 1), wave, lane);

  f4_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // the wave's eight 16-column n-tiles inside the 256-row B tile; for FFN tiles 0..3 are gate
  // columns [64wn, +64) and tiles 4..7 the up columns of the same range
  int ncol[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ncol[j] = kFfn ? (j < 4 ? 64 * wn + 16 * j : 128 + 64 * wn + 16 * (j - 4)) : 128 * wn + 16 * j;

  for (int b = 0; b < nb; ++b) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int t = 8 * b + s;
      const _Float16* A = L.a[t % 3];
      const _Float16* B = L.b[s & 1];
      // produce: activations two steps ahead (clamped at the end: the extra tiles land in ring
      // slots that are never read); weights of the next step; at s == 0 the weight block
      // b+1 starts staging (the staging area was last read before the previous barrier)
      pf_dma_a(L.a[(t + 2) % 3], x, m0, K, min(t + 2, steps - 1), wave, lane);
      if (s == 0 && b > 0) pf_dma_w(L, w1, w2, kFfn, nt, rowb, nb, min(b + 1, nb - 1), wave, lane);
      switch (s) {
        case 0: pf_dequant<1>(wc, L.tbl, L.b[1] + r * kBK); break;
        case 1: pf_dequant<2>(wc, L.tbl, L.b[0] + r * kBK); break;
        case 2: pf_dequant<3>(wc, L.tbl, L.b[1] + r * kBK); break;
        case 3: pf_dequant<4>(wc, L.tbl, L.b[0] + r * kBK); break;
        case 4: pf_dequant<5>(wc, L.tbl, L.b[1] + r * kBK); break;
        case 5: pf_dequant<6>(wc, L.tbl, L.b[0] + r * kBK); break;
        case 6: pf_dequant<7>(wc, L.tbl, L.b[1] + r * kBK); break;
        default:
          if (b + 1 < nb) {   // block b+1 has been staged since step 2 of this block
            pf_read_w(wc, L, r, b + 1);
            pf_dequant<0>(wc, L.tbl, L.b[0] + r * kBK);
          }
      }
      // consume step t
      h8_t bf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) bf[j] = *reinterpret_cast<const h8_t*>(B + (ncol[j] + col) * kBK + 8 * kq);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const h8_t af = *reinterpret_cast<const h8_t*>(A + (128 * wm + 16 * i + col) * kBK + 8 * kq);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
      // step t+1's activations (issued one step earlier) must have landed; the loads issued in
      // this step (4 activation DMAs, plus 7 weight DMAs at s == 0 of blocks b > 0) stay in
      // flight.  Then a barrier without a memory fence (a fence would also wait for those).
      if (s == 0 && b > 0) asm volatile("s_waitcnt vmcnt(11)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(4)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // drain the clamped tail loads before the block exits

  // epilogue: lane (col, kq) of m-tile i, n-tile j holds rows 4kq + e, column col
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 128 * wm + 16 * i + 4 * kq + e;
      if constexpr (EPI == PF_FFN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = nt * (kBN / 2) + ncol[j] + col;
          reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] = tlx_swiglu_bits(acc[i][j][e], acc[i][j + 4][e]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = nt * kBN + ncol[j] + col;
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

int pf_check(const void* w, const void* x, int M, int N, int K, int layout, int ntile) {
  if (M < kBM || (M % kBM) || N < ntile || (N % ntile) || K < 256 || (K & 255)) return TLX_E_ARG;
  if (layout != TLX_LAYOUT_PACKED) return TLX_E_ARG;
  if (((K >> 8) & 1) || !tlx_aligned(w, 16) || !tlx_aligned(x, 16)) return TLX_E_ALIGN;
  return TLX_OK;
}

}  // namespace

extern "C" int tlx_pfg3_ffn(const void* wg, const void* wu, const float* gridf, const uint16_t* x16,
                            uint16_t* out16, int M, int N, int K, int layout, void* stream) {
  int rc = pf_check(wg, x16, M, N, K, layout, kBN / 2);
  if (rc == TLX_OK) rc = pf_check(wu, x16, M, N, K, layout, kBN / 2);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  const int mtiles = M / kBM, ntiles = N / (kBN / 2);
  pf_gemm_kernel<PF_FFN><<<mtiles * ntiles, kThreads, 0, (hipStream_t)stream>>>(
      (const uint8_t*)wg, (const uint8_t*)wu, gridf, (const _Float16*)x16, out16, nullptr, M, N, K, mtiles);
  return tlx_launch_status();
}

extern "C" int tlx_pfg3_iq3d(const void* w, const float* gridf, const uint16_t* x16, const float* res,
                             float* out32, int M, int N, int K, int layout, void* stream) {
  const int rc = pf_check(w, x16, M, N, K, layout, kBN);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  const int mtiles = M / kBM, ntiles = N / kBN;
  pf_gemm_kernel<PF_RES><<<mtiles * ntiles, kThreads, 0, (hipStream_t)stream>>>(
      (const uint8_t*)w, nullptr, gridf, (const _Float16*)x16, out32, res, M, N, K, mtiles);
  return tlx_launch_status();
}

extern "C" int tlx_pfg3_iq3o(const void* w, const float* gridf, const uint16_t* x16, uint16_t* out16,
                             int M, int N, int K, int layout, void* stream) {
  const int rc = pf_check(w, x16, M, N, K, layout, kBN);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  const int mtiles = M / kBM, ntiles = N / kBN;
  pf_gemm_kernel<PF_F16><<<mtiles * ntiles, kThreads, 0, (hipStream_t)stream>>>(
      (const uint8_t*)w, nullptr, gridf, (const _Float16*)x16, out16, nullptr, M, N, K, mtiles);
  return tlx_launch_status();
}
