// The int8-activation (W4A8) prefill branch for gfx950: the activation quantizer of
// engine/pfk_q8.cu and the fused gate+up GEMM of engine/p8_w4ffn7.cu.
//
// Quantizer: per (row, 128-k chunk) s = max(absmax, 1e-6) * (1/127) in float32,
// q = rint(x / s) (half-even, IEEE division) clamped to [-127, 127], row sum of the stored
// int8s.  One wave per chunk (2 halfs a lane); max and sum are exact, so the outputs are
// bit-identical to the reference's.
//
// GEMM: IQ3_XXS weights from the packed7 units, each weight mapped to the linearized
// codebook level lut8[g][j] (1..15) with its sign, int8 activations, v_mfma_i32_16x16x32_i8.
// Each 32-k MFMA step is one IQ3 sub-block, whose scale is sdb = d * ((sw >> 28) + 0.5) *
// 0.5 * 4.0507 = (d * 4.0507 / 4) * (2s + 1): the odd integer 2s + 1 is applied to the
// step's int32 partial in the integer domain (|partial| <= 32 * 127 * 15, so the sum over a
// 128-k chunk stays below 2^24 and converts to float exactly), and the float factor once
// per chunk: g += (sx[m][chunk] * d'[n]) * float(acc).  Same values as the reference's
// per-step float rescale (engine/p8_w4ffn7.cu:123-167), regrouped.
//   * workgroup tile 128 activation rows x 64 output columns (64 gate + 64 up weight rows);
//     4 waves, wave (wm, wn) computes rows 64wm.. x columns 32wn.. of gate and up
//     (16 MFMA tiles of 16 x 16); two workgroups per CU (75.8 KB LDS each);
//   * per 128-k chunk: the chunk's activations (16 KB) and activation scales are DMA'd into
//     LDS a chunk ahead, its packed7 units (8 KB) once the previous chunk's are decoded; the
//     workgroup decodes the units once, one sign-folded table lookup per 4 weights, into an
//     int8 B tile in MFMA fragment order (+ per row the 4 step factors and d'), then each
//     wave runs 4 steps x 16 MFMAs;
//   * activations are stored row-major with the 16-B pieces of row m XOR-swizzled by m & 7,
//     so the 8-B fragment reads of a phase spread over the banks.
#include "tlx_common.h"

namespace {

constexpr int kQch = 128;             // activation quantization chunk = GEMM k-chunk
constexpr float kDelta = 4.0507f;     // codebook step (engine/p8_w4ffn7.cu:46)

// ------------------------------------------------------------------ activation quantizer
__global__ __launch_bounds__(256) void p8_quant_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ xq,
                                                       float* __restrict__ sx, int32_t* __restrict__ rs, int chunks,
                                                       int nch, int K) {
  const int w = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (w >= chunks) return;
  const int m = w / nch, c = w - m * nch;
  const size_t base = (size_t)m * K + (size_t)c * kQch + 2 * lane;
  const uint32_t hv = *reinterpret_cast<const uint32_t*>(x + base);
  const float f0 = tlx_h2f((uint16_t)(hv & 0xFFFFu)), f1 = tlx_h2f((uint16_t)(hv >> 16));
  float am = fmaxf(fabsf(f0), fabsf(f1));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
  const float s = fmaxf(am, 1e-6f) * (1.0f / 127.0f);
  const int q0 = max(-127, min(127, (int)rintf(f0 / s)));
  const int q1 = max(-127, min(127, (int)rintf(f1 / s)));
  *reinterpret_cast<uint16_t*>(xq + base) = (uint16_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8));
  int rsum = q0 + q1;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) rsum += __shfl_xor(rsum, o, 64);
  if (lane == 0) {
    sx[(size_t)m * nch + c] = s;
    rs[(size_t)m * nch + c] = rsum;
  }
}

// ------------------------------------------------------------------ W4A8 FFN GEMM
constexpr int kBM = 128;    // activation rows per tile
constexpr int kBN = 64;     // output columns per tile
constexpr int kThreads = 256;

struct __attribute__((aligned(16))) P8Lds {
  uint8_t a[2][kBM * kQch];   // int8 activations of one chunk, row m at 128m, pieces swizzled
  u4_t w[16 * 32];            // packed7 units of one chunk: 8 gate groups, then 8 up groups
  u2_t b[8][4][64];           // decoded weights: [16-row n-tile][32-k step][lane] (8 int8)
  uint32_t lut[16 * 256];     // (sign nibble << 8 | grid word) -> 4 signed levels
  uint32_t fac[kBM];          // per tile row: 2s + 1 of the chunk's 4 sub-blocks, a byte each
  float dp[kBM];              // per tile row: d * 4.0507 / 4
  float sxs[2][kBM];          // the chunk's activation scales of the tile's rows
};

// Sign-folded level table: entry (sg << 8 | g) = the 4 level bytes of grid word g (0..127),
// byte i negated where bit i of sg is set (byte-wise two's complement, no carries between
// bytes).  Built once per workgroup: thread t fills entries t, t + 256, ...
__device__ __forceinline__ void p8_build_table(uint32_t* tbl, const uint32_t* __restrict__ lut8, int t) {
  const uint32_t l = lut8[t];
#pragma unroll
  for (uint32_t sg = 0; sg < 16; ++sg) {
    const uint32_t m = ((sg * 0x00204081u) & 0x01010101u) * 0xFFu;   // byte i = 0xFF if bit i
    const uint32_t a = l ^ m;
    tbl[(sg << 8) | (uint32_t)t] = ((a & 0x7F7F7F7Fu) + (m & 0x01010101u)) ^ (a & 0x80808080u);
  }
}

struct P8Args {
  const u4_t* w1;
  const u4_t* w2;
  const int8_t* xq;
  const float* sx;
  int K, nch, m0, nt;
};

// DMA of chunk c into buffer buf: activations (16 wave-loads of 8 rows x 128 B; lane l moves
// 16-B piece (l & 7) ^ (row & 7) of row l >> 3 into slot l & 7), units (8 wave-loads of two
// groups), scales (2 wave-loads of 64 rows, 4 B a lane)
__device__ __forceinline__ void p8_dma(P8Lds& L, const P8Args& g, int c, int buf, int wave, int lane) {
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int j = 4 * wave + jj, m = 8 * j + (lane >> 3), p = (lane & 7) ^ (m & 7);
    const int8_t* src = g.xq + (size_t)(g.m0 + m) * g.K + (size_t)kQch * c + 16 * p;
    __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(L.a[buf] + 1024 * j),
                                     16, 0, 0);
  }
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int j = 2 * wave + jj, G = 2 * j + (lane >> 5);
    const u4_t* base = G < 8 ? g.w1 : g.w2;
    const u4_t* src = base + ((size_t)(8 * g.nt + (G & 7)) * g.nch + c) * 32 + (lane & 31);
    __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(L.w + 64 * j), 16, 0,
                                     0);
  }
  if (wave < 2) {
    const float* src = g.sx + (size_t)(g.m0 + 64 * wave + lane) * g.nch + c;
    __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(L.sxs[buf] + 64 * wave),
                                     4, 0, 0);
  }
}

// Decode the chunk's 512 units (2 per thread): unit u = (group G, row r, sub-block c) of tile
// row R = 8 (G & 7) + r (+ 64 for the up groups) -> B tile [R / 16][c][16 cc + R % 16] for
// lane-chunk cc (8 weights: grid words q & 0xFF, q >> 8; signs sidx bits 0-3, 4-6 + parity)
__device__ __forceinline__ void p8_decode(P8Lds& L, int t) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = t + kThreads * i, G = u >> 5, r = (u >> 2) & 7, c = u & 3;
    const int R = 8 * (G & 7) + r + (G >= 8 ? 64 : 0);
    const u4_t unit = L.w[u];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const uint32_t qv = ((cc < 2 ? unit.x : unit.y) >> (16 * (cc & 1))) & 0xFFFFu;
      const uint32_t sidx = (unit.z >> (7 * cc)) & 0x7Fu;
      const uint32_t par = __builtin_popcount(sidx) & 1u;
      const uint32_t v0 = L.lut[((sidx & 0xFu) << 8) | (qv & 0xFFu)];
      const uint32_t v1 = L.lut[(((sidx >> 4) | (par << 3)) << 8) | (qv >> 8)];
      L.b[R >> 4][c][16 * cc + (R & 15)] = u2_t{v0, v1};
    }
    reinterpret_cast<uint8_t*>(L.fac)[4 * R + c] = (uint8_t)(2u * (unit.z >> 28) + 1u);
    if (c == 0) L.dp[R] = tlx_h2f((uint16_t)(unit.w & 0xFFFFu)) * 0.25f * kDelta;
  }
}

__global__ __launch_bounds__(kThreads, 2) void p8w4_ffn_kernel(const u4_t* __restrict__ w1, const u4_t* __restrict__ w2,
                                                               const uint32_t* __restrict__ lut8,
                                                               const int8_t* __restrict__ xq,
                                                               const float* __restrict__ sx,
                                                               uint16_t* __restrict__ out, int M, int N, int K,
                                                               int mtiles, int ntiles) {
  __shared__ P8Lds L;
  const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const int col = lane & 15, kq = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  int mt, nt;
  if ((ntiles & 7) == 0) {   // XCD x = id % 8 sweeps the m-tiles of n-tiles x, x + 8, ...
    const int l = (int)blockIdx.x >> 3;
    nt = ((int)blockIdx.x & 7) + 8 * (l / mtiles);
    mt = l % mtiles;
  } else {
    mt = (int)blockIdx.x % mtiles;
    nt = (int)blockIdx.x / mtiles;
  }
  P8Args g;
  g.w1 = w1; g.w2 = w2; g.xq = xq; g.sx = sx; g.K = K;
  g.nch = K / kQch; g.m0 = mt * kBM; g.nt = nt;

  p8_build_table(L.lut, lut8, t);
  p8_dma(L, g, 0, 0, wave, lane);

  // the wave's n-tiles: gate 2wn, 2wn + 1, then the matching up tiles
  int jt[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) jt[q] = (q < 2 ? 0 : 4) + 2 * wn + (q & 1);

  f4_t facc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) facc[i][q] = f4_t{0.f, 0.f, 0.f, 0.f};

  typedef int i4_t __attribute__((ext_vector_type(4)));
  const i4_t zero = {0, 0, 0, 0};
  for (int c = 0; c < g.nch; ++c) {
    const int buf = c & 1;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this chunk's DMA
    __syncthreads();
    p8_decode(L, t);
    __syncthreads();
    if (c + 1 < g.nch) p8_dma(L, g, c + 1, buf ^ 1, wave, lane);

    // per (m-tile, n-tile): its 4 sub-block steps back to back, so the int32 partial is
    // transient: acc = sum_s (2s + 1)_s * mfma_s (v_mad_i32_i24: every MFMA partial is
    // below 2^23), then one float update per chunk
    uint32_t f[4];
    long B[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[q] = L.fac[16 * jt[q] + col];
#pragma unroll
      for (int s = 0; s < 4; ++s) B[q][s] = __builtin_bit_cast(long, L.b[jt[q]][s][lane]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 64 * wm + 16 * i + col;
      long A[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int slot = (2 * s + (kq >> 1)) ^ (row & 7);
        A[s] = *reinterpret_cast<const long*>(L.a[buf] + 128 * row + 16 * slot + 8 * (kq & 1));
      }
      const f4_t sv = *reinterpret_cast<const f4_t*>(&L.sxs[buf][64 * wm + 16 * i + 4 * kq]);
      // step s's four MFMAs (one per n-tile) are issued while step s - 1's results are
      // rescaled: a result is read four MFMAs after it was issued, with no wait states
      i4_t acc[4], pr[2][4];
#pragma unroll
      for (int s = 0; s <= 4; ++s) {
        if (s < 4) {
#pragma unroll
          for (int q = 0; q < 4; ++q) pr[s & 1][q] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[s], B[q][s], zero, 0, 0, 0);
        }
        if (s > 0) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int fs = (int)((f[q] >> (8 * (s - 1))) & 0xFFu);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int v = fs * ((pr[(s - 1) & 1][q][r] << 8) >> 8);   // 24-bit operands: v_mad_i32_i24
              acc[q][r] = s == 1 ? v : acc[q][r] + v;
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float dq = L.dp[16 * jt[q] + col];
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[i][q][r] = __builtin_fmaf(sv[r] * dq, (float)acc[q][r], facc[i][q][r]);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = g.m0 + 64 * wm + 16 * i + 4 * kq + r;
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        const int n = kBN * nt + 16 * (2 * wn + qq) + col;
        out[(size_t)m * N + n] = tlx_swiglu_bits(facc[i][qq][r], facc[i][qq + 2][r]);
      }
    }
}

}  // namespace

extern "C" int tlx_p8_quant(const uint16_t* x16, int8_t* xq, float* sx, int32_t* rs, int M, int K, void* stream) {
  TLX_RET_IF(M < 1 || K < kQch || (K % kQch), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(x16, 4) || !tlx_aligned(xq, 2) || !tlx_aligned(sx, 4) || !tlx_aligned(rs, 4), TLX_E_ALIGN);
  const int nch = K / kQch;
  const long chunks = (long)M * nch;
  TLX_RET_IF(chunks > 0x7FFFFFFFL - 4, TLX_E_ARG);
  p8_quant_kernel<<<(unsigned)((chunks + 3) / 4), 256, 0, (hipStream_t)stream>>>(x16, xq, sx, rs, (int)chunks, nch, K);
  return tlx_launch_status();
}

extern "C" int tlx_p8w4_ffn(const void* w1u, const void* w2u, const int8_t* lut8, const int8_t* xq, const float* sx,
                            uint16_t* out16, int M, int N, int K, int layout, void* stream) {
  TLX_RET_IF(layout != TLX_LAYOUT_PACK7, TLX_E_ARG);
  TLX_RET_IF(M < kBM || (M % kBM) || N < kBN || (N % kBN) || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w1u, 16) || !tlx_aligned(w2u, 16) || !tlx_aligned(xq, 16) || !tlx_aligned(sx, 4) ||
                 !tlx_aligned(lut8, 4) || !tlx_aligned(out16, 2),
             TLX_E_ALIGN);
  const int mtiles = M / kBM, ntiles = N / kBN;
  p8w4_ffn_kernel<<<mtiles * ntiles, kThreads, 0, (hipStream_t)stream>>>(
      (const u4_t*)w1u, (const u4_t*)w2u, (const uint32_t*)lut8, xq, sx, out16, M, N, K, mtiles, ntiles);
  return tlx_launch_status();
}
