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
//
// The merged form (pf_gemm3m, engine/pf_gemm3m.cu:1-16,229): up to three weight matrices of
// different formats that share the activations, one launch, plain fp16 epilogue; a workgroup's
// n-tile selects its segment.  Besides packed7 IQ3_XXS a segment may be GGUF Q4_K (144-B
// blocks), GGUF Q5_K (176-B blocks) or Q6_K in the padded 212-B blocks of pack_w1c
// (engine/pack_w1c.py:33-45), the classes the reference's merged twins mix (attention q/k/v:
// engine/build_p7b.py:64-77; GDN qkv + gate: :58-63).  For those, thread (row tid / 2, half
// tid % 2) decodes its 16 weights of sub-block t + 1 during step t into the other B tile, from
// 16-B pieces each wave staged in LDS by DMA at step t - 1 (aligned covers of the fields its rows
// need; the ring takes the place of the IQ3_XXS table): each weight becomes the reference's operand
// fp16 of the GGUF value computed in fp32 -- Q4_K / Q5_K fp16((d*sc)*q - dmin*m) (one fma:
// (d*sc)*q is exact in fp32), Q6_K fp16((d*sc)*(q - 32)) -- the dequantizers of
// engine/pf_gemm3m.cu:84-136 (dq_c2 / dq_c3 / dq_c4).
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
  _Float16 a[3][kTile];                   // activation ring: 16-row groups, row-major, swizzled
  _Float16 b[2][kTile];                   // dequantized weights, fragment order
  union {
    struct {
      uint32_t tbl[4096 * 2];             // IQ3_XXS: sign-folded grid table, 4 fp16 per entry
      u4_t w[2][kBN * 4];                 // IQ3_XXS: packed7 units of one 128-k chunk: [group][r*4+c]
    };
    u4_t kq[2][kWaves][5][TLX_WAVE];      // k-quants: two stages of each wave's 16-B weight pieces
  };
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
  const uint8_t* wkq;    // k-quant formats: the tile's first weight row
  uint32_t rowb;         // k-quant formats: bytes per weight row
};

// Weight formats of a GEMM segment: packed7 IQ3_XXS units, GGUF Q4_K / Q5_K blocks, Q6_K padded
// 212-B blocks ([pad 2][d 2][sc 16][ql 128][qh 64]).
enum PfFmt { PF_IQ3 = 0, PF_Q4K = 1, PF_Q5K = 2, PF_Q6P = 3 };

__host__ __device__ constexpr int pf_block_bytes(int f) {
  return f == PF_Q4K ? 144 : f == PF_Q5K ? 176 : f == PF_Q6P ? 212 : 128;
}

// K-quant weights reach the B tile through LDS, a half-block (128 weights: sub-blocks 4h'..4h'+3,
// one 128-k chunk) at a time: on the step before a half-block starts each wave DMAs (16-B LDS-DMA
// loads, one 1 KB slab per instruction) the aligned 16-B pieces that cover what its 32 tile rows
// need for it into one stage of a two-stage ring; on each step the thread pair of each row decodes
// the next sub-block from there.  Pieces per row (P): Q4_K the 16-B header and the half-block's
// 64 qs bytes (5); Q5_K the header, the 32 qh bytes and the 64 qs bytes (7); Q6_K (4-B aligned
// fields) the 80-B cover of its 64 ql bytes, the 48-B cover of its 32 qh bytes and the 32-B cover
// of d and the scales (10).  Staged per sub-block instead, the header (and Q5_K's qh bytes, Q6_K's
// shared ql / qh bytes) moved 2-4 times per half-block.  Piece p of a wave's half-block goes to
// slab byte 16 p (row p / P, piece p % P); lanes past 32 P re-load the last piece.
template <int FMT> constexpr int pf_kq_pieces() { return FMT == PF_Q4K ? 5 : FMT == PF_Q5K ? 7 : 10; }
template <int FMT> constexpr int pf_kq_dmas() { return (32 * pf_kq_pieces<FMT>() + TLX_WAVE - 1) / TLX_WAVE; }

// Byte offset from the row start of piece q (0 .. P-1) of sub-block j.
template <int FMT>
__device__ __forceinline__ uint32_t pf_kq_piece_off(int j, int q) {
  const uint32_t b = (uint32_t)(j >> 3), s = (uint32_t)(j & 7);
  const uint32_t blk = (uint32_t)pf_block_bytes(FMT) * b;
  if constexpr (FMT == PF_Q4K) {   // header, then the half-block's 64 qs bytes
    return blk + (q == 0 ? 0u : 16u * (uint32_t)q + 64u * (s >> 2));
  } else if constexpr (FMT == PF_Q5K) {   // header, the 32 qh bytes, then the half-block's 64 qs bytes
    return blk + (q < 3 ? 16u * (uint32_t)q : 16u * (uint32_t)q + 64u * (s >> 2));
  } else {
    // Q6_K is staged a half-block (128 weights = sub-blocks 4 h' .. 4 h' + 3, one 128-k chunk) at a
    // time: its 64 ql bytes start at blk + 20 + 64 h', its 32 qh bytes at blk + 148 + 32 h', both
    // 4 (b + 1) mod 16 past a 16-B boundary (blk = 212 b is 4 b mod 16); the header cover (d, the
    // 16 scales) starts at blk rounded down.  Pieces 0-4: the ql cover, 5-7: the qh cover, 8-9: the
    // header; a cover that starts on a boundary needs one piece fewer, which re-loads its last.
    const uint32_t hp = s >> 2, m = 4u * ((b + 1u) & 3u), mh = 4u * (b & 3u);
    if (q < 5) return blk + 20u + 64u * hp - m + 16u * min((uint32_t)q, m == 0 ? 3u : 4u);
    if (q < 8) return blk + 148u + 32u * hp - m + 16u * min((uint32_t)q - 5u, m == 0 ? 1u : 2u);
    return blk - mh + 16u * ((uint32_t)q - 8u);
  }
}

// Stage the pieces of sub-block j into ring stage `stage` (wave-uniform; pf_kq_dmas loads).
template <int FMT>
__device__ __forceinline__ void pf_kq_dma(PfLds& L, int stage, const uint8_t* __restrict__ wt, uint32_t rowb,
                                          int j, int wave, int lane) {
  constexpr int P = pf_kq_pieces<FMT>();
#pragma unroll
  for (int i = 0; i < pf_kq_dmas<FMT>(); ++i) {
    const int p = min(TLX_WAVE * i + lane, 32 * P - 1);
    const int r = p / P, q = p - r * P;
    const uint8_t* src = wt + (size_t)(32 * wave + r) * rowb + pf_kq_piece_off<FMT>(j, q);
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(&L.kq[stage][wave][i][0]), 16, 0, 0);
  }
}

// One thread's bytes of a sub-block, read back from its wave's slab.
struct PfKq {
  u4_t q;      // Q4_K / Q5_K: 16 qs bytes (nibble s & 1); Q6_K: 16 ql bytes (nibble g >= 2)
  u4_t hb;     // Q5_K: qh bytes 16h .. 16h + 15 (bit s); Q6_K: qh bytes (bits 2g, 2g + 1)
  u4_t hdr;    // Q4_K / Q5_K: d, dmin, the 12 packed scale bytes; Q6_K: .x = d
  uint32_t sc; // Q6_K: the scale dword holding sc[8 h' + h + 2 g]
};

template <int FMT>
__device__ __forceinline__ void pf_kq_read(PfKq& r, const PfLds& L, int stage, int j, int wave, int lane) {
  constexpr int P = pf_kq_pieces<FMT>();
  const int h = lane & 1;
  const uint8_t* cb = reinterpret_cast<const uint8_t*>(&L.kq[stage][wave][0][0]) + 16 * P * (lane >> 1);
  if constexpr (FMT == PF_Q4K) {   // sub-block j's pair (j & 7) / 2 of the half-block's two
    r.hdr = *reinterpret_cast<const u4_t*>(cb);
    r.q = *reinterpret_cast<const u4_t*>(cb + 16 + 32 * ((j >> 1) & 1) + 16 * h);
  } else if constexpr (FMT == PF_Q5K) {
    r.hdr = *reinterpret_cast<const u4_t*>(cb);
    r.hb = *reinterpret_cast<const u4_t*>(cb + 16 + 16 * h);
    r.q = *reinterpret_cast<const u4_t*>(cb + 48 + 32 * ((j >> 1) & 1) + 16 * h);
  } else {   // the row's half-block slab: ql cover (80 B), qh cover (48 B), header cover (32 B)
    const uint32_t b = (uint32_t)(j >> 3), s = (uint32_t)(j & 7);
    const uint32_t m = 4u * ((b + 1u) & 3u), mh = 4u * (b & 3u);
    const uint32_t* ql = reinterpret_cast<const uint32_t*>(cb + m + 32 * (s & 1) + 16 * h);
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(cb + 80 + m + 16 * h);
    r.q = u4_t{ql[0], ql[1], ql[2], ql[3]};
    r.hb = u4_t{qh[0], qh[1], qh[2], qh[3]};
    r.hdr.x = *reinterpret_cast<const uint16_t*>(cb + 128 + mh + 2);
    const uint32_t i = 8u * (s >> 2) + (uint32_t)h + 2u * (s & 3u);
    r.sc = *reinterpret_cast<const uint32_t*>(cb + 128 + mh + 4 + (i & ~3u));
  }
}

// fp16 of an fp32 value, round to nearest even (the reference's __float2half)
__device__ __forceinline__ uint32_t pf_pack2(float a, float b) {
  const h2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// The 16 operand values of sub-block j for half h into pieces 2h, 2h + 1 of tile row r.
template <int FMT>
__device__ __forceinline__ void pf_kq_dequant(const PfKq& r, _Float16* bt, int row, int j, int h) {
  const int s = j & 7;
  uint32_t w[8];
  if constexpr (FMT == PF_Q4K || FMT == PF_Q5K) {
    const uint32_t hx = r.hdr.x;
    const float d = tlx_h2f((uint16_t)(hx & 0xFFFFu)), dmin = tlx_h2f((uint16_t)(hx >> 16));
    // 6-bit scale and min of sub-block s from the 12 packed bytes (ggml get_scale_min_k4)
    const uint32_t q03 = r.hdr.y, q47 = r.hdr.z, q811 = r.hdr.w;
    auto byte = [](uint32_t v, int i) { return (v >> (8 * i)) & 0xFFu; };
    uint32_t sc, mn;
    if (s < 4) {
      sc = byte(q03, s) & 63u;
      mn = byte(q47, s) & 63u;
    } else {
      sc = (byte(q811, s - 4) & 0xFu) | ((byte(q03, s - 4) >> 6) << 4);
      mn = (byte(q811, s - 4) >> 4) | ((byte(q47, s - 4) >> 6) << 4);
    }
    const float A = d * (float)sc, B = dmin * (float)mn;   // exact in fp32
    const uint32_t sh = 4u * (uint32_t)(s & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = (r.q[i] >> sh) & 0x0F0F0F0Fu;
      uint32_t hi = 0;
      if constexpr (FMT == PF_Q5K) hi = ((r.hb[i] >> s) & 0x01010101u) << 4;
      const uint32_t qv = v | hi;
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = __builtin_fmaf(A, (float)((qv >> (8 * e)) & 0xFFu), -B);
      w[2 * i] = pf_pack2(f[0], f[1]);
      w[2 * i + 1] = pf_pack2(f[2], f[3]);
    }
  } else {
    // A * (q - 32) has at most 11 + 7 + 5 = 23 significant bits: exact in f32, so v_fma_mix's
    // one rounding of the product (the level as an fp16 integer) is fp16(f32 product)
    const int hp = s >> 2, g = s & 3;
    const float d = tlx_h2f((uint16_t)r.hdr.x);
    const int sci = (8 * hp + h + 2 * g) & 3;
    const float A = d * (float)(int8_t)((r.sc >> (8 * sci)) & 0xFFu);
    const uint32_t nsh = g >= 2 ? 4u : 0u, hsh = 2u * (uint32_t)g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t qv = ((r.q[i] >> nsh) & 0x0F0F0F0Fu) | (((r.hb[i] >> hsh) & 0x03030303u) << 4);
      w[2 * i] = tlx_mix2_f16(A, tlx_bytes_h2(qv, 0, 32.f));
      w[2 * i + 1] = tlx_mix2_f16(A, tlx_bytes_h2(qv, 1, 32.f));
    }
  }
  *reinterpret_cast<u4_t*>(bt + pf_frag(row, 2 * h)) = u4_t{w[0], w[1], w[2], w[3]};
  *reinterpret_cast<u4_t*>(bt + pf_frag(row, 2 * h + 1)) = u4_t{w[4], w[5], w[6], w[7]};
}

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

// Ring stage of sub-block j's pieces: each half-block (128 k) has a stage, alternating
template <int FMT>
__device__ __forceinline__ int pf_kq_stage(int j) { return (j >> 2) & 1; }

// One k-step of a k-quant segment: the operand loads of step t; the decode of sub-block t + 1
// (staged at step t - 1 at the latest: the two activation loads issued after it may still be in
// flight); on the step before a half-block starts (t + 2 = 0 mod 4), that half-block's pieces
// into the other stage; the activations of step t + 2; the MFMAs, which the scheduler
// interleaves with the decode; the barrier.
template <int FMT>
__device__ __forceinline__ void pf_kq_step(PfLds& L, f4_t (&acc)[kMI][8], const PfArgs& g, const int* bg, int aoff,
                                           int t, int ra, int wave, int wm, int lane) {
  PfFrag f;
  pf_load_frag(f, L.a[ra], L.b[t & 1], bg, aoff, wm, lane);
  const int j1 = min(t + 1, g.tlast);
  asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  PfKq kr;
  pf_kq_read<FMT>(kr, L, pf_kq_stage<FMT>(j1), j1, wave, lane);
  pf_kq_dequant<FMT>(kr, L.b[(t + 1) & 1], (int)threadIdx.x >> 1, j1, lane & 1);
  const bool wdma = ((t + 2) & 3) == 0 && t + 2 <= g.tlast;   // weight pieces this step (wave-uniform)
  if (wdma) pf_kq_dma<FMT>(L, pf_kq_stage<FMT>(t + 2), g.wkq, g.rowb, t + 2, wave, lane);
  const int ra2 = ra == 0 ? 2 : ra - 1;
  pf_dma_a(L.a[ra2], g.x, g.m0, g.K, min(t + 2, g.tlast), wave, lane);
  pf_mfma<0, kMI>(acc, f);
  // step t+1's activations (issued at step t-1) must have landed; this step's weight pieces and
  // activations stay in flight
  __builtin_amdgcn_sched_barrier(0);
  static_assert(kLdW == 2, "the wait counts below assume 2 A loads per wave per step");
  if (!wdma) {
    asm volatile("s_waitcnt vmcnt(2)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else if constexpr (pf_kq_dmas<FMT>() == 3) {   // Q4_K
    asm volatile("s_waitcnt vmcnt(5)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else if constexpr (pf_kq_dmas<FMT>() == 4) {   // Q5_K
    asm volatile("s_waitcnt vmcnt(6)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    static_assert(pf_kq_dmas<FMT>() == 5, "Q6_K: 5 weight loads on a half-block step");
    asm volatile("s_waitcnt vmcnt(7)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
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

// (m-tile, n-tile) of tile index tau: when there are m-tiles for all 8 XCDs, workgroup tau runs
// on XCD tau % 8 and that XCD sweeps the n-tiles of m-tiles x, x+8, ... in turn
__device__ __forceinline__ void pf_tile_of(int tau, int mtiles, int ntiles, int& mt, int& nt) {
  if ((mtiles & 7) == 0) {
    const int l = tau >> 3;
    mt = (tau & 7) + 8 * (l / ntiles);
    nt = l % ntiles;
  } else {
    mt = tau % mtiles;
    nt = tau / mtiles;
  }
}

// One workgroup's tile (or k-range segment of a split tile: seg >= 0, chunks [h0, h1)): the
// prologue, the k-steps, then the epilogue or the part store.  nt: the tile's n-tile within its
// matrix (or matrix pair); wkq: k-quant formats, the matrix.
template <int EPI, int FMT>
__device__ __forceinline__ void pf_tile(PfLds& L, const u4_t* __restrict__ w1, const u4_t* __restrict__ w2,
                                        const uint8_t* __restrict__ wkq, const float* __restrict__ gridf,
                                        const _Float16* __restrict__ x, void* __restrict__ out,
                                        const float* __restrict__ res, int N, int K, int mt, int nt, int h0, int h1,
                                        int seg, const PfSk& sk) {
  constexpr bool kFfn = EPI == PF_FFN;
  // wave index as a scalar: the per-wave DMA selection branches on SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int nch = K / 128;
  PfArgs g;
  g.w1 = w1; g.w2 = w2; g.x = x; g.K = K; g.nch = nch;
  g.m0 = mt * kBM; g.nt = nt;
  g.tlast = 4 * h1 - 1; g.hlast = h1 - 1;
  g.wkq = nullptr;
  g.rowb = 0;
  const int s0 = 4 * h0;

  if constexpr (FMT == PF_IQ3) {
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
  } else {
    // prologue: activation steps s0, s0+1 and the weight pieces of sub-blocks s0, s0+1; sub-block s0
    // decoded (every segment starts on a 128-k chunk)
    g.rowb = (uint32_t)(pf_block_bytes(FMT) * (K >> 8));
    g.wkq = wkq + (size_t)(nt * kBN) * g.rowb;
    pf_kq_dma<FMT>(L, pf_kq_stage<FMT>(s0), g.wkq, g.rowb, s0, wave, lane);   // the half-block of s0 .. s0 + 3
    pf_dma_a(L.a[0], x, g.m0, K, s0, wave, lane);
    pf_dma_a(L.a[1], x, g.m0, K, s0 + 1, wave, lane);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    PfKq kr;
    pf_kq_read<FMT>(kr, L, pf_kq_stage<FMT>(s0), s0, wave, lane);
    pf_kq_dequant<FMT>(kr, L.b[s0 & 1], threadIdx.x >> 1, s0, lane & 1);
    __syncthreads();
  }

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
  if constexpr (FMT == PF_IQ3) {
    for (int t = s0; t <= g.tlast; ++t) {
      pf_step<kFfn>(L, acc, g, bg, aoff, t, ra, wave, wm, lane);
      ra = ra == 2 ? 0 : ra + 1;
    }
  } else {
    for (int t = s0; t <= g.tlast; ++t) {
      pf_kq_step<FMT>(L, acc, g, bg, aoff, t, ra, wave, wm, lane);
      ra = ra == 2 ? 0 : ra + 1;
    }
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

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void pf_gemm_kernel(
    const u4_t* __restrict__ w1, const u4_t* __restrict__ w2, const float* __restrict__ gridf,
    const _Float16* __restrict__ x, void* __restrict__ out, const float* __restrict__ res, int M, int N,
    int K, int mtiles, int ntiles, const PfSk sk) {
  __shared__ PfLds L;
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
  pf_tile_of(tau, mtiles, ntiles, mt, nt);
  pf_tile<EPI, PF_IQ3>(L, w1, w2, nullptr, gridf, x, out, res, N, K, mt, nt, h0, h1, seg, sk);
}

// The merged form: up to three segments (matrices of any PfFmt sharing x), fp16 outputs; the
// n-tiles of all segments form one tile range, a workgroup's n-tile selects its segment.
struct PfSeg {
  const void* w;
  uint16_t* out;
  int n;        // rows (output columns)
  int fmt;      // PfFmt
  int nt0;      // first n-tile of the segment in the merged range
};
struct PfMulti {
  PfSeg seg[3];
  int nseg;
};

__global__ __launch_bounds__(kThreads, 1) void pfm_gemm_kernel(const PfMulti mseg, const float* __restrict__ gridf,
                                                               const _Float16* __restrict__ x, int K, int mtiles,
                                                               int ntiles) {
  __shared__ PfLds L;
  int mt, ntg;
  pf_tile_of((int)blockIdx.x, mtiles, ntiles, mt, ntg);
  int s = 0;
  while (s + 1 < mseg.nseg && ntg >= mseg.seg[s + 1].nt0) ++s;
  const PfSeg sg = mseg.seg[s];
  const int nt = ntg - sg.nt0, nch = K / 128;
  const PfSk none{0, 0, 1, nullptr};
  const u4_t* w = static_cast<const u4_t*>(sg.w);
  const uint8_t* wb = static_cast<const uint8_t*>(sg.w);
  switch (sg.fmt) {
    case PF_IQ3: pf_tile<PF_F16, PF_IQ3>(L, w, nullptr, nullptr, gridf, x, sg.out, nullptr, sg.n, K, mt, nt, 0, nch, -1, none); break;
    case PF_Q4K: pf_tile<PF_F16, PF_Q4K>(L, nullptr, nullptr, wb, gridf, x, sg.out, nullptr, sg.n, K, mt, nt, 0, nch, -1, none); break;
    case PF_Q5K: pf_tile<PF_F16, PF_Q5K>(L, nullptr, nullptr, wb, gridf, x, sg.out, nullptr, sg.n, K, mt, nt, 0, nch, -1, none); break;
    default: pf_tile<PF_F16, PF_Q6P>(L, nullptr, nullptr, wb, gridf, x, sg.out, nullptr, sg.n, K, mt, nt, 0, nch, -1, none); break;
  }
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
  pf_tile_of(tau, mtiles, ntiles, mt, nt);
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

extern "C" int tlx_pfg3m(const void* const* w, uint16_t* const* out, const int* n, const int* type,
                         const int* layout, int nseg, const float* gridf, const uint16_t* x16, int M, int K,
                         void* stream) {
  TLX_RET_IF(w == nullptr || out == nullptr || n == nullptr || type == nullptr || layout == nullptr, TLX_E_ARG);
  TLX_RET_IF(nseg < 1 || nseg > 3, TLX_E_ARG);
  // k-quant blocks are 256 wide and every segment starts its k-loop on a 128-k chunk
  TLX_RET_IF(M < kBM || (M % kBM) || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(x16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  PfMulti ms{};
  int ntiles = 0;
  for (int s = 0; s < nseg; ++s) {
    TLX_RET_IF(n[s] < kBN || (n[s] % kBN), TLX_E_ARG);
    int f;
    if (type[s] == TLX_TYPE_IQ3_XXS && layout[s] == TLX_LAYOUT_PACK7) f = PF_IQ3;
    else if (type[s] == TLX_TYPE_Q4_K && layout[s] == TLX_LAYOUT_RAW) f = PF_Q4K;
    else if (type[s] == TLX_TYPE_Q5_K && layout[s] == TLX_LAYOUT_RAW) f = PF_Q5K;
    else if (type[s] == TLX_TYPE_Q6_K && layout[s] == TLX_LAYOUT_PACKED) f = PF_Q6P;
    else return TLX_E_ARG;
    TLX_RET_IF(!tlx_aligned(w[s], 16) || !tlx_aligned(out[s], 16), TLX_E_ALIGN);
    ms.seg[s] = PfSeg{w[s], out[s], n[s], f, ntiles};
    ntiles += n[s] / kBN;
  }
  ms.nseg = nseg;
  const int mtiles = M / kBM;
  pfm_gemm_kernel<<<mtiles * ntiles, kThreads, 0, (hipStream_t)stream>>>(ms, gridf, (const _Float16*)x16, K, mtiles,
                                                                         ntiles);
  return tlx_launch_status();
}
