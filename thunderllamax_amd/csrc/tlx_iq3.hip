// IQ3_XXS kernels for gfx950: bit-exact dequantization and the MFMA decode GEMV family
// (FFN gate+up + SwiGLU, down + residual, fused attention q/k/v, plain GEMV).
//
// GEMV design (one kernel for every M in 1..16):
//   * a workgroup owns a tile of 16 weight rows; its waves split the K blocks between them
//     (block b goes to wave b % WAVES) and reduce through LDS in a fixed order, so the
//     result does not depend on scheduling;
//   * lane l of a wave owns weight row (l & 15) and the 64 consecutive k of each 256-block
//     starting at 64*(l >> 4): one 16-B load of its 8 grid-index words, one 8-B load of its
//     two scale/sign words, one 2-B load of the block's d;
//   * each of the 8 lane-chunks (8 weights) becomes the B operand of one
//     v_mfma_f32_16x16x32_f16; the A operand is the matching 8 activations of row (l & 15)
//     (rows >= M load a valid row; their outputs are never stored).  MFMA sums over k, and k
//     is paired the same way in A and B, so the lane -> k assignment inside an instruction
//     is free;
//   * the decoded operand is exact: |grid| * (2s+1)/4 with the sign folded in (at most 10
//     significant bits, so exact in fp16); the per-block d is applied once per block to the
//     fp32 MFMA partial.  Products are therefore the exact products of the GGUF weight and
//     the fp16 activation, accumulated in fp32;
//   * grid magnitude and sign come from one LDS lookup per 4 weights in a 4096-entry table
//     (sign nibble << 8 | grid index) of four fp16 values, built per workgroup from the
//     caller's gridf buffer.
#include "tlx_common.h"

#include <mutex>

namespace {

constexpr int kIq3BlockBytes = 98;
constexpr int kTblEntries = 4096;
constexpr int kTile = 16;
constexpr int kXtMinM = 6;  // from this M on, activations are read from the tile-ordered copy

enum Epi { EPI_F16 = 0, EPI_SWIGLU = 1, EPI_RESID = 2 };

// 8 signed grid magnitudes of one lane-chunk: q word = two grid indices, sidx = the 7-bit
// sign field; the 8th sign is the parity of sidx.
__device__ __forceinline__ h8_t iq3_chunk(const u2_t* tbl, uint32_t qw, uint32_t sidx) {
  const uint32_t par = __builtin_popcount(sidx) & 1u;
  const uint32_t i0 = ((sidx & 0xFu) << 8) | (qw & 0xFFu);
  const uint32_t i1 = (((sidx >> 4) | (par << 3)) << 8) | ((qw >> 8) & 0xFFu);
  const u2_t a = tbl[i0];
  const u2_t b = tbl[i1];
  return __builtin_bit_cast(h8_t, u4_t{a.x, a.y, b.x, b.y});
}

__device__ __forceinline__ h8_t splat8(_Float16 v) { return h8_t{v, v, v, v, v, v, v, v}; }

struct Iq3Seg {
  const uint8_t* w0;   // weights (packed rows)
  const uint8_t* w1;   // second matrix of a pair (SwiGLU up), else null
  void* out;           // fp16 [M][n] or fp32 [M][n]
  const float* res;    // residual [M][n] (EPI_RESID)
  int n;               // rows in this segment
  int tile0;           // first workgroup of this segment
};

struct Iq3Launch {
  Iq3Seg seg[4];
  int nseg;
  const float* gridf;
  const _Float16* x;   // activations [M][K], or (xt) the tile-ordered copy [K/8][16][8]
  int xt;
  int otile;           // TLX_OUT_TILEORD: outputs in the tile-ordered form (tiled records only)
  int M, K;
  int layout;          // TLX_LAYOUT_RAW, TLX_LAYOUT_PACKED or TLX_LAYOUT_TILED
  void* ws;            // GEMV workspace (kWsBytes) or nullptr: iq3_launch then takes the attached one
  int noks;            // 1: ws has only the base regions (kWsBaseBytes): no k-split form
};

template <int NMAT>
struct Iq3Regs {
  u4_t qs[NMAT];
  u2_t sw[NMAT];
  uint32_t d[NMAT];
};

// Loads one block of the lane's row: 16 B of grid indices, 8 B of scale/sign words, the d.
// Offsets are 32-bit (a matrix is < 4 GiB) from the matrix base.
// The per-block strides are those of the layout: 64/32/2 B (packed rows) or 98 B (GGUF blocks,
// whose fields are only 2-B aligned: the loads are unaligned there).
template <int NMAT>
__device__ __forceinline__ void iq3_load(Iq3Regs<NMAT>& r, const uint8_t* const* base, uint32_t qoff,
                                         uint32_t soff, uint32_t doff, uint32_t qst, uint32_t sst,
                                         uint32_t dst, int b) {
#pragma unroll
  for (int i = 0; i < NMAT; ++i) {
    r.qs[i] = tlx_ldu<u4_t>(base[i] + (qoff + qst * b));
    r.sw[i] = tlx_ldu<u2_t>(base[i] + (soff + sst * b));
    r.d[i] = tlx_ldu<uint16_t>(base[i] + (doff + dst * b));
  }
}

// The same registers from the packed7 units (TLX_LAYOUT_PACK7, engine/pack_w7.py:7-21): the lane's
// 64 k of block b are sub-blocks c0, c0 + 1 of chunk 2b + (kq >> 1) (c0 = 2 (kq & 1)), two adjacent
// 16-B units [q u16 x4][sw][d][pad] of its row: q words 0..3 then 4..7, the two scale/sign words,
// the block's d.  The values are those the packed rows give, so the GEMV results are bit-identical.
template <int NMAT>
__device__ __forceinline__ void iq3_load7(Iq3Regs<NMAT>& r, const uint8_t* const* base, uint32_t off, int b) {
#pragma unroll
  for (int i = 0; i < NMAT; ++i) {
    const uint8_t* p = base[i] + (off + 1024u * (uint32_t)b);
    const u4_t u0 = *reinterpret_cast<const u4_t*>(p);
    const u4_t u1 = *reinterpret_cast<const u4_t*>(p + 16);
    r.qs[i] = u4_t{u0.x, u0.y, u1.x, u1.y};
    r.sw[i] = u2_t{u0.z, u1.z};
    r.d[i] = u0.w;
  }
}

// P7: 0 = packed rows / GGUF blocks (strided fields), 1 = packed7 units
template <int NMAT, int EPI, int WAVES, int P7>
__global__ __launch_bounds__(WAVES * TLX_WAVE) void iq3_gemv_kernel(const Iq3Launch a) {
  __shared__ u2_t tbl[kTblEntries];
  tlx_iq3_table(tbl, a.gridf);
  __syncthreads();

  int s = 0;
  while (s + 1 < a.nseg && (int)blockIdx.x >= a.seg[s + 1].tile0) ++s;
  const Iq3Seg& sg = a.seg[s];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;
  const int K = a.K, M = a.M, nb = K >> 8;
  const uint32_t rowb = (uint32_t)kIq3BlockBytes * nb;
  const int tile = (int)blockIdx.x - sg.tile0;
  const int row0 = tile * kTile;
  uint32_t qoff, soff, doff, qst, sst, dst;
  {
    // tail tile: clamp the loads, mask the stores
    const bool raw = a.layout == TLX_LAYOUT_RAW;
    const int row = min(row0 + col, sg.n - 1);
    const uint32_t roff = (uint32_t)row * rowb;
    qoff = roff + (raw ? 2u : 0u) + 16u * kq;
    soff = roff + (raw ? 66u : 64u * nb) + 8u * kq;
    doff = roff + (raw ? 0u : 96u * nb);
    qst = raw ? 98u : 64u;
    sst = raw ? 98u : 32u;
    dst = raw ? 98u : 2u;
    if constexpr (P7)   // unit (row & 7, c0) of chunk kq >> 1 in group row >> 3 (2 * nb chunks a group)
      qoff = ((uint32_t)((row >> 3) * 2 * nb + (kq >> 1)) * 32u + 4u * (uint32_t)(row & 7) + 2u * (kq & 1)) * 16u;
  }

  const uint8_t* base[NMAT];
  base[0] = sg.w0;
  if constexpr (NMAT == 2) base[1] = sg.w1;

  // Activation rows >= M only reach output rows that are never stored, so those lanes load a
  // valid row instead of being masked: no branches, and the wait counters stay exact.  From the
  // tile-ordered copy (M >= kXtMinM) the 4 lanes of a quad read 64 contiguous bytes.
  const _Float16* xr = a.xt ? a.x + (size_t)(1024 * kq + 8 * col)
                            : a.x + (size_t)min(col, M - 1) * K + 64 * kq;
  const int xbs = a.xt ? 4096 : 256, xcs = a.xt ? 128 : 8;  // halves per block / per chunk

  f4_t acc[NMAT];
#pragma unroll
  for (int i = 0; i < NMAT; ++i) acc[i] = f4_t{0.f, 0.f, 0.f, 0.f};

  auto load = [&](Iq3Regs<NMAT>& r, int blk) {
    if constexpr (P7) iq3_load7<NMAT>(r, base, qoff, blk);
    else iq3_load<NMAT>(r, base, qoff, soff, doff, qst, sst, dst, blk);
  };
  int b = wave;
  Iq3Regs<NMAT> cur;
  if (b < nb) load(cur, b);
  for (; b < nb; b += WAVES) {
    // this block's activations first, then the next block's weights: waiting for the
    // activations leaves the weight prefetch in flight
    h8_t X[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) X[t] = *reinterpret_cast<const h8_t*>(xr + xbs * b + xcs * t);
    Iq3Regs<NMAT> nxt;
    const bool more = b + WAVES < nb;
    if (more) load(nxt, b + WAVES);

#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      const _Float16 ks0 = (_Float16)((float)(2u * (cur.sw[i].x >> 28) + 1u) * 0.25f);
      const _Float16 ks1 = (_Float16)((float)(2u * (cur.sw[i].y >> 28) + 1u) * 0.25f);
      f4_t D = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t qd = cur.qs[i][t >> 1];
        const uint32_t qw = (t & 1) ? (qd >> 16) : (qd & 0xFFFFu);
        const uint32_t sw = (t < 4) ? cur.sw[i].x : cur.sw[i].y;
        const uint32_t sidx = (sw >> (7 * (t & 3))) & 0x7Fu;
        const h8_t B = iq3_chunk(tbl, qw, sidx) * splat8(t < 4 ? ks0 : ks1);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(X[t], B, D, 0, 0, 0);
      }
      const float d = tlx_h2f((uint16_t)cur.d[i]);
      acc[i] += d * D;
    }
    if (more) cur = nxt;
  }

  // fixed-order split-K reduction through LDS (the table is dead after this barrier)
  __syncthreads();
  if constexpr (WAVES > 1) {
    float* red = reinterpret_cast<float*>(tbl);
    if (wave > 0) {
#pragma unroll
      for (int i = 0; i < NMAT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(((wave - 1) * NMAT + i) * 4 + r) * TLX_WAVE + lane] = acc[i][r];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < WAVES; ++w)
#pragma unroll
      for (int i = 0; i < NMAT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] += red[(((w - 1) * NMAT + i) * 4 + r) * TLX_WAVE + lane];
  }

  // lane (col, kq) holds D[m = 4*kq + r][col]
  const int n = row0 + col;
  if (n >= sg.n) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kq + r;
    if (m >= M) break;
    const size_t o = (size_t)m * sg.n + n;
    if constexpr (EPI == EPI_SWIGLU) {
      reinterpret_cast<uint16_t*>(sg.out)[o] = tlx_swiglu_bits(acc[0][r], acc[1][r]);
    } else if constexpr (EPI == EPI_RESID) {
      reinterpret_cast<float*>(sg.out)[o] = sg.res[o] + (float)(_Float16)acc[0][r];
    } else {
      reinterpret_cast<uint16_t*>(sg.out)[o] = tlx_f2h_bits(acc[0][r]);
    }
  }
}

// The tile-ordered activation copy: xt[kc][col][0..7] = x[min(col, M - 1)][8kc .. 8kc + 7].
__global__ __launch_bounds__(256) void iq3_xt_kernel(const _Float16* __restrict__ x,
                                                     _Float16* __restrict__ xt, int M, int K) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);  // (kc, col)
  if (i >= (K >> 3) * 16) return;
  const int kc = i >> 4, col = i & 15;
  *reinterpret_cast<u4_t*>(xt + (size_t)i * 8) =
      *reinterpret_cast<const u4_t*>(x + (size_t)min(col, M - 1) * K + 8 * kc);
}

template <int NMAT, int EPI>
int iq3_launch(Iq3Launch& a, int tiles, hipStream_t st) {
  const int nb = a.K >> 8;
  if (a.ws == nullptr) {
    const int rc = tlx_workspace(&a.ws);
    if (rc != TLX_OK) return rc;
  }
  if (a.layout == TLX_LAYOUT_TILED && a.ws == nullptr) return TLX_E_NOWS;   // parts and counters
  // same values, same arithmetic: only the activation loads change (larger K reads x directly);
  // a.xt set by the caller: a.x already is the tile-ordered copy (written by a producer)
  const bool staged = a.layout == TLX_LAYOUT_TILED &&
                      tlx_iq3s_stages_x(NMAT, a.M, a.seg[0].n, a.K, a.nseg, !a.noks);  // no copy needed
  // without a workspace the packed-row GEMV reads x directly (same values, slower loads)
  if (!a.xt && !staged && a.ws != nullptr && a.M >= kXtMinM && (size_t)a.K * 16 * 2 <= kWsXtBytes) {
    _Float16* xt = reinterpret_cast<_Float16*>(static_cast<uint8_t*>(a.ws) + kWsXtOff);
    iq3_xt_kernel<<<(a.K / 8 * 16 + 255) / 256, 256, 0, st>>>(a.x, xt, a.M, a.K);
    const int lrc = tlx_launch_status();
    if (lrc != TLX_OK) return lrc;
    a.x = xt;
    a.xt = 1;
  }
  if (a.layout == TLX_LAYOUT_TILED) {
    const void* w[4];
    void* out[4];
    int n[4];
    for (int i = 0; i < a.nseg; ++i) {
      w[i] = a.seg[i].w0;
      out[i] = a.seg[i].out;
      n[i] = a.seg[i].n;
    }
    return tlx_iq3s_launch(NMAT, EPI, a.nseg, w, a.seg[0].w1, out, n, a.seg[0].res, a.gridf, a.x, a.xt, a.M,
                           a.K, a.ws, !a.noks, a.otile != 0, st);
  }
  if (a.otile) return TLX_E_ARG;   // the tile-ordered output exists for the tiled records only
  int waves = 4;
  while (tiles * waves < 4096 && waves < 16 && nb >= 4 * waves) waves *= 2;
  const bool p7 = a.layout == TLX_LAYOUT_PACK7;
  switch (waves) {
    case 4:
      if (p7) iq3_gemv_kernel<NMAT, EPI, 4, 1><<<tiles, 4 * TLX_WAVE, 0, st>>>(a);
      else iq3_gemv_kernel<NMAT, EPI, 4, 0><<<tiles, 4 * TLX_WAVE, 0, st>>>(a);
      break;
    case 8:
      if (p7) iq3_gemv_kernel<NMAT, EPI, 8, 1><<<tiles, 8 * TLX_WAVE, 0, st>>>(a);
      else iq3_gemv_kernel<NMAT, EPI, 8, 0><<<tiles, 8 * TLX_WAVE, 0, st>>>(a);
      break;
    default:
      if (p7) iq3_gemv_kernel<NMAT, EPI, 16, 1><<<tiles, 16 * TLX_WAVE, 0, st>>>(a);
      else iq3_gemv_kernel<NMAT, EPI, 16, 0><<<tiles, 16 * TLX_WAVE, 0, st>>>(a);
      break;
  }
  return tlx_launch_status();
}



// Splits the activation-form flags off `layout`; TLX_E_ARG for flags the entry point does not take.
int iq3_flags(int& layout, int allowed, Iq3Launch& a) {
  const int fl = layout & (TLX_OUT_TILEORD | TLX_IN_TILEORD);
  if (fl & ~allowed) return TLX_E_ARG;
  layout &= ~(TLX_OUT_TILEORD | TLX_IN_TILEORD);
  a.otile = (fl & TLX_OUT_TILEORD) ? 1 : 0;
  a.xt = (fl & TLX_IN_TILEORD) ? 1 : 0;
  return TLX_OK;
}

int iq3_check(const void* w, int M, int N, int K, int layout) {
  if (M < 1 || M > TLX_MAX_M || N < 1 || K < 256 || (K & 255)) return TLX_E_ARG;
  if (layout != TLX_LAYOUT_PACKED && layout != TLX_LAYOUT_RAW && layout != TLX_LAYOUT_TILED &&
      layout != TLX_LAYOUT_PACK7)
    return TLX_E_ARG;
  // packed7 units come in 8-row groups (N % 8 == 0) and are read as 16-B vectors
  if (layout == TLX_LAYOUT_PACK7 && (N & 7)) return TLX_E_ARG;
  if (layout == TLX_LAYOUT_PACK7 && !tlx_aligned(w, 16)) return TLX_E_ALIGN;
  // packed rows: the operand loads are dword-aligned when the row bytes 98*NB are (NB even);
  // tiled records are 1632 B (16-B aligned fields); GGUF blocks are 2-B aligned throughout
  if (layout == TLX_LAYOUT_PACKED && (((K >> 8) & 1) || !tlx_aligned(w, 4))) return TLX_E_ALIGN;
  if (layout == TLX_LAYOUT_TILED && !tlx_aligned(w, 16)) return TLX_E_ALIGN;
  if (!tlx_aligned(w, 2)) return TLX_E_ALIGN;
  // kernels address a matrix with 32-bit byte offsets (tiled: 102-B records of whole tiles)
  const size_t bytes = layout == TLX_LAYOUT_TILED  ? (size_t)(N + kTile - 1) / kTile * kTile * 102 * (K >> 8)
                      : layout == TLX_LAYOUT_PACK7 ? (size_t)N * 128 * (K >> 8)
                                                   : (size_t)N * kIq3BlockBytes * (K >> 8);
  if (bytes > 0xFFFFFFFFull) return TLX_E_ARG;
  return TLX_OK;
}

inline int tiles_of(int n) { return (n + kTile - 1) / kTile; }

// ------------------------------------------------------------------ dequantization
// One thread per lane-chunk (8 weights).  Exact fp32 arithmetic in the reference order
// d*((sw>>28)+0.5)*0.5, then *grid, then *sign; fp16 output rounds that exact value once.
__global__ __launch_bounds__(256) void iq3_dequant_kernel(const uint8_t* __restrict__ w,
                                                          const float* __restrict__ gridf,
                                                          void* __restrict__ out, int64_t rows,
                                                          int nb, int layout, int out_f16) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // chunk index
  const int64_t nchunk = rows * nb * 32;
  if (c >= nchunk) return;
  const int lc = (int)(c & 31);
  const int64_t rb = c >> 5;  // row * nb + b
  const int b = (int)(rb % nb);
  const int64_t row = rb / nb;
  uint32_t q, sw;
  uint16_t dbits;
  if (layout == TLX_LAYOUT_RAW) {
    const uint8_t* blk = w + rb * kIq3BlockBytes;
    dbits = tlx_ldu<uint16_t>(blk);
    q = tlx_ldu<uint16_t>(blk + 2 + 2 * lc);
    sw = tlx_ldu<uint32_t>(blk + 66 + 4 * (lc >> 2));
  } else {
    const uint8_t* rp = w + row * (int64_t)(kIq3BlockBytes * nb);
    q = tlx_ldu<uint16_t>(rp + 64 * b + 2 * lc);
    sw = tlx_ldu<uint32_t>(rp + 64 * nb + 32 * b + 4 * (lc >> 2));
    dbits = tlx_ldu<uint16_t>(rp + 96 * nb + 2 * b);
  }
  const float d = tlx_h2f(dbits);
  const float db = d * ((float)(sw >> 28) + 0.5f) * 0.5f;
  const uint32_t sidx = (sw >> (7 * (lc & 3))) & 0x7Fu;
  const uint32_t sbyte = sidx | ((__builtin_popcount(sidx) & 1u) << 7);
  const float4 g0 = reinterpret_cast<const float4*>(gridf)[q & 0xFFu];
  const float4 g1 = reinterpret_cast<const float4*>(gridf)[q >> 8];
  const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const int64_t k0 = rb * 256 + 8 * lc;
  if (out_f16) {
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = tlx_f2h_bits(db * g[j] * (((sbyte >> j) & 1u) ? -1.f : 1.f));
    uint4 pk;
    __builtin_memcpy(&pk, v, 16);
    reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + k0)[0] = pk;
  } else {
    float* o = reinterpret_cast<float*>(out) + k0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = db * g[j] * (((sbyte >> j) & 1u) ? -1.f : 1.f);
  }
}

}  // namespace

extern "C" int tlx_iq3xxs_dequant(const void* w, const float* gridf, void* out, int64_t rows,
                                  int64_t kdim, int layout, int out_f16, void* stream) {
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255), TLX_E_ARG);
  TLX_RET_IF(layout != TLX_LAYOUT_RAW && layout != TLX_LAYOUT_PACKED, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(out, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  const int nb = (int)(kdim >> 8);
  const int64_t nchunk = rows * nb * 32;
  const int64_t grid = (nchunk + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  iq3_dequant_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)w, gridf, out, rows, nb, layout, out_f16);
  return tlx_launch_status();
}

extern "C" int tlx_ffn8(const void* wg, const void* wu, const float* gridf, const uint16_t* hhx_f16,
                        uint16_t* gact_f16, int M, int N, int K, int layout, void* stream) {
  Iq3Launch a{};
  int rc = iq3_flags(layout, TLX_OUT_TILEORD | TLX_IN_TILEORD, a);
  if (rc == TLX_OK) rc = iq3_check(wg, M, N, K, layout);
  if (rc == TLX_OK) rc = iq3_check(wu, M, N, K, layout);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(a.otile && (layout != TLX_LAYOUT_TILED || (N & 7)), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(hhx_f16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  a.seg[0] = Iq3Seg{(const uint8_t*)wg, (const uint8_t*)wu, gact_f16, nullptr, N, 0};
  a.layout = layout;
  a.nseg = 1;
  a.gridf = gridf;
  a.x = (const _Float16*)hhx_f16;
  a.M = M;
  a.K = K;
  return iq3_launch<2, EPI_SWIGLU>(a, tiles_of(N), (hipStream_t)stream);
}

// ------------------------------------------------------------------ ffn8 that allocates nothing
// tlx_ffn8_noalloc runs tlx_ffn8's kernels on this file's own scratch instead of an attached
// workspace: `scratch` is a file-scope device array with the GEMV workspace's base regions
// (kWsBaseBytes, about 3 MB; no k-split region, which only single-matrix GEMVs use), one copy per
// device, held until the process ends.  In host code the array's name
// is not a device address: the address is looked up once per device (hipGetSymbolAddress, with
// the device current) and only that pointer is passed to kernels.
namespace {

__device__ __align__(256) uint8_t scratch[kWsBaseBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];   // per-device address of `scratch`

}  // namespace

// The current device's address of `scratch` (resolved on the first use on a device; also called
// by tlx_attach_workspace, the library's set-up call).
int tlx_scratch_init(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TLX_E_NODEV;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* q = nullptr;
    const hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
    if (e != hipSuccess || q == nullptr) return e != hipSuccess ? (int)e : TLX_E_NODEV;
    g_scratch_ptr[dev] = q;
  }
  if (ptr != nullptr) *ptr = g_scratch_ptr[dev];
  return TLX_OK;
}

extern "C" int tlx_ffn8_noalloc(const void* wg, const void* wu, const float* gridf, const uint16_t* hhx_f16,
                                uint16_t* gact_f16, int M, int N, int K, int layout, void* stream) {
  int rc = iq3_check(wg, M, N, K, layout);
  if (rc == TLX_OK) rc = iq3_check(wu, M, N, K, layout);
  TLX_RET_IF(rc != TLX_OK, rc);
  // the scratch's activation-copy region holds K * 32 bytes: K <= 65536
  TLX_RET_IF((size_t)K * 16 * 2 > kWsXtBytes, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(hhx_f16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  void* ws = nullptr;
  rc = tlx_scratch_init(&ws);
  TLX_RET_IF(rc != TLX_OK, rc);
  // the scratch keeps the last call's contents: the arrival counters start this call at zero
  rc = tlx_ws_clear_counters(ws, (hipStream_t)stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  Iq3Launch a{};
  a.seg[0] = Iq3Seg{(const uint8_t*)wg, (const uint8_t*)wu, gact_f16, nullptr, N, 0};
  a.layout = layout;
  a.nseg = 1;
  a.gridf = gridf;
  a.x = (const _Float16*)hhx_f16;
  a.M = M;
  a.K = K;
  a.ws = ws;
  a.noks = 1;
  return iq3_launch<2, EPI_SWIGLU>(a, tiles_of(N), (hipStream_t)stream);
}

extern "C" int tlx_ffn8_hh(const void* wg, const void* wu, const float* gridf, const float* x,
                           const uint16_t* attn_out, const float* nw2, float* hh, uint16_t* hhx_f16,
                           uint16_t* gact_f16, int M, int N, int K, int layout, void* stream) {
  int rc = iq3_check(wg, M, N, K, layout);
  if (rc == TLX_OK) rc = iq3_check(wu, M, N, K, layout);
  if (rc == TLX_OK) rc = attn_out == nullptr || hh == nullptr ? TLX_E_ARG : tlx_rms_check(x, attn_out, nw2, hh, hhx_f16, M, K);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gridf, 16), TLX_E_ALIGN);
  Iq3Launch a{};
  a.seg[0] = Iq3Seg{(const uint8_t*)wg, (const uint8_t*)wu, gact_f16, nullptr, N, 0};
  a.layout = layout;
  a.nseg = 1;
  a.gridf = gridf;
  a.x = (const _Float16*)hhx_f16;
  a.M = M;
  a.K = K;
  _Float16* xt = nullptr;
  const bool staged = layout == TLX_LAYOUT_TILED && tlx_iq3s_stages_x(2, M, N, K, 1, true);
  rc = tlx_workspace(&a.ws);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(layout == TLX_LAYOUT_TILED && a.ws == nullptr, TLX_E_NOWS);
  if (!staged && a.ws != nullptr && M >= kXtMinM && (size_t)K * 16 * 2 <= kWsXtBytes) {   // the producer writes the GEMV's copy
    xt = reinterpret_cast<_Float16*>(static_cast<uint8_t*>(a.ws) + kWsXtOff);
    a.x = xt;
    a.xt = 1;
  }
  rc = tlx_rms_launch(true, x, attn_out, nw2, hh, hhx_f16, xt, M, K, (hipStream_t)stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  return iq3_launch<2, EPI_SWIGLU>(a, tiles_of(N), (hipStream_t)stream);
}

extern "C" int tlx_down8(const void* wd, const float* gridf, const uint16_t* gact_f16,
                         const float* hh, float* y, int M, int N, int K, int layout, void* stream) {
  Iq3Launch a{};
  int rc = iq3_flags(layout, TLX_IN_TILEORD, a);
  if (rc == TLX_OK) rc = iq3_check(wd, M, N, K, layout);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(!tlx_aligned(gact_f16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  a.seg[0] = Iq3Seg{(const uint8_t*)wd, nullptr, y, hh, N, 0};
  a.layout = layout;
  a.nseg = 1;
  a.gridf = gridf;
  a.x = (const _Float16*)gact_f16;
  a.M = M;
  a.K = K;
  return iq3_launch<1, EPI_RESID>(a, tiles_of(N), (hipStream_t)stream);
}

extern "C" int tlx_iq3_gemv(const void* w, const float* gridf, const uint16_t* x_f16,
                            uint16_t* out_f16, int M, int N, int K, int layout, void* stream) {
  Iq3Launch a{};
  int rc = iq3_flags(layout, TLX_OUT_TILEORD | TLX_IN_TILEORD, a);
  if (rc == TLX_OK) rc = iq3_check(w, M, N, K, layout);
  TLX_RET_IF(rc != TLX_OK, rc);
  TLX_RET_IF(a.otile && (layout != TLX_LAYOUT_TILED || (N & 7)), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(x_f16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  a.seg[0] = Iq3Seg{(const uint8_t*)w, nullptr, out_f16, nullptr, N, 0};
  a.layout = layout;
  a.nseg = 1;
  a.gridf = gridf;
  a.x = (const _Float16*)x_f16;
  a.M = M;
  a.K = K;
  return iq3_launch<1, EPI_F16>(a, tiles_of(N), (hipStream_t)stream);
}

// IQ3_XXS segments of the fused attention projections (tlx_attn.hip): up to three matrices
// sharing the activations, one launch.  With launch == false only the arguments are checked.
int tlx_iq3_segments(const void* const* w, uint16_t* const* out, const int* n, int nseg,
                     const float* gridf, const uint16_t* xh_f16, int M, int K, int layout,
                     bool launch, void* stream) {
  TLX_RET_IF(nseg < 1 || nseg > 4, TLX_E_ARG);
  for (int i = 0; i < nseg; ++i) {
    const int rc = iq3_check(w[i], M, n[i], K, layout);
    TLX_RET_IF(rc != TLX_OK, rc);
  }
  TLX_RET_IF(!tlx_aligned(xh_f16, 16) || !tlx_aligned(gridf, 16), TLX_E_ALIGN);
  if (layout == TLX_LAYOUT_TILED) {   // checked before any launch of the fused projections
    void* ws = nullptr;
    const int rc = tlx_workspace(&ws);
    TLX_RET_IF(rc != TLX_OK, rc);
    TLX_RET_IF(ws == nullptr, TLX_E_NOWS);
  }
  if (!launch) return TLX_OK;
  Iq3Launch a{};
  int tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    a.seg[i] = Iq3Seg{(const uint8_t*)w[i], nullptr, out[i], nullptr, n[i], tiles};
    tiles += tiles_of(n[i]);
  }
  a.nseg = nseg;
  a.gridf = gridf;
  a.x = (const _Float16*)xh_f16;
  a.M = M;
  a.K = K;
  a.layout = layout;
  return iq3_launch<1, EPI_F16>(a, tiles, (hipStream_t)stream);
}

// Up to four IQ3_XXS matrices sharing the activations, fp16 out, one launch.
extern "C" int tlx_iq3_gemv_multi(const void* const* w, uint16_t* const* out, const int* n, int nseg,
                                  const float* gridf, const uint16_t* x_f16, int M, int K, int layout,
                                  void* stream) {
  TLX_RET_IF(w == nullptr || out == nullptr || n == nullptr, TLX_E_ARG);
  const int rc = tlx_iq3_segments(w, out, n, nseg, gridf, x_f16, M, K, layout, false, stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  return tlx_iq3_segments(w, out, n, nseg, gridf, x_f16, M, K, layout, true, stream);
}
