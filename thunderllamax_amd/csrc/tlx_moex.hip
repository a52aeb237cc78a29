// MoE expert GEMMs for the weight classes of the reference's real checkpoint (its Qwen3.6-35B-A3B
// GGUF mix): IQ3_S routed gate/up (gxu_gm, engine/mm/MM_E_gxu_gm.cu:86-93; pair walk gx8e256up,
// engine/mm/MM_P1_gx8e256up.cu:15-20), Q6_K routed down (gxm_dn6, engine/mm/MM_B_gxm_dn6.cu:18-25;
// pair walk gx8e256dn6, engine/mm/MM_P2_gx8e256dn6.cu:9-13), the Q8_0 shared expert (shexp8,
// engine/mm/MM_P2_shexp8.cu:8-13), and bit-exact IQ3_S / Q8_0 dequantizers.
//
// Slabs as the reference's: expert e's IQ3_S gate/up slab at ptbl[e] -- 512 gate rows, then 512 up
// rows 450,560 B in (GATE_B), 880 B a row (8 blocks of 110 B, k = 2048); its Q6_K down slab at
// ptbl_dn[e] -- 2048 rows of 420 B (2 raw 210-B blocks, k = 512); the shared expert's Q8_0 gate and
// up rows (512 x 2176 B, k = 2048) and down rows (2048 x 544 B, k = 512).
//
// Three kernels.  gx_kernel (batches: gate+up, the shared expert's down, and the routed down where
// parts is not 8-B aligned): a workgroup owns 16 output columns per wave of one expert -- gate+up:
// 4 waves, 64 gate rows and the matching 64 up rows, so the SwiGLU pairs meet in one lane; down: 8
// waves, 128 rows -- and the token rows a pass at a time (128 sorted, 64 dense).  K runs in chunks
// of 64: the pass's activations (f32 -> fp16, round to nearest even) and the column block's weight
// rows, dequantized to the reference's operands -- fp16 of the fp32 GGUF value, as gxu_gm stages them -- go to LDS
// (rows padded to 72 halfs: the 16 rows of a fragment read fall in distinct 16-B slots); then wave
// w runs v_mfma_f32_16x16x32_f16 over its 16 columns for every 16-token group of the pass.  Token
// lists: sorted (the expert's bin from eoff / plist, in passes of 128) or dense (every position:
// the shared expert).  gv_kernel (decode: the pair walk, one pair per item, pair p running expert
// eids[p]; the shared expert at P <= 16): the same operands, built in registers (its section).
// gq_dn_kernel (the routed down over the sorted pairs): gv_kernel's register-built operands with
// the expert's activations resident in LDS (its section).
//
// Every routed form also reads tiled slabs (layout TLX_LAYOUT_TILED; tlx_pack_iq3s_tiled /
// tlx_pack_q6k_tiled, this library's own): the same bytes regrouped per 16-row tile and 256-weight
// block so that a lane's bytes of each field are one contiguous run; only the fetches differ.
//
// IQ3_S's 512-entry grid is a run-time argument (float[512][4]), as in the reference.
#include "tlx_common.h"

namespace {

constexpr int kHid = 2048, kFf = 512, kE = 256, kMaxPairs = 16384;
// waves per staged-form workgroup, 16 output columns each (measured at M = 2048: gate+up 4 / 8 /
// 16 waves 313 / 332 / 409 us; down 235 / 204 / 267 us)
template <bool UP> constexpr int gx_waves() { return UP ? 4 : 8; }
constexpr int kGxKc = 64;           // k per chunk (LDS stage)
constexpr int kGxLd = kGxKc + 8;    // LDS row stride (halfs): fragment reads of 16 rows hit 16 distinct 16-B slots
constexpr uint32_t kIq3sGate = kFf * 880;   // GATE_B: the up rows' offset in an IQ3_S slab
constexpr int kIq3sRow = kHid / 256 * 110;   // 880 B: an IQ3_S gate/up row (k = 2048)
constexpr int kQ6kRow = kFf / 256 * 210;     // 420 B: a Q6_K down row (k = 512)

enum GxCls { GX_IQ3S = 0, GX_Q6K = 1, GX_Q80 = 2 };
enum GxForm { GX_SORTED = 0, GX_PAIRS = 1, GX_DENSE = 2 };

template <int CLS> struct GxFmt;   // bytes per block, weights per block
template <> struct GxFmt<GX_IQ3S> { static constexpr int kBlk = 110, kPer = 256; };
template <> struct GxFmt<GX_Q6K> { static constexpr int kBlk = 210, kPer = 256; };
template <> struct GxFmt<GX_Q80> { static constexpr int kBlk = 34, kPer = 32; };

// token rows per pass of gx_kernel: 128 for the sorted pairs (an expert's pairs in one pass at
// M = 2048, so its weights are dequantized once: gate+up 317 -> 296 us, down 207 -> 180 us), 64
// for the dense form (the shared expert: twice the items to spread over the CUs)
template <int FORM> constexpr int gx_tok() { return FORM == GX_SORTED ? 128 : 64; }

struct GxArgs {
  const uint64_t* ptbl;    // routed: slab address per expert
  const uint8_t* w0;       // dense: gate rows (gate+up) or down rows
  const uint8_t* w1;       // dense gate+up: up rows
  const uint16_t* eids;    // pair walk: expert of each pair
  const int* eoff;         // sorted: bin offsets [E + 1]
  const uint16_t* plist;   // sorted: pair ids in bin order
  const float* x;          // gate+up: f32 [P][2048] (routed: row pair >> 3); down: f32 [pairs or P][512]
  const float* grid;       // IQ3_S grid f32 [512][4]
  void* out;               // gate+up: f32 [pairs or P][512]; down: f16 [pairs][2048] or (dense) f32 [P][2048]
  int P;
  int items;               // work items: experts (sorted), pairs (pair walk) or 64-position passes (dense)
};


// The decode form reads weight bytes through global-address-space pointers: global loads count on
// the vector-memory counter only (flat loads also on the LDS one, so a wait for an LDS read waits
// for the weight loads in flight too).  The LDS-staged form keeps generic pointers: measured, its
// flat loads run the M = 2048 gate+up faster (313 vs 350 us), the down alike.  Records are only
// 2-B aligned (110-, 210- and 34-B blocks): gx_ld reads through an under-aligned type.
using gbyte = const __attribute__((address_space(1))) uint8_t;

template <typename T>
__device__ __forceinline__ T gx_ld(gbyte* p) {
  typedef T __attribute__((aligned(1))) T1;
  return *reinterpret_cast<const __attribute__((address_space(1))) T1*>(p);
}

// The 16 weights k0 .. k0 + 15 (k0 % 16 == 0) of one row as f32 GGUF values, in two steps: fetch
// (the raw bytes into registers, so a chunk's loads can be issued a chunk ahead) and decode.
// IQ3_S (MM_P0_d2_repack.py:95-120): sub-block j = kib / 32 (db = d (1 + 2 nib)), half hf: index
// bytes qs[8j + 4hf ..], high bits 4hf .. of qh[j], sign bytes signs[4j + 2hf ..].
// Q6_K raw block (210 B: ql[128] qh[64] sc[16] d): half h = kib / 128, quarter g, l0 = 0 or 16:
// (d * sc[8h + l0/16 + 2g]) * (q - 32), q = ql nibble | 2 qh bits << 4 (MM_P2_ports.py:21-45).
// Q8_0 block (34 B: d, q i8[32]), half (k0 / 16) & 1: d * q (exact in fp32).
// the fetches' loads: global address space (they then wait on the vector-memory counter only; a
// flat load also counts in the LDS counter, so every LDS wait would wait for the weights in flight;
// measured: the M = 2048 sorted gate+up 262.7 -> 259.2 us)
template <typename T>
__device__ __forceinline__ T gx_ldf(const uint8_t* p) {
  return gx_ld<T>((gbyte*)p);
}

template <int CLS> struct GxRaw;
template <> struct GxRaw<GX_IQ3S> { uint32_t dn, qs, hs; };   // d | nib << 16, index bytes, qh nibble | signs << 8
template <> struct GxRaw<GX_Q6K> { uint32_t ds; u4_t ql, qh; };   // d | sc << 16 | (kib & 255) << 24
template <> struct GxRaw<GX_Q80> { uint32_t d; u4_t q; };

// TL: the slab is in the tiled layout (records of 16 rows x 256 weights; tlx_pack_iq3s_tiled /
// tlx_pack_q6k_tiled), rowp still the row's start as if in GGUF rows (a tile spans the same bytes),
// col the row's place in its 16-row tile.
template <int CLS, bool TL = false>
__device__ __forceinline__ GxRaw<CLS> gx_fetch(const uint8_t* rowp, int k0, int col = 0) {
  // an opaque copy of the row pointer: the loads below then take their field offsets as
  // immediates on one address (measured: the M = 2048 gate+up 327 -> 313 us)
  uint64_t pv = (uint64_t)rowp;
  asm volatile("" : "+v"(pv));
  const uint8_t* row = (const uint8_t*)pv;
  GxRaw<CLS> r;
  if constexpr (TL && CLS == GX_IQ3S) {
    // record (tile, block): lane l = 16 kq + col's 16 index bytes at 16 l, 8 sign bytes at
    // 1024 + 8 l, 2 high-bit bytes at 1536 + 2 l, scale byte at 1664 + l; d at 1728 + 2 col
    const uint8_t* rec = row - (size_t)col * kIq3sRow + (size_t)(k0 >> 8) * 1760;
    const int kib = k0 & 255, kq = kib >> 6, sj = (kib >> 5) & 1, hf = (kib >> 4) & 1, l = 16 * kq + col;
    const uint32_t nib = (gx_ldf<uint8_t>(rec + 1664 + l) >> (4 * sj)) & 15u;
    r.dn = gx_ldf<uint16_t>(rec + 1728 + 2 * col) | (nib << 16);
    r.qs = gx_ldf<uint32_t>(rec + 16 * l + 8 * sj + 4 * hf);
    r.hs = ((uint32_t)(gx_ldf<uint8_t>(rec + 1536 + 2 * l + sj) >> (4 * hf)) & 15u) |
           ((uint32_t)gx_ldf<uint16_t>(rec + 1024 + 8 * l + 4 * sj + 2 * hf) << 8);
  } else if constexpr (TL && CLS == GX_Q6K) {
    // record (tile, block): lane l = 16 kq + col's 32 low bytes at 32 l; row col's high bytes of
    // half h at 2048 + 32 (16 h + col); lane l's 4 scale bytes at 3072 + 4 l; d at 3328 + 2 col
    const uint8_t* rec = row - (size_t)col * kQ6kRow + (size_t)(k0 >> 8) * 3360;
    const int kib = k0 & 255, h = kib >> 7, g = (kib >> 5) & 3, l0 = kib & 31;
    const int bs = 2 * g + (l0 >> 4);   // scale byte 8 h + bs: lane kq 2 h + ((bs >> 1) & 1), slot below
    const int ls = 16 * (2 * h + ((bs >> 1) & 1)) + col;
    r.ds = gx_ldf<uint16_t>(rec + 3328 + 2 * col) | ((uint32_t)gx_ldf<uint8_t>(rec + 3072 + 4 * ls + (bs & 1) + 2 * (bs >> 2)) << 16) |
           ((uint32_t)kib << 24);
    r.ql = gx_ldf<u4_t>(rec + 32 * (16 * (2 * h + (g & 1)) + col) + l0);
    r.qh = gx_ldf<u4_t>(rec + 2048 + 32 * (16 * h + col) + l0);
  } else if constexpr (CLS == GX_IQ3S) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 110;
    const int kib = k0 & 255, j = kib >> 5, hf = (kib >> 4) & 1;
    const uint32_t nib = (gx_ldf<uint8_t>(b + 106 + (j >> 1)) >> (4 * (j & 1))) & 15u;
    r.dn = gx_ldf<uint16_t>(b) | (nib << 16);
    r.qs = gx_ldf<uint32_t>(b + 2 + 8 * j + 4 * hf);
    r.hs = ((uint32_t)(gx_ldf<uint8_t>(b + 66 + j) >> (4 * hf)) & 15u) | ((uint32_t)gx_ldf<uint16_t>(b + 74 + 4 * j + 2 * hf) << 8);
  } else if constexpr (CLS == GX_Q6K) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 210;
    const int kib = k0 & 255, h = kib >> 7, g = (kib >> 5) & 3, l0 = kib & 31;
    r.ds = gx_ldf<uint16_t>(b + 208) | ((uint32_t)gx_ldf<uint8_t>(b + 192 + 8 * h + (l0 >> 4) + 2 * g) << 16) | ((uint32_t)kib << 24);
    r.ql = gx_ldf<u4_t>(b + 64 * h + 32 * (g & 1) + l0);
    r.qh = gx_ldf<u4_t>(b + 128 + 32 * h + l0);
  } else {
    const uint8_t* b = row + (size_t)(k0 >> 5) * 34;
    r.d = gx_ldf<uint16_t>(b);
    r.q = gx_ldf<u4_t>(b + 2 + 16 * ((k0 >> 4) & 1));
  }
  return r;
}

template <int CLS>
__device__ __forceinline__ void gx_decode(float* v, const GxRaw<CLS>& r, const float4* grid) {
  if constexpr (CLS == GX_IQ3S) {
    const float db = tlx_h2f((uint16_t)(r.dn & 0xFFFFu)) * (float)(1u + 2u * (r.dn >> 16));   // exact
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // index byte i: weights 4i .. 4i+3
      const uint32_t idx = ((r.qs >> (8 * i)) & 255u) | (((r.hs >> i) & 1u) << 8);
      const float4 g = grid[idx];
      const uint32_t sg = r.hs >> (8 + 4 * i);
      const float gv[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float w = db * gv[c];
        v[4 * i + c] = ((sg >> c) & 1u) ? -w : w;
      }
    }
  } else if constexpr (CLS == GX_Q6K) {
    const float t = tlx_h2f((uint16_t)(r.ds & 0xFFFFu)) * (float)(int8_t)(uint8_t)(r.ds >> 16);
    const int g = (int)(r.ds >> 29) & 3;   // (kib >> 5) & 3
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      const uint32_t lb = (r.ql[l >> 2] >> (8 * (l & 3))) & 255u, hb = (r.qh[l >> 2] >> (8 * (l & 3))) & 255u;
      const int lo = (g >> 1) ? (int)(lb >> 4) : (int)(lb & 15u);
      const int q = lo | (int)(((hb >> (2 * g)) & 3u) << 4);
      v[l] = t * (float)(q - 32);
    }
  } else {
    const float d = tlx_h2f((uint16_t)r.d);
#pragma unroll
    for (int l = 0; l < 16; ++l) v[l] = d * (float)(int8_t)(uint8_t)(r.q[l >> 2] >> (8 * (l & 3)));
  }
}

// IQ3_S lookups for the fp16 operands, in LDS: the grid as fp16 (4 halves an entry, 8 B -- exact for
// the IQ3_S grid's integer levels; other values take one extra rounding, to fp16, before the
// product) and the fp16 sign masks of 4 weights per sign nibble (16 entries: all in distinct
// banks, so a wave's lookups do not conflict)
struct GvLut {
  uint2 grid[512];
  uint2 smask[16];
};

template <bool G> struct GvLutSlot { GvLut v; };
template <> struct GvLutSlot<false> {};

template <int NT>
__device__ __forceinline__ void gv_lut_fill(GvLut& L, const float* gridf, int t) {
  for (int i = t; i < 512; i += NT) {
    const float4 g = reinterpret_cast<const float4*>(gridf)[i];
    L.grid[i] = uint2{(uint32_t)tlx_f2h_bits(g.x) | ((uint32_t)tlx_f2h_bits(g.y) << 16),
                      (uint32_t)tlx_f2h_bits(g.z) | ((uint32_t)tlx_f2h_bits(g.w) << 16)};
  }
  if (t < 16)
    L.smask[t] = uint2{((t & 1u) << 15) | (((t >> 1) & 1u) << 31), (((t >> 2) & 1u) << 15) | (((t >> 3) & 1u) << 31)};
}

// The 16 weights as fp16 operands, bit for bit the fp16 of gx_decode's values: the products of a
// block scale and an integer level are exact in f32 for all three classes (IQ3_S: fp16 d times
// 1 + 2 nib times a level <= 15, <= 20 bits; Q8_0: d times an int8, <= 19; Q6_K: d times an int8
// scale times q - 32, <= 23), so v_fma_mix's one rounding to fp16 is the reference's.
template <int CLS>
__device__ __forceinline__ void gx_decode_h(u4_t* h, const GxRaw<CLS>& r, const GvLut* lut) {
  if constexpr (CLS == GX_IQ3S) {
    const float db = tlx_h2f((uint16_t)(r.dn & 0xFFFFu)) * (float)(1u + 2u * (r.dn >> 16));   // exact
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // index byte i: weights 4i .. 4i+3
      const uint2 g = lut->grid[((r.qs >> (8 * i)) & 255u) | (((r.hs >> i) & 1u) << 8)];
      const uint2 m = lut->smask[(r.hs >> (8 + 4 * i)) & 15u];
      h[i >> 1][2 * (i & 1)] = tlx_mix2_f16(db, g.x) ^ m.x;
      h[i >> 1][2 * (i & 1) + 1] = tlx_mix2_f16(db, g.y) ^ m.y;
    }
  } else if constexpr (CLS == GX_Q80) {
    const float d = tlx_h2f((uint16_t)r.d);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u4 = r.q[j] ^ 0x80808080u;   // int8 + 128
      h[j >> 1][2 * (j & 1)] = tlx_mix2_f16(d, tlx_bytes_h2(u4, 0, 128.f));
      h[j >> 1][2 * (j & 1) + 1] = tlx_mix2_f16(d, tlx_bytes_h2(u4, 1, 128.f));
    }
  } else {   // Q6_K: t = d * sc, weights l = 0 .. 15 of quarter g
    const float t = tlx_h2f((uint16_t)(r.ds & 0xFFFFu)) * (float)(int8_t)(uint8_t)(r.ds >> 16);
    const uint32_t g = (r.ds >> 29) & 3u;   // (kib >> 5) & 3
    const uint32_t nsh = (g >> 1) * 4u, hsh = 2u * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t q4 = ((r.ql[j] >> nsh) & 0x0F0F0F0Fu) | (((r.qh[j] >> hsh) & 0x03030303u) << 4);
      h[j >> 1][2 * (j & 1)] = tlx_mix2_f16(t, tlx_bytes_h2(q4, 0, 32.f));   // t * (q - 32)
      h[j >> 1][2 * (j & 1) + 1] = tlx_mix2_f16(t, tlx_bytes_h2(q4, 1, 32.f));
    }
  }
}

template <bool UP, bool GRID, int TOK>
struct alignas(16) GxLds {   // 16-B fragment reads and stores
  _Float16 x[TOK * kGxLd];
  _Float16 w[(UP ? 2 : 1) * 16 * gx_waves<UP>() * kGxLd];
  GvLutSlot<GRID> lut;
  int xrow[TOK];
  int orow[TOK];
};

template <int CLS>
__device__ __forceinline__ void gx_dequant16(float* v, const uint8_t* row, int k0, const float4* grid) {
  gx_decode<CLS>(v, gx_fetch<CLS>(row, k0), grid);
}

// blk: the workgroup's index in its part of the grid (parts start at multiples of 8); L: any
// GxLds<UP, *, >= gx_tok<FORM>()> that holds the IQ3_S lookups when CLS needs them
template <int CLS, bool UP, int FORM, bool TL, typename LDS>
__device__ __forceinline__ void gx_body(LDS& L, const GxArgs& a, int blk) {
  constexpr int K = UP ? kHid : kFf;
  constexpr int NW = gx_waves<UP>(), NT = 64 * NW, CO = 16 * NW;   // waves, threads, output columns
  constexpr int NR = (UP ? 2 : 1) * CO;                   // staged weight rows
  constexpr int RB = (UP ? kFf : kHid) / CO;              // column blocks per matrix
  constexpr int ROWB = K / GxFmt<CLS>::kPer * GxFmt<CLS>::kBlk;
  constexpr bool GRID = CLS == GX_IQ3S;
  constexpr int TOK = gx_tok<FORM>();
  static_assert(sizeof(L.xrow) / sizeof(int) >= TOK, "LDS token rows");
  static_assert(FORM != GX_PAIRS, "the pair walk is gv_kernel's");
  constexpr int NG = TOK / 16;                            // 16-token MFMA groups per pass
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, col = lane & 15, kq = lane >> 4;
  // Workgroups go to the 8 XCDs round robin (block b to XCD b % 8), each XCD with its own L2.  The RB
  // column blocks of one item are all placed on one XCD, so the item's activation rows -- read by
  // every column block -- come from HBM once and from that XCD's L2 after.
  const int slot = blk >> 3;
  const int rb = slot % RB, item = slot / RB * 8 + (blk & 7);
  if (item >= a.items) return;   // the grid is padded to a multiple of 8 items

  // the work item: token list, weight matrices
  int beg = 0, ntot = 0;
  const uint8_t* wg = nullptr;
  const uint8_t* wu = nullptr;
  if constexpr (FORM == GX_SORTED) {
    beg = a.eoff[item];
    ntot = a.eoff[item + 1] - beg;
    if (ntot <= 0) return;   // uniform per workgroup
    wg = reinterpret_cast<const uint8_t*>(a.ptbl[item]);
  } else {
    beg = item * TOK;
    ntot = min(TOK, a.P - beg);
    wg = a.w0;
  }
  if constexpr (UP) wu = FORM == GX_DENSE ? a.w1 : wg + kIq3sGate;
  const GvLut* lut = nullptr;
  if constexpr (GRID) {
    gv_lut_fill<NT>(L.lut.v, a.grid, t);
    lut = &L.lut.v;
  }

  for (int p0 = 0; p0 < ntot; p0 += TOK) {
    const int nt = min(TOK, ntot - p0);
    const int ng = (nt + 15) >> 4;
    __syncthreads();   // the previous pass is done with the token rows
    if (t < TOK) {
      int xr = -1, orw = -1;
      if (t < nt) {
        const int pr = FORM == GX_SORTED ? (int)a.plist[beg + p0 + t] : beg + p0 + t;   // pair or position
        orw = pr;
        xr = (UP && FORM != GX_DENSE) ? (pr >> 3) : pr;
      }
      L.xrow[t] = xr;
      L.orow[t] = orw;
    }
    f4_t acc[NG][UP ? 2 : 1];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int m = 0; m < (UP ? 2 : 1); ++m) acc[g][m] = f4_t{0.f, 0.f, 0.f, 0.f};

    // the thread's weight units (staged row R, 16-weight piece q) and activation pieces
    constexpr int NU = NR * (kGxKc / 16) / NT;       // units per thread (1 or 2)
    constexpr int NX = (TOK * kGxKc / 8 + NT - 1) / NT;   // activation pieces per thread
    static_assert(NR * (kGxKc / 16) % NT == 0, "units");
    const uint8_t* urow[NU];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int R = (t + i * NT) >> 2;
      urow[i] = ((UP && R >= CO) ? wu : wg) + (size_t)(rb * CO + (R & (CO - 1))) * ROWB;
    }
    GxRaw<CLS> raw[NU];
    float4 xv[NX][2];
    // the activations' source rows for this thread's pieces (row 0 stands in past the pass: loaded,
    // then replaced by zeros, so the loads stay unconditional)
    int xo[NX];
    bool xz[NX];
    __syncthreads();   // the token rows are visible
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int pc = t + i * NT;
      const int xr = pc < TOK * kGxKc / 8 ? L.xrow[pc >> 3] : -1;
      xz[i] = xr < 0;
      xo[i] = (xr < 0 ? 0 : xr) * K + 8 * (pc & 7);
    }
#define GX_FETCH(KC)                                                                                 \
  {                                                                                                  \
    _Pragma("unroll") for (int i = 0; i < NU; ++i)                                                   \
      raw[i] = gx_fetch<CLS, TL>(urow[i], (KC) * kGxKc + 16 * ((t + i * NT) & 3), ((t + i * NT) >> 2) & 15); \
    _Pragma("unroll") for (int i = 0; i < NX; ++i) {                                                 \
      const float4* src = reinterpret_cast<const float4*>(a.x + (size_t)xo[i] + (KC) * kGxKc);       \
      xv[i][0] = src[0];                                                                             \
      xv[i][1] = src[1];                                                                             \
    }                                                                                                \
  }
    // gate+up (32 chunks): the next chunk's loads are issued before this chunk's MFMAs; down (8
    // chunks): measured faster without (the prefetch registers cost occupancy)
    constexpr bool PIPE = K / kGxKc > 8;
    if constexpr (PIPE) GX_FETCH(0)
    for (int kc = 0; kc < K / kGxKc; ++kc) {
      if constexpr (!PIPE) GX_FETCH(kc)
      __syncthreads();   // the previous chunk's fragment reads are done
#pragma unroll
      for (int i = 0; i < NX; ++i) {
        const int pc = t + i * NT;
        if (pc < 16 * ng * (kGxKc / 8)) {   // the pass's 16-token groups only (the MFMAs read no other row)
          const float4 z = float4{0.f, 0.f, 0.f, 0.f};
          const float4 u = xz[i] ? z : xv[i][0], w = xz[i] ? z : xv[i][1];
          const h8_t h = {(_Float16)u.x, (_Float16)u.y, (_Float16)u.z, (_Float16)u.w,
                          (_Float16)w.x, (_Float16)w.y, (_Float16)w.z, (_Float16)w.w};
          *reinterpret_cast<h8_t*>(L.x + (pc >> 3) * kGxLd + 8 * (pc & 7)) = h;
        }
      }
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = t + i * NT;
        u4_t h[2];
        gx_decode_h<CLS>(h, raw[i], lut);
        *reinterpret_cast<u4_t*>(L.w + (u >> 2) * kGxLd + 16 * (u & 3)) = h[0];
        *reinterpret_cast<u4_t*>(L.w + (u >> 2) * kGxLd + 16 * (u & 3) + 8) = h[1];
      }
      if constexpr (PIPE) {
        if (kc + 1 < K / kGxKc) GX_FETCH(kc + 1)   // in flight over this chunk's MFMAs
      }
      __syncthreads();
#pragma unroll
      for (int s = 0; s < kGxKc / 32; ++s) {
        const int ko = 32 * s + 8 * kq;
        const h8_t bg = *reinterpret_cast<const h8_t*>(L.w + (16 * wave + col) * kGxLd + ko);
        h8_t bu;
        if constexpr (UP) bu = *reinterpret_cast<const h8_t*>(L.w + (CO + 16 * wave + col) * kGxLd + ko);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g < ng) {
            const h8_t ax = *reinterpret_cast<const h8_t*>(L.x + (16 * g + col) * kGxLd + ko);
            acc[g][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bg, acc[g][0], 0, 0, 0);
            if constexpr (UP) acc[g][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bu, acc[g][1], 0, 0, 0);
          }
        }
      }
    }
    // lane (col, kq) holds tokens 16 g + 4 kq + r of output column rb * 64 + 16 wave + col
    const int n = rb * CO + 16 * wave + col;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g >= ng) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = 16 * g + 4 * kq + r;
        if (tk >= nt) continue;
        const size_t o = (size_t)L.orow[tk];
        if constexpr (UP) {
          const float gv = acc[g][0][r], uv = acc[g][1][r];
          reinterpret_cast<float*>(a.out)[o * kFf + n] = gv / (1.f + expf(-gv)) * uv;
        } else if constexpr (FORM == GX_DENSE) {
          reinterpret_cast<float*>(a.out)[o * kHid + n] = acc[g][0][r];
        } else {
          reinterpret_cast<_Float16*>(a.out)[o * kHid + n] = (_Float16)acc[g][0][r];
        }
      }
    }
  }
}

#undef GX_FETCH

template <int CLS, bool UP, int FORM, bool TL>
__global__ __launch_bounds__(64 * gx_waves<UP>()) void gx_kernel(const GxArgs a) {
  __shared__ GxLds<UP, CLS == GX_IQ3S, gx_tok<FORM>()> L;
  gx_body<CLS, UP, FORM, TL>(L, a, (int)blockIdx.x);
}

// The sorted form (class RCLS) and the Q8_0 shared expert's dense form in one launch: workgroups
// below nra run the routed experts (args a), the rest the shared expert (args b) -- each part its
// own launch's code, so the outputs are the separate launches' bit for bit.  The shared expert's
// workgroups come last, filling the routed grid's last round.
template <int RCLS, bool UP, bool TL>
__global__ __launch_bounds__(64 * gx_waves<UP>()) void gx_sh_kernel(const GxArgs a, const GxArgs b, int nra) {
  __shared__ GxLds<UP, RCLS == GX_IQ3S, gx_tok<GX_SORTED>()> L;   // the larger pass
  const int blk = (int)blockIdx.x;
  if (blk < nra)
    gx_body<RCLS, UP, GX_SORTED, TL>(L, a, blk);
  else
    gx_body<GX_Q80, UP, GX_DENSE, false>(L, b, blk - nra);   // the shared expert: GGUF rows
}

// ------------------------------------------------------------------ decode form (GEMV-shaped)
// Items of at most 16 tokens -- the pair walk (one token a pair) and the shared expert at P <= 16
// -- bypass the LDS weight stage: a 16-row tile (gate+up: the gate tile and its up tile) is walked
// by KS waves, each over K / KS of k, in units of 256 weights.  Lane (col, kq) fetches the bytes
// of row col that hold its 64 weights of a unit (contiguous in the record where the class allows)
// straight into registers, a few units ahead, and builds the B operand of each of the unit's 8
// k-steps from them.  Which 8 weights a lane feeds a step is a fixed permutation of the unit's k
// (gv_koff); the activations -- fp16 in LDS, natural k order -- are read at the same k, so the
// products and their sums are those of the LDS-staged form up to the order of the fp32 sums.
constexpr int kGvTok = 16;

template <int CLS> struct GvRaw;
template <> struct GvRaw<GX_IQ3S> { u4_t qs; uint32_t sg0, sg1, dq, sc; };    // dq: d | qh pair << 16
template <> struct GvRaw<GX_Q6K> { u4_t ql0, ql1, qh0, qh1; uint32_t sc, d; };  // sc: 4 scale bytes
template <> struct GvRaw<GX_Q80> { u4_t q0, q1, q2, q3; uint32_t d; };          // d: two blocks' d

// Lane kq's bytes of unit u of a row.
// IQ3_S (110-B block = unit): weights 64 kq .. 64 kq + 63 -- index bytes qs[16 kq ..], high bits
// qh[2 kq], qh[2 kq + 1], sign bytes signs[8 kq ..], scale byte 106 + kq (sub-blocks 2 kq, 2 kq + 1).
// Q6_K (210-B block = unit): ql bytes 32 kq .. 32 kq + 31, both nibbles (half h = kq / 2, c = kq % 2:
// weights 128 h + 32 c + l and 128 h + 64 + 32 c + l), qh bytes 32 h .. 32 h + 31, scale bytes
// 8 h + 2 c + {0, 1, 4, 5}.
// Q8_0 (8 blocks of 34 B = unit): blocks 2 kq and 2 kq + 1.
// TL: the tiled layout (row: the row's start as in GGUF rows; its place in the tile is the lane's
// col): lane l = 16 kq + col's bytes are one contiguous run of every record region.
template <int CLS, bool TL = false>
__device__ __forceinline__ GvRaw<CLS> gv_fetch(gbyte* row, int u, int kq) {
  GvRaw<CLS> r;
  if constexpr (TL && CLS == GX_IQ3S) {
    const int col = (int)threadIdx.x & 15, l = 16 * kq + col;
    gbyte* rec = row - (size_t)col * kIq3sRow + (size_t)u * 1760;
    r.qs = gx_ld<u4_t>(rec + 16 * l);
    const uint64_t sg = gx_ld<uint64_t>(rec + 1024 + 8 * l);
    r.sg0 = (uint32_t)sg;
    r.sg1 = (uint32_t)(sg >> 32);
    r.dq = gx_ld<uint16_t>(rec + 1728 + 2 * col) | ((uint32_t)gx_ld<uint16_t>(rec + 1536 + 2 * l) << 16);
    r.sc = rec[1664 + l];
  } else if constexpr (TL && CLS == GX_Q6K) {
    const int col = (int)threadIdx.x & 15, l = 16 * kq + col;
    gbyte* rec = row - (size_t)col * kQ6kRow + (size_t)u * 3360;
    r.ql0 = gx_ld<u4_t>(rec + 32 * l);
    r.ql1 = gx_ld<u4_t>(rec + 32 * l + 16);
    r.qh0 = gx_ld<u4_t>(rec + 2048 + 32 * (16 * (kq >> 1) + col));
    r.qh1 = gx_ld<u4_t>(rec + 2048 + 32 * (16 * (kq >> 1) + col) + 16);
    r.sc = gx_ld<uint32_t>(rec + 3072 + 4 * l);
    r.d = gx_ld<uint16_t>(rec + 3328 + 2 * col);
  } else if constexpr (CLS == GX_IQ3S) {
    gbyte* b = row + (size_t)u * 110;
    r.qs = gx_ld<u4_t>(b + 2 + 16 * kq);
    const uint64_t sg = gx_ld<uint64_t>(b + 74 + 8 * kq);
    r.sg0 = (uint32_t)sg;
    r.sg1 = (uint32_t)(sg >> 32);
    r.dq = gx_ld<uint16_t>(b) | ((uint32_t)gx_ld<uint16_t>(b + 66 + 2 * kq) << 16);
    r.sc = b[106 + kq];
  } else if constexpr (CLS == GX_Q6K) {
    gbyte* b = row + (size_t)u * 210;
    const int h = kq >> 1, c = kq & 1;
    r.ql0 = gx_ld<u4_t>(b + 32 * kq);
    r.ql1 = gx_ld<u4_t>(b + 32 * kq + 16);
    r.qh0 = gx_ld<u4_t>(b + 128 + 32 * h);
    r.qh1 = gx_ld<u4_t>(b + 128 + 32 * h + 16);
    r.sc = gx_ld<uint16_t>(b + 192 + 8 * h + 2 * c) | ((uint32_t)gx_ld<uint16_t>(b + 196 + 8 * h + 2 * c) << 16);
    r.d = gx_ld<uint16_t>(b + 208);
  } else {
    gbyte* b = row + (size_t)u * 272 + 68 * kq;
    r.q0 = gx_ld<u4_t>(b + 2);
    r.q1 = gx_ld<u4_t>(b + 18);
    r.q2 = gx_ld<u4_t>(b + 36);
    r.q3 = gx_ld<u4_t>(b + 52);
    r.d = gx_ld<uint16_t>(b) | ((uint32_t)gx_ld<uint16_t>(b + 34) << 16);
  }
  return r;
}

// the unit-relative k of the 8 weights lane kq feeds k-step s (they are consecutive)
template <int CLS>
__device__ __forceinline__ int gv_koff(int kq, int s) {
  if constexpr (CLS == GX_Q6K) return 128 * (kq >> 1) + 32 * (kq & 1) + 64 * (s >> 2) + 8 * (s & 3);
  return 64 * kq + 8 * s;
}

// B operand of k-step s: fp16 of the GGUF values, the product of the block scale and the integer
// level rounded to fp16 (exact in f32 for the three classes: gx_decode's operands bit for bit)
template <int CLS, int S>
__device__ __forceinline__ h8_t gv_decode(const GvRaw<CLS>& r, int kq, const GvLut* lut) {
  if constexpr (CLS == GX_IQ3S) {
    const float db = tlx_h2f((uint16_t)(r.dq & 0xFFFFu)) * (float)(1u + 2u * ((r.sc >> (4 * (S >> 2))) & 15u));
    const uint32_t qsw = r.qs[S >> 1] >> (16 * (S & 1));
    const uint32_t qh = r.dq >> (16 + 2 * S);
    const uint2 g0 = lut->grid[(qsw & 255u) | ((qh & 1u) << 8)];
    const uint2 g1 = lut->grid[((qsw >> 8) & 255u) | ((qh & 2u) << 7)];
    const uint32_t sb = (S < 4 ? r.sg0 : r.sg1) >> (8 * (S & 3));
    const uint2 m0 = lut->smask[sb & 15u], m1 = lut->smask[(sb >> 4) & 15u];
    // (each word's last write is the sign XOR, an instruction the compiler sees: no guard needed)
    const u4_t h = {tlx_mix2_f16(db, g0.x) ^ m0.x, tlx_mix2_f16(db, g0.y) ^ m0.y, tlx_mix2_f16(db, g1.x) ^ m1.x, tlx_mix2_f16(db, g1.y) ^ m1.y};
    return __builtin_bit_cast(h8_t, h);
  } else if constexpr (CLS == GX_Q6K) {
    constexpr int n = S >> 2, q = S & 3;
    const u4_t& ql = (q < 2) ? r.ql0 : r.ql1;
    const u4_t& qv = (q < 2) ? r.qh0 : r.qh1;
    const uint32_t sh = 2u * (uint32_t)(kq & 1) + 4u * n;   // the quarter's 2 high bits
    const float t = tlx_h2f((uint16_t)r.d) * (float)(int8_t)(uint8_t)(r.sc >> (8 * ((q >> 1) + 2 * n)));
    u4_t h;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t q4 = ((ql[2 * (q & 1) + j] >> (4 * n)) & 0x0F0F0F0Fu) | (((qv[2 * (q & 1) + j] >> sh) & 0x03030303u) << 4);
      h[2 * j] = tlx_mix2_f16(t, tlx_bytes_h2(q4, 0, 32.f));       // t * (q - 32)
      h[2 * j + 1] = tlx_mix2_f16(t, tlx_bytes_h2(q4, 1, 32.f));
    }
    tlx_mfma_operand_guard(h);
    return __builtin_bit_cast(h8_t, h);
  } else {
    constexpr int blk = S >> 2, q = S & 3;
    const u4_t& qv = blk ? ((q < 2) ? r.q2 : r.q3) : ((q < 2) ? r.q0 : r.q1);
    const float d = tlx_h2f((uint16_t)(r.d >> (16 * blk)));
    u4_t h;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t u4 = qv[2 * (q & 1) + j] ^ 0x80808080u;   // int8 + 128
      h[2 * j] = tlx_mix2_f16(d, tlx_bytes_h2(u4, 0, 128.f));
      h[2 * j + 1] = tlx_mix2_f16(d, tlx_bytes_h2(u4, 1, 128.f));
    }
    tlx_mfma_operand_guard(h);
    return __builtin_bit_cast(h8_t, h);
  }
}

template <int CLS, bool UP, int FORM, int KS, int NW>
struct GvShape {
  static constexpr int K = UP ? kHid : kFf, NU = K / 256, NM = UP ? 2 : 1;
  static constexpr int TW = NW / KS;                     // tiles per workgroup (NW waves)
  static constexpr int RB = (UP ? kFf : kHid) / (16 * TW);   // workgroups per item
  static constexpr int TOKR = FORM == GX_PAIRS ? 1 : kGvTok;   // staged token rows
  static constexpr int LDX = K + 8;                      // token row stride (halfs)
};

// XD (the dense form at P <= kGvTok): the token rows are read from memory (f32 -> fp16, as staged)
// a unit at a time instead of staged in LDS -- no LDS but the k-split sums, so the form can share a
// launch with a pair walk (tlx_moe_up3s_pairs_sh) without lowering its occupancy; the same operands.
template <int CLS, bool UP, int FORM, int KS, int NW, bool TL, bool XD>
__device__ __forceinline__ void gv_body(_Float16* xs, GvLutSlot<CLS == GX_IQ3S>& lslot, f4_t* red, const GxArgs& a,
                                        int blk) {
  using S = GvShape<CLS, UP, FORM, KS, NW>;
  constexpr int NT = 64 * NW;
  constexpr int K = S::K, NU = S::NU, NM = S::NM, TW = S::TW, RB = S::RB, TOKR = S::TOKR, LDX = S::LDX;
  constexpr int ROWB = K / GxFmt<CLS>::kPer * GxFmt<CLS>::kBlk;
  constexpr int UW = NU / KS;                            // units per wave
  constexpr int DEPTH = UW < 4 ? UW : 4;                 // units in flight
  constexpr bool GRID = CLS == GX_IQ3S;
  static_assert(NU % KS == 0 && NW % KS == 0, "k split");
  static_assert(!XD || FORM == GX_DENSE, "direct token rows: the dense form");
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, col = lane & 15, kq = lane >> 4;
  const int tile = wave / KS, kp = wave % KS;
  // the XCD-aware order of gx_kernel: an item's workgroups on one XCD
  int rb, item;
  if constexpr (FORM == GX_DENSE) {   // one item at decode: its column blocks over all XCDs
    rb = blk % RB;
    item = blk / RB;
  } else {
    const int slot = blk >> 3;
    rb = slot % RB;
    item = slot / RB * 8 + (blk & 7);
  }
  if (item >= a.items) return;

  int beg, nt;
  gbyte* wg;
  if constexpr (FORM == GX_PAIRS) {
    beg = item;
    nt = 1;
    wg = reinterpret_cast<gbyte*>(a.ptbl[a.eids[item]]);
  } else {
    beg = item * kGvTok;
    nt = min(kGvTok, a.P - beg);
    wg = (gbyte*)a.w0;
  }
  gbyte* wu = UP ? (FORM == GX_DENSE ? (gbyte*)a.w1 : wg + kIq3sGate) : wg;
  const GvLut* lut = nullptr;
  if constexpr (GRID) {
    gv_lut_fill<NT>(lslot.v, a.grid, t);
    lut = &lslot.v;
  }
  // token rows, fp16 (round to nearest even); rows past the item repeat its last (not stored)
  // (dense: the item's nt rows only -- the lanes of rows past it read unstaged LDS, and their
  // MFMA rows are never stored)
  for (int pc = t; pc < (XD ? 0 : FORM == GX_DENSE ? nt : TOKR) * (K / 8); pc += NT) {
    const int r = pc / (K / 8), k8 = pc - r * (K / 8);
    const int xr = FORM == GX_PAIRS ? (UP ? beg >> 3 : beg) : beg + min(r, nt - 1);
    const float4* src = reinterpret_cast<const float4*>(a.x + (size_t)xr * K + 8 * k8);
    const float4 u = src[0], v = src[1];
    const h8_t h = {(_Float16)u.x, (_Float16)u.y, (_Float16)u.z, (_Float16)u.w,
                    (_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    *reinterpret_cast<h8_t*>(xs + r * LDX + 8 * k8) = h;
  }

  const int n = rb * (16 * TW) + 16 * tile + col;   // output column (weight row) of the lane
  gbyte* rows[NM];
  rows[0] = wg + (size_t)n * ROWB;
  if constexpr (UP) rows[NM - 1] = wu + (size_t)n * ROWB;
  const int u0 = kp * UW;
  GvRaw<CLS> raw[UW][NM];
#pragma unroll
  for (int u = 0; u < DEPTH; ++u)
#pragma unroll
    for (int m = 0; m < NM; ++m) raw[u][m] = gv_fetch<CLS, TL>(rows[m], u0 + u, kq);
  __syncthreads();   // token rows, lookups
  const _Float16* xrow = xs + (FORM == GX_PAIRS ? 0 : col) * LDX;
  const float* xgrow = XD ? a.x + (size_t)(beg + min(col, nt - 1)) * K : nullptr;   // XD: the lane's token row
  f4_t acc[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) acc[m] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < UW; ++u) {
    if (u + DEPTH < UW) {
#pragma unroll
      for (int m = 0; m < NM; ++m) raw[u + DEPTH][m] = gv_fetch<CLS, TL>(rows[m], u0 + u + DEPTH, kq);
    }
    const _Float16* xu = xrow + 256 * (u0 + u);
    // XD: the lane's activations of half a unit (4 k-steps) in registers at a time
    float4 xd[XD ? 8 : 1][1];
    auto xload = [&](int h) {
      if constexpr (XD) {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const float4* src = reinterpret_cast<const float4*>(xgrow + 256 * (u0 + u) + gv_koff<CLS>(kq, 4 * h + s2));
          xd[2 * s2][0] = src[0];
          xd[2 * s2 + 1][0] = src[1];
        }
      }
    };
    xload(0);
#define GV_STEP(SS)                                                                          \
  {                                                                                          \
    h8_t ax;                                                                                 \
    if constexpr (XD) {                                                                      \
      const float4 p0 = xd[2 * ((SS) & 3)][0], p1 = xd[2 * ((SS) & 3) + 1][0];               \
      ax = h8_t{(_Float16)p0.x, (_Float16)p0.y, (_Float16)p0.z, (_Float16)p0.w,              \
                (_Float16)p1.x, (_Float16)p1.y, (_Float16)p1.z, (_Float16)p1.w};             \
    } else {                                                                                 \
      ax = *reinterpret_cast<const h8_t*>(xu + gv_koff<CLS>(kq, SS));                        \
    }                                                                                        \
    _Pragma("unroll") for (int m = 0; m < NM; ++m) {                                         \
      const h8_t bw = gv_decode<CLS, SS>(raw[u][m], kq, lut);                        \
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw, acc[m], 0, 0, 0);              \
    }                                                                                        \
  }
    GV_STEP(0) GV_STEP(1) GV_STEP(2) GV_STEP(3)
    xload(1);
    GV_STEP(4) GV_STEP(5) GV_STEP(6) GV_STEP(7)
#undef GV_STEP
  }
  // k-split: the tile's waves add in kp order
  if constexpr (KS > 1) {
    if (kp != 0) {
#pragma unroll
      for (int m = 0; m < NM; ++m) red[(((kp - 1) * TW + tile) * NM + m) * 64 + lane] = acc[m];
    }
    __syncthreads();
    if (kp != 0) return;
#pragma unroll
    for (int j = 1; j < KS; ++j)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[m] += red[(((j - 1) * TW + tile) * NM + m) * 64 + lane];
  }
  // lane (col, kq) holds tokens 4 kq + r of column n
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int tk = 4 * kq + r;
    if (tk >= nt) continue;
    const size_t o = (size_t)(beg + (FORM == GX_PAIRS ? 0 : tk));
    if constexpr (UP) {
      const float gv = acc[0][r], uv = acc[NM - 1][r];
      reinterpret_cast<float*>(a.out)[o * kFf + n] = gv / (1.f + expf(-gv)) * uv;
    } else if constexpr (FORM == GX_DENSE) {
      reinterpret_cast<float*>(a.out)[o * kHid + n] = acc[0][r];
    } else {
      reinterpret_cast<_Float16*>(a.out)[o * kHid + n] = (_Float16)acc[0][r];
    }
  }
}

template <int CLS, bool UP, int FORM, int KS, int NW, bool TL>
__global__ __launch_bounds__(64 * NW) void gv_kernel(const GxArgs a) {
  using S = GvShape<CLS, UP, FORM, KS, NW>;
  __shared__ __attribute__((aligned(16))) _Float16 xs[S::TOKR * S::LDX];
  __shared__ GvLutSlot<CLS == GX_IQ3S> lslot;
  __shared__ f4_t red[KS > 1 ? (KS - 1) * S::TW * S::NM * 64 : 1];
  gv_body<CLS, UP, FORM, KS, NW, TL, false>(xs, lslot, red, a, (int)blockIdx.x);
}

// The pair walk (class RCLS, 4 waves, KSR) and the Q8_0 shared expert's dense form at P <= kGvTok
// (direct token rows, 4 waves, KSS) in one launch: workgroups below nra walk the pairs (args a), the
// rest run the shared expert (args b) -- each part its own code, the separate launches' bits.
template <int RCLS, bool UP, int KSR, bool TL, int KSS>
__global__ __launch_bounds__(256) void gv_psh_kernel(const GxArgs a, const GxArgs b, int nra) {
  using SR = GvShape<RCLS, UP, GX_PAIRS, KSR, 4>;
  using SS = GvShape<GX_Q80, UP, GX_DENSE, KSS, 4>;
  constexpr int RR = KSR > 1 ? (KSR - 1) * SR::TW * SR::NM * 64 : 1, RS = KSS > 1 ? (KSS - 1) * SS::TW * SS::NM * 64 : 1;
  __shared__ __attribute__((aligned(16))) _Float16 xs[SR::TOKR * SR::LDX];
  __shared__ GvLutSlot<RCLS == GX_IQ3S> lslot;
  __shared__ GvLutSlot<false> nolut;
  __shared__ f4_t red[RR > RS ? RR : RS];
  const int blk = (int)blockIdx.x;
  if (blk < nra)
    gv_body<RCLS, UP, GX_PAIRS, KSR, 4, TL, false>(xs, lslot, red, a, blk);
  else
    gv_body<GX_Q80, UP, GX_DENSE, KSS, 4, false, true>(xs, nolut, red, b, blk - nra);
}

template <int CLS, bool UP, int FORM, int KS, int NW, bool TL = false>
int gv_launch(const GxArgs& a, int items, hipStream_t st) {
  GxArgs b = a;
  b.items = items;
  constexpr int RB = GvShape<CLS, UP, FORM, KS, NW>::RB;
  const int nblk = FORM == GX_DENSE ? items * RB : (items + 7) / 8 * 8 * RB;
  gv_kernel<CLS, UP, FORM, KS, NW, TL><<<(unsigned)nblk, 64 * NW, 0, st>>>(b);
  return tlx_launch_status();
}

// ------------------------------------------------------------------ batched down, register decode
// Down projections of batches (an expert's sorted pairs, or a chunk of positions for the shared
// expert) with the item's activations resident in LDS: a workgroup stages up to kGqTok token rows
// of act as fp16 once per pass, then its 8 waves walk 2048 / RB weight rows of the item in 16-row
// tiles (a contiguous run of tiles a wave).  Each lane fetches the bytes of its 64 weights of a
// 256-weight unit straight into registers (gv_fetch, DEPTH units ahead) and builds each k-step's 8
// operands there (gv_decode: the other forms' operands bit for bit); every operand feeds all of the
// pass's 16-token groups.  The weights are the MFMA's first operand, so a lane's four outputs are
// four consecutive rows of one token: one 8-B (fp16 parts) or 16-B (f32) store.
constexpr int kGqTok = 128;
constexpr int kGqLdx = kFf + 8;   // token row stride (halfs): a fragment's 16 rows fall in distinct banks

struct alignas(16) GqLds {
  _Float16 x[kGqTok * kGqLdx];
  int orow[kGqTok];
};

template <int CLS> constexpr int gq_unit_bytes() { return CLS == GX_Q80 ? 8 * 34 : GxFmt<CLS>::kBlk; }

// The wave's tiles for one pass of NG token groups: per unit, 8 k-steps of one decoded operand
// and NG MFMAs; the next unit's bytes into the freed ring slot; a tile's outputs after its last unit.
template <int CLS, int FORM, int NU, int UNITS, int DEPTH, int NG, typename F>
__device__ __forceinline__ void gq_tiles(const GqLds& L, const GxArgs& a, GvRaw<CLS> (&raw)[DEPTH], F& fetch,
                                         int tile0, int nt, int col, int kq) {
  const _Float16* xl = L.x + col * kGqLdx;   // token row 16 g + col: + 16 g kGqLdx
  f4_t acc[NG];
  for (int q0 = 0; q0 < UNITS; q0 += DEPTH) {
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
      const int q = q0 + r;
      if (r % NU == 0) {   // DEPTH % NU == 0: unit r % NU of tile q / NU
#pragma unroll
        for (int g = 0; g < NG; ++g) acc[g] = f4_t{0.f, 0.f, 0.f, 0.f};
      }
      const _Float16* xu = xl + 256 * (r % NU);
#define GQ_STEP(SS)                                                                                  \
  {                                                                                                  \
    const h8_t bw = gv_decode<CLS, SS>(raw[r], kq, nullptr);                                         \
    _Pragma("unroll") for (int g = 0; g < NG; ++g) {                                                 \
      const h8_t ax = *reinterpret_cast<const h8_t*>(xu + 16 * g * kGqLdx + gv_koff<CLS>(kq, SS));   \
      acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bw, ax, acc[g], 0, 0, 0);                      \
    }                                                                                                \
  }
      GQ_STEP(0) GQ_STEP(1) GQ_STEP(2) GQ_STEP(3) GQ_STEP(4) GQ_STEP(5) GQ_STEP(6) GQ_STEP(7)
#undef GQ_STEP
      raw[r] = fetch(min(q + DEPTH, UNITS - 1));   // past the end: the last unit again
      if (r % NU == NU - 1) {
        // lane (col, kq) holds rows 4 kq .. 4 kq + 3 of the tile for token 16 g + col
        const int n0 = 16 * (tile0 + q / NU) + 4 * kq;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int tk = 16 * g + col;
          if (tk < nt) {
            const size_t o = (size_t)L.orow[tk] * kHid + n0;
            if constexpr (FORM == GX_DENSE) {
              *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(a.out) + o) = acc[g];
            } else {
              const h2_t lo = {(_Float16)acc[g][0], (_Float16)acc[g][1]};
              const h2_t hi = {(_Float16)acc[g][2], (_Float16)acc[g][3]};
              *reinterpret_cast<uint2*>(reinterpret_cast<_Float16*>(a.out) + o) =
                  uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
            }
          }
        }
      }
    }
  }
}

// blk: the workgroup's index in its part of the grid (parts start at multiples of 8)
template <int CLS, int FORM, int RB, int DEPTH, bool TL>
__device__ __forceinline__ void gq_dn_body(GqLds& L, const GxArgs& a, int blk) {
  constexpr int K = kFf, NU = K / 256, NW = 8;
  constexpr int ROWB = NU * gq_unit_bytes<CLS>();
  constexpr int TILES = kHid / 16 / RB, TPW = TILES / NW, UNITS = TPW * NU;
  static_assert(TILES % NW == 0 && UNITS % DEPTH == 0 && DEPTH % NU == 0, "tiling");
  static_assert(FORM != GX_PAIRS, "the pair walk is gv_kernel's");
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, col = lane & 15, kq = lane >> 4;
  // an item's RB workgroups on one XCD (block b runs on XCD b % 8): its act rows come from HBM once
  const int slot = blk >> 3;
  const int rb = slot % RB, item = slot / RB * 8 + (blk & 7);
  if (item >= a.items) return;
  int beg, ntot;
  gbyte* w;
  if constexpr (FORM == GX_SORTED) {
    beg = a.eoff[item];
    ntot = a.eoff[item + 1] - beg;
    w = reinterpret_cast<gbyte*>(a.ptbl[item]);
  } else {
    beg = item * kGqTok;
    ntot = min(kGqTok, a.P - beg);
    w = (gbyte*)a.w0;
  }
  if (ntot <= 0) return;   // uniform per workgroup
  const int tile0 = rb * TILES + wave * TPW;
  gbyte* wrow = w + (size_t)(16 * tile0 + col) * ROWB;   // the lane's row in the wave's first tile
  auto fetch = [&](int q) { return gv_fetch<CLS, TL>(wrow + (size_t)(16 * (q / NU)) * ROWB, q % NU, kq); };

  for (int p0 = 0; p0 < ntot; p0 += kGqTok) {
    const int nt = min(kGqTok, ntot - p0), ng = (nt + 15) >> 4;
    // the first units' loads do not depend on the staging: issued first
    GvRaw<CLS> raw[DEPTH];
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) raw[r] = fetch(r);
    __syncthreads();   // the previous pass is done with the rows
    if (t < nt) L.orow[t] = FORM == GX_SORTED ? (int)a.plist[beg + p0 + t] : beg + p0 + t;
    __syncthreads();
    // the pass's token rows as fp16 (round to nearest even); rows nt .. 16 ng - 1 zero.  Thread t
    // converts k-piece t % 64 of rows t / 64 + 8 j, four rows' loads in flight at a time.
    {
      const int k8 = t & 63, r0 = t >> 6;
      for (int j0 = 0; j0 < 2 * ng; j0 += 4) {
        float4 v[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = r0 + 8 * (j0 + j);
          const int xr = r < nt ? L.orow[r] : 0;
          const float4* src = reinterpret_cast<const float4*>(a.x + (size_t)xr * K + 8 * k8);
          v[j][0] = src[0];
          v[j][1] = src[1];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = r0 + 8 * (j0 + j);
          if (r < 16 * ng) {
            const bool z = r >= nt;
            const float4 u = z ? float4{0.f, 0.f, 0.f, 0.f} : v[j][0], s = z ? float4{0.f, 0.f, 0.f, 0.f} : v[j][1];
            const h8_t h = {(_Float16)u.x, (_Float16)u.y, (_Float16)u.z, (_Float16)u.w,
                            (_Float16)s.x, (_Float16)s.y, (_Float16)s.z, (_Float16)s.w};
            *reinterpret_cast<h8_t*>(L.x + r * kGqLdx + 8 * k8) = h;
          }
        }
      }
    }
    __syncthreads();

    // the tile walk, specialized on the pass's group count (no branch around a load or an MFMA)
    switch (ng) {
      case 1: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 1>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 2: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 2>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 3: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 3>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 4: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 4>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 5: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 5>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 6: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 6>(L, a, raw, fetch, tile0, nt, col, kq); break;
      case 7: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 7>(L, a, raw, fetch, tile0, nt, col, kq); break;
      default: gq_tiles<CLS, FORM, NU, UNITS, DEPTH, 8>(L, a, raw, fetch, tile0, nt, col, kq); break;
    }
  }
}

template <int CLS, int FORM, int RB, int DEPTH, bool TL>
__global__ __launch_bounds__(512) void gq_dn_kernel(const GxArgs a) {
  __shared__ GqLds L;
  gq_dn_body<CLS, FORM, RB, DEPTH, TL>(L, a, (int)blockIdx.x);
}

#ifndef GQ_RRB
#define GQ_RRB 1
#endif
#ifndef GQ_DEPTH
#define GQ_DEPTH 2
#endif
constexpr int kGqRrb = GQ_RRB, kGqDepth = GQ_DEPTH;

// ------------------------------------------------------------------ dequantizers (bit-exact)
// One thread per (row, 16-weight piece).
template <int CLS>
__global__ __launch_bounds__(256) void gx_dequant_kernel(const uint8_t* __restrict__ w, const float* __restrict__ gridf,
                                                         void* __restrict__ out, int64_t rows, int kdim, int out_f16) {
  constexpr bool GRID = CLS == GX_IQ3S;
  __shared__ float4 grid[GRID ? 512 : 1];
  __shared__ GvLutSlot<GRID> lslot;
  const GvLut* lut = nullptr;
  if constexpr (GRID) {
    for (int i = threadIdx.x; i < 512; i += 256) grid[i] = reinterpret_cast<const float4*>(gridf)[i];
    gv_lut_fill<256>(lslot.v, gridf, threadIdx.x);
    lut = &lslot.v;
    __syncthreads();
  }
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int np = kdim >> 4;
  if (u >= rows * np) return;
  const int64_t r = u / np;
  const int pi = (int)(u - r * np);
  const int64_t rowb = (int64_t)kdim / GxFmt<CLS>::kPer * GxFmt<CLS>::kBlk;
  const uint8_t* row = w + r * rowb;
  const int64_t o = r * kdim + 16 * pi;
  if (out_f16) {   // the GEMMs' operand path (gx_decode_h)
    u4_t h[2];
    gx_decode_h<CLS>(h, gx_fetch<CLS>(row, 16 * pi), lut);
    uint32_t* o32 = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(out) + o);   // 4-B aligned: o % 16 == 0
#pragma unroll
    for (int l = 0; l < 8; ++l) o32[l] = h[l >> 2][l & 3];
  } else {
    float v[16];
    gx_dequant16<CLS>(v, row, 16 * pi, grid);
#pragma unroll
    for (int l = 0; l < 16; ++l) reinterpret_cast<float*>(out)[o + l] = v[l];
  }
}

template <int CLS, bool UP, int FORM, bool TL = false>
int gx_launch(const GxArgs& a, int items, hipStream_t st) {
  constexpr int RB = (UP ? kFf : kHid) / (16 * gx_waves<UP>());
  GxArgs b = a;
  b.items = items;
  gx_kernel<CLS, UP, FORM, TL><<<(unsigned)((items + 7) / 8 * 8 * RB), 64 * gx_waves<UP>(), 0, st>>>(b);
  return tlx_launch_status();
}

}  // namespace

extern "C" int tlx_iq3s_dequant(const void* w, const float* gridf, void* out, int64_t rows, int64_t kdim, int out_f16,
                                void* stream) {
  TLX_RET_IF(w == nullptr || gridf == nullptr || out == nullptr, TLX_E_ARG);
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255) || kdim > (1 << 24), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 2) || !tlx_aligned(gridf, 16) || !tlx_aligned(out, 4), TLX_E_ALIGN);
  const int64_t units = rows * (kdim >> 4), grid = (units + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  gx_dequant_kernel<GX_IQ3S><<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)w, gridf, out, rows,
                                                                              (int)kdim, out_f16);
  return tlx_launch_status();
}

extern "C" int tlx_q8_0_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16, void* stream) {
  TLX_RET_IF(w == nullptr || out == nullptr, TLX_E_ARG);
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255) || kdim > (1 << 24), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 2) || !tlx_aligned(out, 4), TLX_E_ALIGN);
  const int64_t units = rows * (kdim >> 4), grid = (units + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  gx_dequant_kernel<GX_Q80><<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)w, nullptr, out, rows,
                                                                             (int)kdim, out_f16);
  return tlx_launch_status();
}

// the slabs' layout argument: GGUF rows or this library's tiled records
static bool ckpt_layout_ok(int layout) { return layout == TLX_LAYOUT_RAW || layout == TLX_LAYOUT_TILED; }

extern "C" int tlx_moe_up3s(const uint64_t* ptbl, const int* eoff, const uint16_t* plist, const float* xs,
                            const float* gridf, float* ys, int np, int layout, void* stream) {
  TLX_RET_IF(!ptbl || !eoff || !plist || !xs || !gridf || !ys, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl, 8) || !tlx_aligned(xs, 16) || !tlx_aligned(gridf, 16) || !tlx_aligned(ys, 4), TLX_E_ALIGN);
  GxArgs a{};
  a.ptbl = ptbl; a.eoff = eoff; a.plist = plist; a.x = xs; a.grid = gridf; a.out = ys;
  if (layout == TLX_LAYOUT_TILED) return gx_launch<GX_IQ3S, true, GX_SORTED, true>(a, kE, (hipStream_t)stream);
  return gx_launch<GX_IQ3S, true, GX_SORTED>(a, kE, (hipStream_t)stream);
}

extern "C" int tlx_moe_up3s_pairs(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* gridf,
                                  float* ys, int np, int layout, void* stream) {
  TLX_RET_IF(!ptbl || !eids || !xs || !gridf || !ys, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl, 8) || !tlx_aligned(xs, 16) || !tlx_aligned(gridf, 16) || !tlx_aligned(ys, 4), TLX_E_ALIGN);
  GxArgs a{};
  a.ptbl = ptbl; a.eids = eids; a.x = xs; a.grid = gridf; a.out = ys;
  if (layout == TLX_LAYOUT_TILED) return gv_launch<GX_IQ3S, true, GX_PAIRS, 4, 4, true>(a, np, (hipStream_t)stream);
  return gv_launch<GX_IQ3S, true, GX_PAIRS, 4, 4>(a, np, (hipStream_t)stream);
}

// the routed Q6_K down over the sorted pairs: the register-decode form (8-B stores a lane), else the
// LDS-staged one
template <bool TL>
static int dn6_sorted_tl(GxArgs a, hipStream_t st) {
  a.items = kE;
  if (tlx_aligned(a.out, 8)) {
    gq_dn_kernel<GX_Q6K, GX_SORTED, kGqRrb, kGqDepth, TL><<<(unsigned)((kE + 7) / 8 * 8 * kGqRrb), 512, 0, st>>>(a);
    return tlx_launch_status();
  }
  return gx_launch<GX_Q6K, false, GX_SORTED, TL>(a, kE, st);
}

static int dn6_sorted(const GxArgs& a, int layout, hipStream_t st) {
  return layout == TLX_LAYOUT_TILED ? dn6_sorted_tl<true>(a, st) : dn6_sorted_tl<false>(a, st);
}

extern "C" int tlx_moe_dn6(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                           const uint16_t* plist, const float* act, uint16_t* parts, int np, int layout,
                           void* stream) {
  (void)items;   // the reference's slots; this form walks eoff / plist itself
  (void)nitp;
  TLX_RET_IF(!ptbl_dn || !eoff || !plist || !act || !parts, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl_dn, 8) || !tlx_aligned(act, 16) || !tlx_aligned(parts, 2), TLX_E_ALIGN);
  GxArgs a{};
  a.ptbl = ptbl_dn; a.eoff = eoff; a.plist = plist; a.x = act; a.out = parts;
  return dn6_sorted(a, layout, (hipStream_t)stream);
}

extern "C" int tlx_moe_dn6_pairs(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, uint16_t* parts,
                                 int np, int layout, void* stream) {
  TLX_RET_IF(!ptbl_dn || !eids || !act || !parts, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl_dn, 8) || !tlx_aligned(act, 16) || !tlx_aligned(parts, 2), TLX_E_ALIGN);
  GxArgs a{};
  a.ptbl = ptbl_dn; a.eids = eids; a.x = act; a.out = parts;
  if (layout == TLX_LAYOUT_TILED) return gv_launch<GX_Q6K, false, GX_PAIRS, 1, 4, true>(a, np, (hipStream_t)stream);
  return gv_launch<GX_Q6K, false, GX_PAIRS, 1, 4>(a, np, (hipStream_t)stream);
}

// the shared expert's decode k-split (4 waves a workgroup: the shape the pair walks' launches share)
constexpr int kShKsUp = 4, kShKsDn = 2;

// the shared expert's two launches (decode form at P <= kGvTok)
static int moe_shared8_up(const void* wg, const void* wu, const float* x, float* act, int P, hipStream_t st) {
  GxArgs a{};
  a.w0 = (const uint8_t*)wg; a.w1 = (const uint8_t*)wu; a.x = x; a.out = act; a.P = P;
  if (P <= kGvTok) return gv_launch<GX_Q80, true, GX_DENSE, kShKsUp, 4>(a, 1, st);
  return gx_launch<GX_Q80, true, GX_DENSE>(a, (P + gx_tok<GX_DENSE>() - 1) / gx_tok<GX_DENSE>(), st);
}

static int moe_shared8_dn(const void* wd, const float* act, float* y, int P, hipStream_t st) {
  GxArgs b{};
  b.w0 = (const uint8_t*)wd; b.x = act; b.out = y; b.P = P;
  if (P <= kGvTok) return gv_launch<GX_Q80, false, GX_DENSE, kShKsDn, 4>(b, 1, st);
  return gx_launch<GX_Q80, false, GX_DENSE>(b, (P + gx_tok<GX_DENSE>() - 1) / gx_tok<GX_DENSE>(), st);
}

// the pair walk (a, np items) + the shared expert's dense form with direct token rows (b, P <= kGvTok)
template <int RCLS, bool UP, int KSR, bool TL, int KSS>
static int gv_psh_launch(const GxArgs& a, int np, const GxArgs& b, hipStream_t st) {
  GxArgs ra = a, sb = b;
  ra.items = np;
  sb.items = 1;
  const int nra = (np + 7) / 8 * 8 * GvShape<RCLS, UP, GX_PAIRS, KSR, 4>::RB;
  const int nsb = GvShape<GX_Q80, UP, GX_DENSE, KSS, 4>::RB;
  gv_psh_kernel<RCLS, UP, KSR, TL, KSS><<<(unsigned)(nra + nsb), 256, 0, st>>>(ra, sb, nra);
  return tlx_launch_status();
}

// routed sorted form (a, kE items) + the shared expert's dense form (b) in one launch, P > kGvTok
template <int RCLS, bool UP, bool TL>
static int gx_sh_launch(const GxArgs& a, const GxArgs& b, hipStream_t st) {
  constexpr int RB = (UP ? kFf : kHid) / (16 * gx_waves<UP>());
  GxArgs ra = a, sb = b;
  ra.items = kE;
  sb.items = (b.P + gx_tok<GX_DENSE>() - 1) / gx_tok<GX_DENSE>();
  const int nra = (kE + 7) / 8 * 8 * RB, nsb = (sb.items + 7) / 8 * 8 * RB;
  gx_sh_kernel<RCLS, UP, TL><<<(unsigned)(nra + nsb), 64 * gx_waves<UP>(), 0, st>>>(ra, sb, nra);
  return tlx_launch_status();
}

extern "C" int tlx_moe_up3s_sh(const uint64_t* ptbl, const int* eoff, const uint16_t* plist, const float* xs,
                               const float* gridf, float* ys, int np, const void* wg8, const void* wu8, float* sact,
                               int P, int layout, void* stream) {
  TLX_RET_IF(!ptbl || !eoff || !plist || !xs || !gridf || !ys || !wg8 || !wu8 || !sact, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || P > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl, 8) || !tlx_aligned(xs, 16) || !tlx_aligned(gridf, 16) || !tlx_aligned(ys, 4),
             TLX_E_ALIGN);
  TLX_RET_IF(!tlx_aligned(wg8, 2) || !tlx_aligned(wu8, 2) || !tlx_aligned(sact, 16), TLX_E_ALIGN);
  const hipStream_t st = (hipStream_t)stream;
  GxArgs a{};
  a.ptbl = ptbl; a.eoff = eoff; a.plist = plist; a.x = xs; a.grid = gridf; a.out = ys;
  if (P <= kGvTok) {   // the shared expert's decode form is another kernel: two launches
    const int rc = layout == TLX_LAYOUT_TILED ? gx_launch<GX_IQ3S, true, GX_SORTED, true>(a, kE, st)
                                              : gx_launch<GX_IQ3S, true, GX_SORTED>(a, kE, st);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared8_up(wg8, wu8, xs, sact, P, st);
  }
  GxArgs b{};
  b.w0 = (const uint8_t*)wg8; b.w1 = (const uint8_t*)wu8; b.x = xs; b.out = sact; b.P = P;
  if (layout == TLX_LAYOUT_TILED) return gx_sh_launch<GX_IQ3S, true, true>(a, b, st);
  return gx_sh_launch<GX_IQ3S, true, false>(a, b, st);
}

extern "C" int tlx_moe_dn6_sh(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                              const uint16_t* plist, const float* act, uint16_t* parts, int np, const void* wd8,
                              const float* sact, float* shared, int P, int layout, void* stream) {
  (void)items;   // the reference's slots; this form walks eoff / plist itself
  (void)nitp;
  TLX_RET_IF(!ptbl_dn || !eoff || !plist || !act || !parts || !wd8 || !sact || !shared, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || P > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl_dn, 8) || !tlx_aligned(act, 16) || !tlx_aligned(parts, 2), TLX_E_ALIGN);
  TLX_RET_IF(!tlx_aligned(wd8, 2) || !tlx_aligned(sact, 16) || !tlx_aligned(shared, 4), TLX_E_ALIGN);
  const hipStream_t st = (hipStream_t)stream;
  GxArgs a{};
  a.ptbl = ptbl_dn; a.eoff = eoff; a.plist = plist; a.x = act; a.out = parts;
  if (P <= kGvTok) {
    const int rc = dn6_sorted(a, layout, st);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared8_dn(wd8, sact, shared, P, st);
  }
  if (tlx_aligned(parts, 8)) {
    // the routed register-decode form and the shared expert's staged form: two launches (their LDS
    // footprints differ: in one launch the shared part would run at one workgroup per CU)
    const int rc = dn6_sorted(a, layout, st);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared8_dn(wd8, sact, shared, P, st);
  }
  GxArgs b{};
  b.w0 = (const uint8_t*)wd8; b.x = sact; b.out = shared; b.P = P;
  if (layout == TLX_LAYOUT_TILED) return gx_sh_launch<GX_Q6K, false, true>(a, b, st);
  return gx_sh_launch<GX_Q6K, false, false>(a, b, st);
}

extern "C" int tlx_moe_shared8(const void* wg, const void* wu, const void* wd, const float* x, float* y, float* act,
                               int P, void* stream) {
  TLX_RET_IF(!wg || !wu || !wd || !x || !y || !act, TLX_E_ARG);
  TLX_RET_IF(P < 1 || P > kMaxPairs, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(wg, 2) || !tlx_aligned(wu, 2) || !tlx_aligned(wd, 2), TLX_E_ALIGN);
  TLX_RET_IF(!tlx_aligned(x, 16) || !tlx_aligned(act, 16) || !tlx_aligned(y, 4), TLX_E_ALIGN);
  hipStream_t st = (hipStream_t)stream;
  const int r = moe_shared8_up(wg, wu, x, act, P, st);   // decode (P <= 16): the GEMV-shaped form
  TLX_RET_IF(r != TLX_OK, r);
  return moe_shared8_dn(wd, act, y, P, st);
}

extern "C" int tlx_moe_up3s_pairs_sh(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* gridf,
                                     float* ys, int np, const void* wg8, const void* wu8, float* sact, int P,
                                     int layout, void* stream) {
  TLX_RET_IF(!ptbl || !eids || !xs || !gridf || !ys || !wg8 || !wu8 || !sact, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || P > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl, 8) || !tlx_aligned(xs, 16) || !tlx_aligned(gridf, 16) || !tlx_aligned(ys, 4),
             TLX_E_ALIGN);
  TLX_RET_IF(!tlx_aligned(wg8, 2) || !tlx_aligned(wu8, 2) || !tlx_aligned(sact, 16), TLX_E_ALIGN);
  const hipStream_t st = (hipStream_t)stream;
  GxArgs a{};
  a.ptbl = ptbl; a.eids = eids; a.x = xs; a.grid = gridf; a.out = ys;
  if (P > kGvTok) {   // the shared expert's batch form is another kernel: two launches
    const int rc = layout == TLX_LAYOUT_TILED ? gv_launch<GX_IQ3S, true, GX_PAIRS, 4, 4, true>(a, np, st)
                                              : gv_launch<GX_IQ3S, true, GX_PAIRS, 4, 4>(a, np, st);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared8_up(wg8, wu8, xs, sact, P, st);
  }
  GxArgs b{};
  b.w0 = (const uint8_t*)wg8; b.w1 = (const uint8_t*)wu8; b.x = xs; b.out = sact; b.P = P;
  if (layout == TLX_LAYOUT_TILED) return gv_psh_launch<GX_IQ3S, true, 4, true, kShKsUp>(a, np, b, st);
  return gv_psh_launch<GX_IQ3S, true, 4, false, kShKsUp>(a, np, b, st);
}

extern "C" int tlx_moe_dn6_pairs_sh(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, uint16_t* parts,
                                    int np, const void* wd8, const float* sact, float* shared, int P, int layout,
                                    void* stream) {
  TLX_RET_IF(!ptbl_dn || !eids || !act || !parts || !wd8 || !sact || !shared, TLX_E_ARG);
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || P > kMaxPairs || !ckpt_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(ptbl_dn, 8) || !tlx_aligned(act, 16) || !tlx_aligned(parts, 2), TLX_E_ALIGN);
  TLX_RET_IF(!tlx_aligned(wd8, 2) || !tlx_aligned(sact, 16) || !tlx_aligned(shared, 4), TLX_E_ALIGN);
  const hipStream_t st = (hipStream_t)stream;
  GxArgs a{};
  a.ptbl = ptbl_dn; a.eids = eids; a.x = act; a.out = parts;
  if (P > kGvTok) {
    const int rc = layout == TLX_LAYOUT_TILED ? gv_launch<GX_Q6K, false, GX_PAIRS, 1, 4, true>(a, np, st)
                                              : gv_launch<GX_Q6K, false, GX_PAIRS, 1, 4>(a, np, st);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared8_dn(wd8, sact, shared, P, st);
  }
  GxArgs b{};
  b.w0 = (const uint8_t*)wd8; b.x = sact; b.out = shared; b.P = P;
  if (layout == TLX_LAYOUT_TILED) return gv_psh_launch<GX_Q6K, false, 1, true, kShKsDn>(a, np, b, st);
  return gv_psh_launch<GX_Q6K, false, 1, false, kShKsDn>(a, np, b, st);
}

// ------------------------------------------------------------------ tiled checkpoint slabs
// One thread per output byte of record (tile, block): the byte's lane l = 16 kq + col (or row col)
// names the GGUF row 16 tile + col and the block byte it copies.
template <int CLS>
__global__ __launch_bounds__(256) void pack_ckpt_tiled_kernel(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ dst, long nbytes, int nb) {
  constexpr int REC = CLS == GX_IQ3S ? 1760 : 3360, BB = CLS == GX_IQ3S ? 110 : 210;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= nbytes) return;
  const long u = i / REC;
  const int o = (int)(i - u * REC);
  const long tile = u / nb;
  const int b = (int)(u - tile * nb);
  int col, sb;   // row in the tile, byte in its block
  if constexpr (CLS == GX_IQ3S) {
    if (o < 1024) {
      col = (o >> 4) & 15; sb = 2 + 16 * (o >> 8) + (o & 15);
    } else if (o < 1536) {
      const int q = o - 1024; col = (q >> 3) & 15; sb = 74 + 8 * (q >> 7) + (q & 7);
    } else if (o < 1664) {
      const int q = o - 1536; col = (q >> 1) & 15; sb = 66 + 2 * (q >> 5) + (q & 1);
    } else if (o < 1728) {
      const int q = o - 1664; col = q & 15; sb = 106 + (q >> 4);
    } else {
      const int q = o - 1728; col = q >> 1; sb = q & 1;
    }
  } else {
    if (o < 2048) {
      col = (o >> 5) & 15; sb = 32 * (o >> 9) + (o & 31);
    } else if (o < 3072) {
      const int q = o - 2048; col = (q >> 5) & 15; sb = 128 + 32 * (q >> 9) + (q & 31);
    } else if (o < 3328) {
      const int q = o - 3072, kq = q >> 6, s = q & 3;
      col = (q >> 2) & 15; sb = 192 + 8 * (kq >> 1) + 2 * (kq & 1) + (s & 1) + 4 * (s >> 1);
    } else {
      const int q = o - 3328; col = q >> 1; sb = 208 + (q & 1);
    }
  }
  dst[i] = src[(tile * 16 + col) * (long)nb * BB + (long)b * BB + sb];
}

template <int CLS>
static int pack_ckpt_tiled(const void* src, void* tiled, int N, int K, void* stream) {
  TLX_RET_IF(!src || !tiled, TLX_E_ARG);
  TLX_RET_IF(N < 16 || (N % 16) || K < 256 || (K % 256), TLX_E_ARG);
  const long nbytes = (long)(N / 16) * (K / 256) * (CLS == GX_IQ3S ? 1760 : 3360);
  TLX_RET_IF((nbytes + 255) / 256 > 0x7fffffff, TLX_E_ARG);
  pack_ckpt_tiled_kernel<CLS><<<(unsigned)((nbytes + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)src, (uint8_t*)tiled, nbytes, K / 256);
  return tlx_launch_status();
}

extern "C" int tlx_pack_iq3s_tiled(const void* src, void* tiled, int N, int K, void* stream) {
  return pack_ckpt_tiled<GX_IQ3S>(src, tiled, N, K, stream);
}

extern "C" int tlx_pack_q6k_tiled(const void* src, void* tiled, int N, int K, void* stream) {
  return pack_ckpt_tiled<GX_Q6K>(src, tiled, N, K, stream);
}
