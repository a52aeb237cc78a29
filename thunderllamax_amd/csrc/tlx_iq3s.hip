// IQ3_XXS decode GEMVs over tile-major records (TLX_LAYOUT_TILED): the records, their device
// repacker, and the balanced GEMV kernel that streams them.
//
// Record (16-row tile t, 256-k block b), 1632 B, records in (tile, block) order:
//   [0, 1024)     slot L = 16*kq + r, 16 B: bits 0..127 of the slot's index stream
//   [1024, 1536)  slot L, 8 B: bits 128..191
//   [1536, 1600)  row r, u32: the 8 sub-block scales s_j = sw[j] >> 28 as nibbles 4j..4j+3
//   [1600, 1632)  row r, u16: the block's d
// Index stream of slot (kq, r): 8 lane-chunks c = 0..7 (GGUF lane-chunk 8kq + c = weights
// 64kq + 8c .. +7 of row r), 24 bits each: two 12-bit lookup indices nib << 8 | g into the
// sign-folded table (tlx_iq3_table), g = the chunk's grid bytes, nib = its sign bits 0..3 and
// 4..6 + parity (the 8th sign).  The sign fields are recovered exactly from the indices, so the
// record is a lossless re-encoding of the GGUF block (102 B per 256 weights against 98): the
// parity the kernel would otherwise count per chunk is stored.
//
// Kernel: one workgroup per CU (persistent), W waves.  The T*NB records ("units") are split into
// G*W equal contiguous ranges, one per wave, so every CU streams the same number of bytes and a
// wave reads its range front to back (each record is 1632 contiguous bytes).  Lane (col, kq)
// decodes row col's slot kq of each record into MFMA B operands exactly as the packed-row GEMV
// does (same products, same per-block d scaling), so a block's contribution is bit-identical to
// that kernel's; the sum over blocks is a fixed order of per-wave partials:
//   * a wave's partial for a tile it does not cover completely goes to LDS; after the loop the
//     lowest contributing wave adds the contributions in wave order;
//   * a tile shared by two workgroups (at most two: a workgroup covers >= NB units) is finished
//     by the second of them to arrive: both write their part to the workspace, wait for those
//     stores to complete, count on a per-boundary counter (self-resetting: 0 -> 1 -> 0), and the
//     second adds lower-range part + upper-range part.
// The order depends only on (N, K, CU count): rows of an M-row call equal an M=1 call bit for bit.
#include "tlx_common.h"

#include <algorithm>

namespace {

constexpr int kTblEntries = 4096;
constexpr uint32_t kRec = 1632;
constexpr int kMaxG = 256;   // workgroups (boundaries) the workspace has slots for

enum Epi { EPI_F16 = 0, EPI_SWIGLU = 1, EPI_RESID = 2 };

// ------------------------------------------------------------------ repacker
// One thread per (record, slot): the slot's 24 B of indices, and for kq == 0 the row's scale word
// and d.  src: raw GGUF blocks (raw = 1) or packed rows [qs 64NB][sw 32NB][d 2NB]; rows >= N zero.
__global__ __launch_bounds__(256) void pack_tiled_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ rec,
                                                         long nslots, int N, int nb, int raw) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= nslots) return;
  const long u = i >> 6;                     // record = tile * nb + b
  const int L = (int)(i & 63), r = L & 15, kq = L >> 4;
  const long tile = u / nb;
  const int b = (int)(u - tile * nb);
  const long row = tile * 16 + r;
  uint8_t* o = rec + u * kRec;
  uint32_t st[6] = {0, 0, 0, 0, 0, 0};
  uint32_t scw = 0, dbits = 0;
  if (row < N) {
    const uint8_t* rp = src + row * 98L * nb;
    const uint8_t* qs = raw ? rp + 98L * b + 2 : rp + 64L * b;
    const uint8_t* sw = raw ? rp + 98L * b + 66 : rp + 64L * nb + 32L * b;
    dbits = raw ? tlx_ldu<uint16_t>(rp + 98L * b) : tlx_ldu<uint16_t>(rp + 96L * nb + 2L * b);
    for (int j = 0; j < 8; ++j) scw |= (tlx_ldu<uint32_t>(sw + 4 * j) >> 28) << (4 * j);
    for (int c = 0; c < 8; ++c) {
      const int lc = 8 * kq + c;                      // GGUF lane-chunk: weights 8lc .. 8lc+7
      const uint32_t w = tlx_ldu<uint32_t>(sw + 4 * (lc >> 2));
      const uint32_t sidx = (w >> (7 * (lc & 3))) & 0x7Fu;
      const uint32_t par = __builtin_popcount(sidx) & 1u;
      const uint32_t i0 = ((sidx & 0xFu) << 8) | qs[2 * lc];
      const uint32_t i1 = (((sidx >> 4) | (par << 3)) << 8) | qs[2 * lc + 1];
      const uint32_t v = i0 | (i1 << 12);             // 24 bits at stream bit 24c
      const int p = 24 * c, d = p >> 5, s = p & 31;
      st[d] |= v << s;
      if (s > 8) st[d + 1] |= v >> (32 - s);
    }
  }
  *reinterpret_cast<u4_t*>(o + 16 * L) = u4_t{st[0], st[1], st[2], st[3]};
  *reinterpret_cast<u2_t*>(o + 1024 + 8 * L) = u2_t{st[4], st[5]};
  if (kq == 0) {
    *reinterpret_cast<uint32_t*>(o + 1536 + 4 * r) = scw;
    *reinterpret_cast<uint16_t*>(o + 1600 + 2 * r) = (uint16_t)dbits;
  }
}

// ------------------------------------------------------------------ GEMV
constexpr int kMaxSeg = 4;   // matrices sharing the activations in one launch (NMAT == 1)

struct SkArgs {
  // segment s: records sw[s] (tiles sT0[s] .. sT0[s+1]-1 of the launch), output sout[s] with
  // sN[s] valid rows and row stride sld[s]; unused segments have sT0 = INT_MAX
  const uint8_t* sw[kMaxSeg];
  void* sout[kMaxSeg];
  int sN[kMaxSeg], sld[kMaxSeg], sT0[kMaxSeg + 1];
  int nseg;
  const uint8_t* w1;   // up matrix (SwiGLU, one segment), else null
  const float* res;    // residual (EPI_RESID, one segment; row stride sld[0])
  const float* gridf;
  const _Float16* x;   // [M][K], or (xt) the tile-ordered copy [K/8][16][8]
  int xt;
  int otile;           // 1: fp16 outputs in the tile-ordered form [N/8][16][8] (all 16 rows)
  int M, K, nb, U, G;
  f4_t* part;          // workspace: boundary g: [lo | hi][NMAT][64 lanes]
  uint32_t* cnt;       // workspace: arrival counter per boundary (0 between calls, self-resetting)
  // k-split form (ks > 1): the K blocks in ks equal ranges of nbk blocks, range r computed by the
  // gk workgroups r*gk .. r*gk+gk-1 over every tile; a tile's range partials are added in range
  // order by the last of its ks arrivals
  int ks, nbk, gk;
  f4_t* kpart;         // workspace: [tile][ks][NMAT][64 lanes]
  uint32_t* kcnt;      // workspace: arrival counter per tile (0 between calls, self-resetting)
};

// segment of launch tile t (wave-uniform)
__device__ __forceinline__ int seg_of(const SkArgs& a, int t) {
  return (t >= a.sT0[1]) + (t >= a.sT0[2]) + (t >= a.sT0[3]);
}

template <int NMAT>
struct Rec {
  u4_t A[NMAT];
  u2_t B[NMAT];
  uint32_t sc[NMAT];
  uint32_t d[NMAT];
};

// Buffer loads: the per-lane part of an address is a fixed VGPR, the per-record part a
// wave-uniform SGPR (soff), the field offset an immediate -- no per-load vector address math.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

template <int NMAT>
__device__ __forceinline__ void rec_load(Rec<NMAT>& r, const __amdgpu_buffer_rsrc_t* rs, int soff, int lane, int col) {
#pragma unroll
  for (int i = 0; i < NMAT; ++i) {
    r.A[i] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(rs[i], 16 * lane, soff, 0));
    r.B[i] = __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(rs[i], 8 * lane + 1024, soff, 0));
    r.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(rs[i], 4 * col + 1536, soff, 0);
    r.d[i] = __builtin_amdgcn_raw_buffer_load_b16(rs[i], 2 * col + 1600, soff, 0);
  }
}

// 12-bit field at bit P of the slot's 192-bit stream s[0..5], as a byte offset into the table
// (8-B entries)
template <int P>
__device__ __forceinline__ uint32_t field_off(const uint32_t* s) {
  constexpr int d = P >> 5, o = P & 31;
  if constexpr (o < 3) {
    return (s[d] << (3 - o)) & 0x7FF8u;
  } else if constexpr (o <= 20) {
    return (s[d] >> (o - 3)) & 0x7FF8u;
  } else {
    return __builtin_amdgcn_alignbit(s[d + 1], s[d], o - 3) & 0x7FF8u;
  }
}

__device__ __forceinline__ h8_t splat8(_Float16 v) { return h8_t{v, v, v, v, v, v, v, v}; }

template <int NMAT, int EPI>
__device__ __forceinline__ void epilogue(const SkArgs& a, const f4_t* acc, int tile, int col, int kq) {
  const int sg = seg_of(a, tile);
  const int n = (tile - a.sT0[sg]) * 16 + col;
  if (n >= a.sN[sg]) return;
  void* out = a.sout[sg];
  const int ld = a.sld[sg];
  if constexpr (EPI != EPI_RESID) {
    if (a.otile) {   // slot m of column group n / 8, every m: rows >= M hold row M-1's value
      uint16_t* o = reinterpret_cast<uint16_t*>(out) + (size_t)(n >> 3) * 128 + (n & 7);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * kq + r;
        o[8 * m] = EPI == EPI_SWIGLU ? tlx_swiglu_bits(acc[0][r], acc[NMAT - 1][r]) : tlx_f2h_bits(acc[0][r]);
      }
      return;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kq + r;
    if (m >= a.M) break;
    const size_t o = (size_t)m * ld + n;
    if constexpr (EPI == EPI_SWIGLU) {
      reinterpret_cast<uint16_t*>(out)[o] = tlx_swiglu_bits(acc[0][r], acc[1][r]);
    } else if constexpr (EPI == EPI_RESID) {
      reinterpret_cast<float*>(out)[o] = a.res[o] + (float)(_Float16)acc[0][r];
    } else {
      reinterpret_cast<uint16_t*>(out)[o] = tlx_f2h_bits(acc[0][r]);
    }
  }
}

// first unit of global wave gw (of GW): ranges are equal to within one unit
__device__ __forceinline__ int unit_of(int gw, int GW, int U) { return (int)(((long)gw * U) / GW); }

// Activations staged in LDS (rows of 2K + 16 bytes: the 16 rows one MFMA fragment reads are in
// distinct 16-B slots) when they fit; the partial tiles reuse the space after the loop.
constexpr int kXsBytes = 120 * 1024;
constexpr int kXsWaves = 8;                                   // workgroup size of the staged form
constexpr int kXsPer = kXsBytes / 16 / (kXsWaves * TLX_WAVE); // 16-B pieces per thread

template <int NMAT, int W, bool XL>
struct SkLds {
  u2_t tbl[kTblEntries];                 // first: table byte offsets are LDS addresses
  union {
    f4_t part[W][2][NMAT][TLX_WAVE];     // partial tiles: [wave][first | last tile]
    uint8_t xs[XL ? kXsBytes : 16];      // staged activations [M][2K + 16 B]
  };
};

// Contribution of one record to the lane's MFMA fragment(s): d/4 * sum_c X[c] . B_c, with B_c
// the chunk's 8 signed grid values times (2s+1) (exact fp16).
template <int NMAT>
__device__ __forceinline__ void rec_dot(f4_t* out, float* dq, const Rec<NMAT>& R, const h8_t* X, const uint8_t* tb,
                                        int kq) {
  // (2s+1) for the lane's two sub-blocks 2kq, 2kq+1; the 1/4 goes with d
  _Float16 ks[NMAT][2];
  uint32_t sv[NMAT][6];
#pragma unroll
  for (int i = 0; i < NMAT; ++i) {
    const uint32_t s2 = R.sc[i] >> (8 * kq);
    ks[i][0] = (_Float16)(float)(2u * (s2 & 15u) + 1u);
    ks[i][1] = (_Float16)(float)(2u * ((s2 >> 4) & 15u) + 1u);
    sv[i][0] = R.A[i].x; sv[i][1] = R.A[i].y; sv[i][2] = R.A[i].z; sv[i][3] = R.A[i].w;
    sv[i][4] = R.B[i].x; sv[i][5] = R.B[i].y;
    out[i] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  // chunk-major: the matrices' MFMA chains interleave, so consecutive MFMAs are independent
#define TLX_CHUNK(c)                                                                                   \
  _Pragma("unroll") for (int i = 0; i < NMAT; ++i) {                                                   \
    const u2_t lo = *reinterpret_cast<const u2_t*>(tb + field_off<24 * (c)>(sv[i]));                   \
    const u2_t hi = *reinterpret_cast<const u2_t*>(tb + field_off<24 * (c) + 12>(sv[i]));              \
    const h8_t Bv = __builtin_bit_cast(h8_t, u4_t{lo.x, lo.y, hi.x, hi.y}) * splat8(ks[i][(c) >> 2]);   \
    out[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(X[c], Bv, out[i], 0, 0, 0);                        \
  }
  TLX_CHUNK(0) TLX_CHUNK(1) TLX_CHUNK(2) TLX_CHUNK(3)
  TLX_CHUNK(4) TLX_CHUNK(5) TLX_CHUNK(6) TLX_CHUNK(7)
#undef TLX_CHUNK
#pragma unroll
  for (int i = 0; i < NMAT; ++i) dq[i] = tlx_h2f((uint16_t)R.d[i]) * 0.25f;
}

// first record of global wave gw: ranges are equal to within one record
__device__ __forceinline__ int range_begin(int gw, int GW, int U) { return unit_of(gw, GW, U); }

// XM: where the activations come from -- 0: x [M][K] in global memory, 1: the tile-ordered copy
// [K/8][16][8] in global memory, 2: x (or the copy's first M rows) staged into LDS by the
// workgroup (W == kXsWaves), every thread loading kXsPer pieces, 3: the same when fewer pieces are
// needed (small M: the loads past the end are skipped).  Staged activations are read from LDS at the point of use (no register
// copy), which leaves room for the shallower record ring below.
template <int NMAT, int EPI, int W, int XM, bool KS>
__global__ __launch_bounds__(W * TLX_WAVE) void iq3s_kernel(const SkArgs a) {
  constexpr bool XS = XM >= 2;   // staged in LDS
  __shared__ SkLds<NMAT, W, XS> L;
  constexpr bool XT = XM == 1;
  static_assert(!KS || NMAT == 1, "the k-split form is for single matrices");

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;
  // KS: record indices below are local to the workgroup's k-range: local record u = tile * nbl +
  // j is global record tile * nb + kr * nbl + j.  Without it they are the global records.
  const int nb = a.nb, nbl = KS ? a.nbk : nb;
  const int kr = KS ? (int)blockIdx.x / a.gk : 0, bx = (int)blockIdx.x - kr * a.gk;
  const int Ul = KS ? a.U / a.ks : a.U, GW = a.gk * W, gw = bx * W + wave;
  int ubeg = range_begin(gw, GW, Ul), uend = range_begin(gw + 1, GW, Ul);
  int last = max(min(uend, Ul) - 1, 0);
  if constexpr (KS) {
    // (pinned to scalar registers: the loop's record positions derive from them and are buffer
    // offsets, which must be scalar)
    ubeg = __builtin_amdgcn_readfirstlane(ubeg);
    uend = __builtin_amdgcn_readfirstlane(uend);
    last = __builtin_amdgcn_readfirstlane(last);
  }
  const bool empty = ubeg >= uend;   // only when there are fewer records than waves
  // Record positions: index u; with KS also its block j = u % nbl within tile t = u / nbl, which
  // the loop advances one record at a time (no divisions there: the load addresses wait on them).
  struct Pos { int u, j, t; };
  auto pos_at = [&](int u) {
    if constexpr (KS)
      return Pos{__builtin_amdgcn_readfirstlane(u), __builtin_amdgcn_readfirstlane(u % nbl),
                 __builtin_amdgcn_readfirstlane(u / nbl)};
    else
      return Pos{u, 0, 0};
  };
  auto advance = [&](Pos& p) {   // p + 1, held at the wave's last record
    // integer forms of the two conditions (no booleans: the compiler keeps those in vector
    // registers across the loop, which would make the record offsets per-lane)
    const int adv = (int)((uint32_t)(p.u - last) >> 31);       // 1 while p.u < last
    const int nj = p.j + adv;
    const int wrap = (int)((uint32_t)(nbl - 1 - nj) >> 31);    // 1 when nj == nbl
    p.u += adv;
    p.j = nj - wrap * nbl;
    p.t += wrap;
  };
  // KS: the loads cover records min(ubeg, last) .. last, at most two tiles (tA, tB), so at most
  // two segments, whose buffer resources and first records are set up here.
  int tA = 0, gA = 0, gB = 0;
  __amdgpu_buffer_rsrc_t rsA, rsB;
  if constexpr (KS) {
    tA = min(ubeg, last) / nbl;
    auto seg_rs = [&](int t, int& g0) {
      const int sg = seg_of(a, t);
      const int u0 = a.sT0[sg] * nb, u1 = min(a.sT0[sg + 1], a.U / nb) * nb;
      g0 = u0;
      return rsrc_of(a.sw[sg], (uint32_t)(u1 - u0) * kRec);
    };
    rsA = seg_rs(tA, gA);
    rsB = seg_rs(last / nbl, gB);
  }
  // record at p: segment, buffer resource(s) and offset (all wave-uniform, in SGPRs)
  auto rload = [&](Rec<NMAT>& R, const Pos& p) {
    __amdgpu_buffer_rsrc_t rs[NMAT];
    int soff;
    if constexpr (KS) {
      const int g = p.t * nb + kr * nbl + p.j;
      const bool inA = p.t == tA;
      rs[0] = inA ? rsA : rsB;
      soff = (g - (inA ? gA : gB)) * (int)kRec;
    } else if constexpr (NMAT == 2) {
      rs[0] = rsrc_of(a.sw[0], (uint32_t)a.U * kRec);
      rs[1] = rsrc_of(a.w1, (uint32_t)a.U * kRec);
      soff = p.u * (int)kRec;
    } else {
      const int sg = seg_of(a, p.u / nb);
      const int u0 = a.sT0[sg] * nb, u1 = min(a.sT0[sg + 1], a.U / nb) * nb;
      rs[0] = rsrc_of(a.sw[sg], (uint32_t)(u1 - u0) * kRec);
      soff = (p.u - u0) * (int)kRec;
    }
    rec_load<NMAT>(R, rs, soff, lane, col);
  };
  // activations: block b, chunk c of lane (col, kq) at byte xv + b * xbs + c * xcs
  constexpr int xbs = XT ? 8192 : 512, xcs = XT ? 256 : 16;
  const __amdgpu_buffer_rsrc_t rx = rsrc_of(a.x, a.xt ? (uint32_t)a.K * 32u : (uint32_t)(a.M * a.K) * 2u);
  const int xv = XT ? 2 * (1024 * kq + 8 * col) : 2 * (min(col, a.M - 1) * a.K + 64 * kq);
  const int xstr = 512 * nbl + 16;                                // staged row bytes (the range's k)
  const uint8_t* xsl = L.xs + min(col, a.M - 1) * xstr + 128 * kq;  // this lane's row, k = 64kq
  auto xload = [&](h8_t* X, const Pos& p) {
    const int b = KS ? kr * nbl + p.j : p.u % nb;
#pragma unroll
    for (int c = 0; c < 8; ++c)
      X[c] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, xv + xcs * c, xbs * b, 0));
  };

  // Record ring of RING buffers: record s is requested RING - 1 records ahead of its use.  With
  // activations from global memory (4 buffers) they are loaded one unit ahead (2 sets), issue order
  // X(s+1), R(s+3), X(s+2), R(s+4), ...: the wait for record s and X(s) leaves the next three
  // records and X(s+1) in flight.  With staged activations the ring is 2 deep: measured faster than
  // 3, 4, 6 or 8 (each wave streams only ~10 records, and requesting more of them up front made
  // the whole launch slower).  The first loads are issued before the table is built (their latency
  // covers it); the grid words the thread turns into table entries are loaded first, so waiting for
  // them leaves the records in flight.
  constexpr int kGw = 1024 / (W * TLX_WAVE);   // grid words (x 4 sign nibbles) per thread
  float4 gv[kGw];
  // staged activations: 16-B pieces p = thread + j * blockDim of x (past the end: the last piece;
  // loads stay unconditional, a repeated piece is stored twice with the same bytes)
  constexpr int kXp = XS ? kXsPer : 1;
  u4_t xp[kXp];
  const int kp = 32 * nbl;   // 16-B pieces per staged row
  const int npc = a.M * kp;
  // Staged piece p (8 k of one row).  Row-major x is read row by row (p = row * kp + k8); the
  // tile-ordered copy [K/8][16][8] k-group by k-group (p = k8 * M + row: consecutive threads read
  // consecutive 16-B rows of a 256-B group).  With p = hi * D + lo, the source piece index and the
  // LDS byte offset are linear in (hi, lo) with per-form coefficients, and a thread's pieces step
  // by the workgroup size, so (hi, lo) advance by (qB, rB) with one carry: no divisions and no
  // branches per piece.  xd: the pieces' LDS byte offsets, for the stores after the table build.
  int xd[kXp];
  if constexpr (XS) {
    const bool xt = a.xt != 0;
    constexpr int B = W * TLX_WAVE;
    const int D = xt ? a.M : kp, qB = B / D, rB = B - qB * D;
    const int sH = xt ? 16 : a.K / 8, s0 = xt ? kr * kp * 16 : kr * kp;
    const int dH = xt ? 16 : xstr, dL = xt ? xstr : 16;
    // past the end: the last piece (row M - 1, k8 kp - 1)
    const int srcL = xt ? 16 * ((kr * kp + kp - 1) * 16 + a.M - 1) : 16 * ((a.M - 1) * (a.K / 8) + kr * kp + kp - 1);
    const int dstL = (a.M - 1) * xstr + 16 * (kp - 1);
    int hi = (int)threadIdx.x / D, lo = (int)threadIdx.x - hi * D;
#pragma unroll
    for (int j = 0; j < kXp; ++j) {
      // (XM 3: the pieces past the end are skipped by a uniform test, not a break: with the
      // loop-carried (hi, lo) a break keeps the loop from unrolling and xp / xd in registers)
      if (XM != 3 || j * B < npc) {
        const bool in = (int)threadIdx.x + j * B < npc;
        xd[j] = in ? hi * dH + lo * dL : dstL;
        xp[j] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                             rx, in ? 16 * (hi * sH + lo + s0) : srcL, 0, 0));
      }
      lo += rB;
      hi += qB;
      const int carry = lo >= D ? 1 : 0;
      lo -= carry * D;
      hi += carry;
    }
  }
#pragma unroll
  for (int j = 0; j < kGw; ++j) gv[j] = reinterpret_cast<const float4*>(a.gridf)[(threadIdx.x + j * W * TLX_WAVE) & 255];
  // (scheduling barriers keep each record's loads together and the records in order: the wait
  // counts in the loop assume that order on entry)
  constexpr int RING = XS ? 2 : 4;
  Rec<NMAT> R[RING];
  h8_t X[XS ? 1 : 2][8];
  __builtin_amdgcn_sched_barrier(0);
  rload(R[0], pos_at(min(ubeg, last)));
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!XS) xload(X[0], pos_at(min(ubeg, last)));
#pragma unroll
  for (int j = 1; j < RING; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    rload(R[j], pos_at(min(ubeg + j, last)));
  }
  // the loop's positions: next record load, next activation load, record computed
  Pos pr = pos_at(min(ubeg + RING, last)), px = pos_at(min(ubeg + 1, last)), ps = pos_at(min(ubeg, last));
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (XS) {
#pragma unroll
    for (int j = 0; j < kXp; ++j) {
      if (XM != 3 || j * W * TLX_WAVE < npc) *reinterpret_cast<u4_t*>(L.xs + xd[j]) = xp[j];
    }
  }
#pragma unroll
  for (int j = 0; j < kGw; ++j) {
    const int e = threadIdx.x + j * W * TLX_WAVE;   // grid word e & 255, sign nibbles 4(e >> 8) ..
    tlx_iq3_table_entries(L.tbl, gv[j], e & 255, e >> 8);
  }
  __syncthreads();
  const uint8_t* tb = reinterpret_cast<const uint8_t*>(L.tbl);

  // a wave touches at most two tiles: records < split belong to the first
  const int tfirst = ubeg / nbl, tlast = empty ? tfirst : (uend - 1) / nbl;
  const int split = min(uend, (tfirst + 1) * nbl);
  f4_t accA[NMAT], accB[NMAT];
#pragma unroll
  for (int i = 0; i < NMAT; ++i) accA[i] = accB[i] = f4_t{0.f, 0.f, 0.f, 0.f};
  auto accum = [&](const f4_t* D, const float* dq, int s) {
    // wave-uniform 0/1 factors on the block scale pick the tile (no branch in the loop)
    const float fA = s < split ? 1.f : 0.f;
    const float fB = s >= split ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      accA[i] += (dq[i] * fA) * D[i];
      accB[i] += (dq[i] * fB) * D[i];
    }
  };
  // activations of record s: staged rows in LDS (read at the point of use), else the register set
  auto xsrc = [&](const Pos& p, int j) -> const h8_t* {
    if constexpr (XS) return reinterpret_cast<const h8_t*>(xsl + 512 * (KS ? p.j : p.u % nb));
    else return X[j & 1];
  };
  // full rounds of RING records: branch-free (a branch in the loop makes the wait counts conservative)
  const int nfull = empty ? 0 : (uend - ubeg) / RING * RING;
  for (int u = ubeg; u < ubeg + nfull; u += RING) {
#pragma unroll
    for (int j = 0; j < RING; ++j) {
      const int s = u + j;
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (!XS) {
        if constexpr (!KS) px.u = min(s + 1, last);
        xload(X[(j + 1) & 1], px);
        if constexpr (KS) advance(px);
      }
      f4_t D[NMAT];
      float dq[NMAT];
      if constexpr (!KS) ps.u = s;
      rec_dot<NMAT>(D, dq, R[j], xsrc(ps, j), tb, kq);
      if constexpr (XS && KS) advance(ps);   // (held only past the last record, where it is unused)
      accum(D, dq, s);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (!KS) pr.u = min(s + RING, last);
      rload(R[j], pr);
      if constexpr (KS) advance(pr);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // the last 0..RING-1 records: already in R[0..RING-2] (and X[0]); nothing more to load
  const int rem = empty ? 0 : (uend - ubeg) - nfull;
  const int ut = ubeg + nfull;
#pragma unroll
  for (int j = 0; j < RING - 1; ++j) {
    if (j < rem) {
      f4_t D[NMAT];
      float dq[NMAT];
      if constexpr (!XS) {
        if (j > 0) xload(X[j & 1], pos_at(ut + j));
      }
      rec_dot<NMAT>(D, dq, R[j], xsrc(pos_at(ut + j), j), tb, kq);
      accum(D, dq, ut + j);
    }
  }
  if constexpr (XS) __syncthreads();   // the parts overwrite the staged activations
  if (!empty) {
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      L.part[wave][0][i][lane] = accA[i];
      L.part[wave][1][i][lane] = accB[i];
    }
  }
  __syncthreads();

  // each tile is finished by the lowest wave of the workgroup that touches it: that wave adds
  // the parts of the waves touching the tile in wave order
  // a tile's sum is final here without the k-split; with it, it is this range's partial: store it,
  // count the arrival, and the last of the tile's ks ranges adds them in range order (same
  // ordering argument as the boundary parts below)
  auto finish = [&](f4_t* acc, int t) {
    if constexpr (!KS) {
      epilogue<NMAT, EPI>(a, acc, t, col, kq);
      return;
    }
    uint64_t* kp = reinterpret_cast<uint64_t*>(a.kpart + (size_t)t * a.ks * NMAT * TLX_WAVE);
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      const u4_t v = __builtin_bit_cast(u4_t, acc[i]);
      uint64_t* q = kp + 2 * ((kr * NMAT + i) * TLX_WAVE + lane);
      __hip_atomic_store(q, (uint64_t)v.x | (uint64_t)v.y << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(q + 1, (uint64_t)v.z | (uint64_t)v.w << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0x0F70);                    // vmcnt(0): the partial's stores are done
    uint32_t prev = 0;   // 0 -> 1 -> .. -> ks-1 -> 0: the last arrival leaves the counter at 0
    if (lane == 0) prev = __builtin_amdgcn_atomic_inc32(&a.kcnt[t], (uint32_t)(a.ks - 1), __ATOMIC_RELAXED, "agent");
    prev = __shfl(prev, 0);
    if (prev != (uint32_t)(a.ks - 1)) return;
    f4_t sum[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; ++i) sum[i] = f4_t{0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < a.ks; ++r)
#pragma unroll
      for (int i = 0; i < NMAT; ++i) {
        const uint64_t* q = kp + 2 * ((r * NMAT + i) * TLX_WAVE + lane);
        const uint64_t w0 = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t w1 = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sum[i] += __builtin_bit_cast(f4_t, u4_t{(uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32)});
      }
    epilogue<NMAT, EPI>(a, sum, t, col, kq);
  };

  const int GWb = bx * W;
  const int u0 = range_begin(GWb, GW, Ul), u1 = range_begin(GWb + W, GW, Ul);
  for (int k = 0; k < (empty ? 0 : 2); ++k) {
    const int t = k == 0 ? tfirst : tlast;
    if (k == 1 && tlast == tfirst) break;
    // a lower wave of the workgroup touches it (the one holding record ubeg - 1; waves between
    // may be empty when the workgroup has fewer records than waves)
    if (k == 0 && ubeg > u0 && ubeg % nbl != 0) continue;
    f4_t acc[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; ++i) acc[i] = f4_t{0.f, 0.f, 0.f, 0.f};
    for (int v = wave; v < W; ++v) {
      const int vb = range_begin(GWb + v, GW, Ul);
      if (vb >= (t + 1) * nbl) break;
      if (range_begin(GWb + v + 1, GW, Ul) == vb) continue;   // an empty range
      const int slot = vb / nbl == t ? 0 : 1;
#pragma unroll
      for (int i = 0; i < NMAT; ++i) acc[i] += L.part[v][slot][i][lane];
    }
    const bool lo_out = t * nbl < u0, hi_out = (t + 1) * nbl > u1;
    if (!lo_out && !hi_out) {
      finish(acc, t);
      continue;
    }
    // shared with the neighbouring workgroup: boundary g = the upper workgroup's index; part 0
    // holds the lower workgroup's (earlier k) sum, part 1 the upper's
    const int g = lo_out ? (int)blockIdx.x : (int)blockIdx.x + 1;
    // Ordering argument.  Every access to the parts and the counter is an agent-scope atomic
    // (coherent across the XCDs' L2s by itself), so no cache-wide write-back or invalidate is
    // needed (an agent-scope release fence would write back each XCD's whole L2).  What is needed
    // is that this wave's part stores have COMPLETED before the counter moves: the workgroup-scope
    // fence orders them for the compiler only (it emits no wait on gfx950), so the wave waits for
    // its outstanding vector-memory operations explicitly (vmcnt counts stores on gfx9).  The
    // second arriver's part loads issue only after the counter's old value has come back (they
    // sit behind the branch on it), i.e. after the first arriver's increment, which followed the
    // completion of the first arriver's stores.
    uint64_t* pp = reinterpret_cast<uint64_t*>(a.part + (size_t)g * 2 * NMAT * TLX_WAVE);
    const int mine = lo_out ? 1 : 0;
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      const u4_t v = __builtin_bit_cast(u4_t, acc[i]);
      uint64_t* q = pp + 2 * ((mine * NMAT + i) * TLX_WAVE + lane);
      __hip_atomic_store(q, (uint64_t)v.x | (uint64_t)v.y << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(q + 1, (uint64_t)v.z | (uint64_t)v.w << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0x0F70);                    // vmcnt(0): the part stores are done
    // Self-resetting arrival count: inc with limit 1 maps 0 -> 1 (first arriver) and 1 -> 0
    // (second arriver), so every completed call leaves each counter at 0 without a reset store.
    uint32_t prev = 0;
    if (lane == 0) prev = __builtin_amdgcn_atomic_inc32(&a.cnt[g], 1u, __ATOMIC_RELAXED, "agent");
    prev = __shfl(prev, 0);
    if (prev != 1u) continue;                              // the other part is not there yet
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      uint64_t w[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t* q = pp + 2 * ((h * NMAT + i) * TLX_WAVE + lane);
        w[h][0] = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        w[h][1] = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const f4_t lo = __builtin_bit_cast(f4_t, u4_t{(uint32_t)w[0][0], (uint32_t)(w[0][0] >> 32),
                                                    (uint32_t)w[0][1], (uint32_t)(w[0][1] >> 32)});
      const f4_t hi = __builtin_bit_cast(f4_t, u4_t{(uint32_t)w[1][0], (uint32_t)(w[1][0] >> 32),
                                                    (uint32_t)w[1][1], (uint32_t)(w[1][1] >> 32)});
      acc[i] = lo + hi;                                    // lower range first: a fixed order
    }
    finish(acc, t);
  }
}

// staged row bytes for nbk blocks of k per row
__host__ __device__ constexpr int xs_row_bytes(int nbk) { return 512 * nbk + 16; }

template <int NMAT, int EPI, int W, bool KS>
void sk_launch_x(const SkArgs& a, hipStream_t st) {
  if constexpr (W == kXsWaves) {
    if (a.M * xs_row_bytes(a.nbk) <= kXsBytes) {   // from x or its tile-ordered copy
      // all kXsPer pieces per thread needed, or fewer (skip the loads past the end)
      if (a.M * 32 * a.nbk > (kXsPer - 1) * W * TLX_WAVE) iq3s_kernel<NMAT, EPI, W, 2, KS><<<a.G, W * TLX_WAVE, 0, st>>>(a);
      else iq3s_kernel<NMAT, EPI, W, 3, KS><<<a.G, W * TLX_WAVE, 0, st>>>(a);
      return;
    }
  }
  if (a.xt) iq3s_kernel<NMAT, EPI, W, 1, KS><<<a.G, W * TLX_WAVE, 0, st>>>(a);
  else iq3s_kernel<NMAT, EPI, W, 0, KS><<<a.G, W * TLX_WAVE, 0, st>>>(a);
}

template <int NMAT, int EPI, int W>
void sk_launch(const SkArgs& a, hipStream_t st) {
  if constexpr (NMAT == 1 && W == kXsWaves) {
    if (a.ks > 1) return sk_launch_x<NMAT, EPI, W, true>(a, st);
  }
  sk_launch_x<NMAT, EPI, W, false>(a, st);
}

template <int NMAT, int EPI>
int sk_dispatch(int W, const SkArgs& a, hipStream_t st) {
  switch (W) {
    case 8: sk_launch<NMAT, EPI, 8>(a, st); break;
    case 4: sk_launch<NMAT, EPI, 4>(a, st); break;
    default: sk_launch<NMAT, EPI, 1>(a, st); break;
  }
  return tlx_launch_status();
}

constexpr int kWd = 8;   // 2 waves per SIMD, ~130-180 VGPRs each: the record ring and two activation sets
constexpr int kKs = 4;   // k-ranges of the k-split form

// k-ranges of a launch.  Long-K single matrices (the down and output projections) have few tiles
// for 256 workgroups and long per-wave record streams; splitting K into kKs ranges, each covered
// by a quarter of the workgroups over every tile, shortens the streams and the activation slice
// each workgroup stages.  It needs whole-block ranges, the workspace's range-partial region, and
// no more tiles than a quarter of the grid keeps within two tiles per wave.  Depends on (N, K,
// the CU count) only, so a row's summation order is the same for every M.
int sk_ranges(int nmat, int nseg, int N, int K, bool kparts) {
  const int G0 = std::min(tlx_cu_count(), kMaxG), gk = G0 / kKs, T = (N + 15) / 16, nb = K / 256;
  if (!kparts || nmat != 1 || nseg != 1 || K < 5632 || nb % kKs != 0 || gk < 1) return 1;
  if (T < gk || T > gk * kWd) return 1;
  if ((size_t)T * 4 > kWsKcntBytes || (size_t)T * kKs * TLX_WAVE * sizeof(f4_t) > kWsKpartBytes) return 1;
  return kKs;
}

}  // namespace

// True when the tiled-record GEMV stages x [M][K] (each workgroup its k-range) in LDS itself (no
// tile-ordered copy needed).
bool tlx_iq3s_stages_x(int nmat, int M, int N, int K, int nseg, bool ws_kparts) {
  const int ks = sk_ranges(nmat, nseg, N, K, ws_kparts);
  return M * xs_row_bytes(K / 256 / ks) <= kXsBytes;
}

// Balanced GEMV over tiled records (called by the IQ3_XXS entry points of tlx_iq3.hip, which
// have validated the arguments and prepared x / xt).  nmat 2 = SwiGLU pair (one segment), epi as
// Epi; nseg matrices w[s] of n[s] rows (NMAT == 1, EPI_F16 when nseg > 1) share the activations.
int tlx_iq3s_launch(int nmat, int epi, int nseg, const void* const* w, const void* w1, void* const* out,
                    const int* n, const float* res, const float* gridf, const _Float16* x, int xt, int M, int K,
                    void* ws, bool ws_kparts, bool out_tileord, hipStream_t st) {
  TLX_RET_IF(ws == nullptr, TLX_E_NOWS);
  TLX_RET_IF(out_tileord && (nseg != 1 || epi == EPI_RESID), TLX_E_ARG);
  static_assert(size_t(kMaxG) * 2 * 2 * TLX_WAVE * sizeof(f4_t) <= kWsCntOff - kWsPartOff, "parts region");
  static_assert(size_t(kMaxG) * 4 <= kWsCntBytes, "counter region");
  TLX_RET_IF(nseg < 1 || nseg > kMaxSeg || (nseg > 1 && (nmat != 1 || epi != EPI_F16)), TLX_E_ARG);
  SkArgs a{};
  a.w1 = (const uint8_t*)w1;
  a.res = res;
  a.gridf = gridf;
  a.x = x;
  a.xt = xt;
  a.otile = out_tileord ? 1 : 0;
  a.M = M;
  a.K = K;
  a.nb = K / 256;
  a.part = reinterpret_cast<f4_t*>(static_cast<uint8_t*>(ws) + kWsPartOff);
  a.cnt = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + kWsCntOff);
  a.kpart = reinterpret_cast<f4_t*>(static_cast<uint8_t*>(ws) + kWsKpartOff);
  a.kcnt = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + kWsKcntOff);
  const int nb = a.nb;
  const int G0 = std::min(tlx_cu_count(), kMaxG);
  constexpr int Wd = kWd;
  const int Tmax = G0 * Wd;   // a launch covers at most G0 * Wd tiles, so a wave touches <= 2 tiles
  const int ks = sk_ranges(nmat, nseg, n[0], K, ws_kparts);

  auto run = [&](SkArgs& b, int T) {
    b.U = T * nb;
    int W = Wd;
    if (ks > 1) {
      // kKs groups of G0 / kKs workgroups, group r over k-range r of every tile (gk <= T: a tile
      // spans at most two workgroups of its group; T <= gk * Wd: a wave touches <= 2 tiles)
      b.ks = ks;
      b.nbk = nb / ks;
      b.gk = G0 / ks;
      b.G = b.gk * ks;
    } else {
      // every wave gets >= 1 record; G <= T makes a workgroup cover >= nb records, so a tile
      // spans at most two workgroups
      int G = std::min(G0, T);
      if (b.U < G * W) G = std::max(1, b.U / W);
      while (W > 1 && b.U < G * W) W = W > 4 ? W / 2 : 1;
      b.ks = 1;
      b.nbk = nb;
      b.gk = b.G = G;
    }
    if (nmat == 2) return sk_dispatch<2, EPI_SWIGLU>(W, b, st);
    if (epi == EPI_RESID) return sk_dispatch<1, EPI_RESID>(W, b, st);
    return sk_dispatch<1, EPI_F16>(W, b, st);
  };
  auto reset = [](SkArgs& b) {
    for (int k = 0; k <= kMaxSeg; ++k) b.sT0[k] = 0x7fffffff;
  };

  int T = 0;
  for (int k = 0; k < nseg; ++k) T += (n[k] + 15) / 16;
  if (nseg > 1 && T <= Tmax) {   // one launch over the concatenated tiles
    SkArgs b = a;
    reset(b);
    b.nseg = nseg;
    int t0 = 0;
    for (int k = 0; k < nseg; ++k) {
      b.sw[k] = (const uint8_t*)w[k];
      b.sout[k] = out[k];
      b.sN[k] = n[k];
      b.sld[k] = n[k];
      b.sT0[k] = t0;
      t0 += (n[k] + 15) / 16;
    }
    b.sT0[nseg] = t0;
    return run(b, t0);
  }
  // one matrix at a time, each in launches of <= Tmax tiles
  const size_t osz = epi == EPI_RESID ? 4 : 2;
  for (int k = 0; k < nseg; ++k) {
    const int Tk = (n[k] + 15) / 16;
    for (int t0 = 0; t0 < Tk; t0 += Tmax) {
      const int T1 = std::min(Tk - t0, Tmax);
      const size_t rec0 = (size_t)t0 * nb * kRec;
      SkArgs b = a;
      reset(b);
      b.nseg = 1;
      b.sw[0] = (const uint8_t*)w[k] + rec0;
      b.w1 = a.w1 ? a.w1 + rec0 : nullptr;
      // row-major: column offset t0 * 16; tile-ordered: column groups 2 t0 of 256 B each
      b.sout[0] = (uint8_t*)out[k] + (out_tileord ? (size_t)t0 * 512 : (size_t)t0 * 16 * osz);
      b.sN[0] = std::min(n[k] - t0 * 16, T1 * 16);
      b.sld[0] = n[k];
      b.sT0[0] = 0;
      b.sT0[1] = T1;
      b.res = res ? res + (size_t)t0 * 16 : nullptr;
      const int r = run(b, T1);
      TLX_RET_IF(r != TLX_OK, r);
    }
  }
  return TLX_OK;
}

extern "C" uint64_t tlx_iq3_tiled_bytes(int N, int K) {
  if (N < 1 || K < 256 || (K % 256)) return 0;
  return (uint64_t)((N + 15) / 16) * (uint64_t)(K / 256) * kRec;
}

extern "C" int tlx_pack_iq3_tiled(const void* src, void* tiled, int N, int K, int src_layout, void* stream) {
  TLX_RET_IF(N < 1 || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(src_layout != TLX_LAYOUT_RAW && src_layout != TLX_LAYOUT_PACKED, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(src, 2) || !tlx_aligned(tiled, 16), TLX_E_ALIGN);
  const long nslots = (long)((N + 15) / 16) * (K / 256) * 64;
  pack_tiled_kernel<<<(unsigned)((nslots + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)src, (uint8_t*)tiled, nslots, N, K / 256, src_layout == TLX_LAYOUT_RAW);
  return tlx_launch_status();
}
