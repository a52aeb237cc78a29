// MoE grouped-expert path for gfx950 (the reference's mm/ family): router top-8 + softmax,
// deterministic expert sort, grouped IQ4_XS gate+up (SwiGLU) and down GEMMs on MFMA, and the
// combine with the shared expert and the residual.
//
// Layouts (as the reference): routed expert e's gate/up slab at ptbl[e] -- 512 gate rows then
// 512 up rows (GATE_B4 = 557,056 bytes apart), 1088 B per row (8 IQ4_XS blocks of 136 B,
// k = 2048); its down slab at ptbl_dn[e] -- 2048 rows x 272 B (k = 512).  Pairs are
// position-major, rank ascending: pair = 8 * pos + rank.
// Tiled slabs (TLX_LAYOUT_TILED, this library's own; tlx_pack_iq4_tiled): the same bytes per
// (16-row tile t, 256-k block b) record of 2176 B, records in (t, b) order (so a slab keeps its
// size and the up rows still start GATE_B4 bytes in):
//   [0, 128)      row r's block header (d, scales_h, scales_l) at 8 r
//   [128, 1152)   lane l = 16 kq + r: row r's quant bytes 16 kq .. 16 kq + 15 (sub-block kq)
//   [1152, 2176)  lane l: row r's quant bytes 64 + 16 kq .. (sub-block kq + 4)
// i.e. the bytes each MFMA lane decodes, in lane order: every wave load reads one contiguous run
// (in GGUF rows the 4 lanes of a 64-B load request touch 4 rows).
//
// Grouped GEMMs: a GEMV form for small batches and a GEMM form for prefill (see each kernel).
// IQ4_XS decode: a 256-entry table maps a quant byte to (kv[lo], kv[hi]) as fp16, so one lookup
// yields the two weights that byte holds (elements j and j+16 of the group); the MFMA k order is
// chosen to pair them (the activations follow the same order), and the group scale d*(ls-32)
// multiplies in fp16.
#include "tlx_common.h"

#include <type_traits>

namespace {

constexpr int kE = 256, kTopK = 8, kHid = 2048, kFf = 512;
constexpr int kGateBytes = kFf * 1088;     // GATE_B4

// ------------------------------------------------------------------ router
// 8 masked-argmax passes over one position's 256 logits held 4 per lane (lane l: experts
// l, l+64, l+128, l+192), wave-wide: larger value wins, equal values go to the lower id.
__device__ __forceinline__ void topk8_wave(float v[4], int lane, uint16_t* eids, float* gates) {
  float m = -3.402823466e38f, ex[kTopK], s8 = 0.f;
  int ids[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    float bv = v[0];
    int bi = lane;
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (r == 0) m = bv;
    ids[r] = bi;
    ex[r] = expf(bv - m);
    s8 += ex[r];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (bi == lane + 64 * j) v[j] = -3.402823466e38f;
  }
  if (lane < kTopK) {
    int id = ids[0];
    float e = ex[0];
#pragma unroll
    for (int r = 1; r < kTopK; ++r)
      if (lane == r) { id = ids[r]; e = ex[r]; }
    eids[lane] = (uint16_t)id;
    gates[lane] = e / s8;
  }
}

// The same 8 passes with a position per 16-lane row (lane l: experts 16 l .. 16 l + 15): the row's
// argmax is 4 DPP exchange steps inside the row (quad swaps, half-row and row mirrors) instead of
// 6 cross-lane shuffles over the wave, which go through the LDS crossbar and serialize 96 round
// trips per position.  Same comparisons, same order of the softmax sums: the same results.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& bv, int& bi) {
  const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, bv), CTRL, 0xF, 0xF, true));
  const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xF, 0xF, true);
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

__device__ __forceinline__ void topk8_row16(const float4 (&in)[4], int l, uint16_t* eids, float* gates) {
  float v[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) { v[4 * q] = in[q].x; v[4 * q + 1] = in[q].y; v[4 * q + 2] = in[q].z; v[4 * q + 3] = in[q].w; }
  float m = -3.402823466e38f, ex[kTopK], s8 = 0.f;
  int ids[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    float bv = v[0];
    int bi = 16 * l;
#pragma unroll
    for (int j = 1; j < 16; ++j)
      if (v[j] > bv) { bv = v[j]; bi = 16 * l + j; }
    argmax_dpp_step<0xB1>(bv, bi);    // quad_perm [1, 0, 3, 2]
    argmax_dpp_step<0x4E>(bv, bi);    // quad_perm [2, 3, 0, 1]
    argmax_dpp_step<0x141>(bv, bi);   // row_half_mirror: quad q with quad 1 - q of each half
    argmax_dpp_step<0x140>(bv, bi);   // row_mirror: half with half
    if (r == 0) m = bv;
    ids[r] = bi;
    ex[r] = expf(bv - m);
    s8 += ex[r];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (bi == 16 * l + j) v[j] = -3.402823466e38f;
  }
  if (l < kTopK) {
    int id = ids[0];
    float e = ex[0];
#pragma unroll
    for (int r = 1; r < kTopK; ++r)
      if (l == r) { id = ids[r]; e = ex[r]; }
    eids[l] = (uint16_t)id;
    gates[l] = e / s8;
  }
}

// a position per 16-lane row, 16 positions per 256-thread workgroup
__global__ __launch_bounds__(256) void moe_topk_kernel(const float* __restrict__ logits, uint16_t* __restrict__ eids,
                                                       float* __restrict__ gates, int P) {
  const int p = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
  if (p >= P) return;   // whole 16-lane rows: the exchanges stay inside a row
  float4 in[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) in[q] = reinterpret_cast<const float4*>(logits + (size_t)p * kE + 16 * l)[q];
  topk8_row16(in, l, eids + (size_t)p * kTopK, gates + (size_t)p * kTopK);
}

// rt8e256: logits = wrt . h, shared gate sg = sigmoid(wsh . h), then the top-8.  One 256-thread
// workgroup per position; logit e is thread e's fixed-order sum (4-way split of k, then the
// partials in order), the shared gate a fixed-order tree.
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ wrt, const float* __restrict__ wsh,
                                                        const float* __restrict__ h, uint16_t* __restrict__ eids,
                                                        float* __restrict__ gates, float* __restrict__ sg) {
  __shared__ float lg[kE];
  __shared__ float shp[256];
  const int p = blockIdx.x, t = threadIdx.x;
  const float4* hr = reinterpret_cast<const float4*>(h + (size_t)p * kHid);
  {
    const float4* wr = reinterpret_cast<const float4*>(wrt + (size_t)t * kHid);
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int i = 0; i < kHid / 16; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 w = wr[q * (kHid / 16) + i], x = hr[q * (kHid / 16) + i];
        part[q] += w.x * x.x + w.y * x.y + w.z * x.z + w.w * x.w;
      }
    }
    lg[t] = ((part[0] + part[1]) + part[2]) + part[3];
    const float2* ws2 = reinterpret_cast<const float2*>(wsh);
    const float2* hr2 = reinterpret_cast<const float2*>(h + (size_t)p * kHid);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 a = ws2[t + 256 * i], b = hr2[t + 256 * i];
      s += a.x * b.x + a.y * b.y;
    }
    shp[t] = s;
  }
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (t < w) shp[t] += shp[t + w];
    __syncthreads();
  }
  if (t < 64) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = lg[t + 64 * j];
    topk8_wave(v, t, eids + (size_t)p * kTopK, gates + (size_t)p * kTopK);
    if (t == 0) sg[p] = 1.f / (1.f + expf(-shp[0]));
  }
}

// ------------------------------------------------------------------ sort
// Deterministic stable counting sort by expert over many workgroups, one launch: workgroup c
// owns pairs [256 c, 256 c + 256).  Every workgroup reads all np keys and counts them per expert
// twice in LDS -- all pairs, and the pairs before its chunk -- with atomic increments (a count does
// not depend on their order); a scan over the experts of the totals gives the bins (expert
// ascending), and bin e's slots for this chunk start after the bin start and the earlier chunks'
// pairs of e.  Inside the chunk, wave w ranks its 64 pairs by 8 ballots over the key bits (the
// lanes holding the same key; rank = those below), after the earlier waves' pairs of each key.
// Bins are therefore in pair order, stable like mmsort8.  Workgroup 0 writes eoff, the items and
// their count.  Items: per expert ceil(count / tok) chunks of its pairs, expert ascending, item =
// expert << 16 | first pair offset, tok = moe_item_tok(np).
constexpr int kMaxPairs = 16384;
constexpr int kTok = 64;         // item size of the GEMV form, and its dense (shared expert) chunk
constexpr int kDenseTok = 32;    // the GEMM form's dense chunk: 2 groups, so the shared expert's
                                 // grids fill the GPU beside the router and the sort
constexpr int kPfTok = 96;       // item size of the GEMM form: up to 6 groups of 16 tokens
// Form per projection by pair count (measured over 4..2048 pairs, tiled slabs): the gate+up GEMV
// form up to 512 pairs (items of 64 pairs), the MFMA form above (items of 96); the down GEMV form
// up to 160 pairs, the act-resident MFMA form above (on the same items).  The shared expert runs
// its GEMV form up to 256 positions.
constexpr int kGvUpMaxPairs = 512;
constexpr int kGvDnMaxPairs = 160;
constexpr int kGvSharedMaxP = 256;
constexpr int kShTok = 16;          // positions per shared-expert chunk of the fused pair walk
constexpr int kSortChunk = 256;     // pairs per sort workgroup (4 waves of 64)

// pairs per work item: 64 up to kGvUpMaxPairs pairs (the gate+up GEMV form's limit; the down
// projection's MFMA form takes the same items), 96 above (at uniform routing over 256 experts an
// expert's count exceeds 96 with odds of ~1e-4, so its weights are streamed once)
__host__ __device__ constexpr int moe_item_tok(int np) { return np <= kGvUpMaxPairs ? kTok : kPfTok; }

// lanes of this wave holding the same 8-bit key as this lane
__device__ __forceinline__ uint64_t same_key_mask(uint32_t key) {
  uint64_t m = ~0ull;
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint64_t bal = __ballot((key >> b) & 1u);
    m &= ((key >> b) & 1u) ? bal : ~bal;
  }
  return m;
}

__global__ __launch_bounds__(kSortChunk) void moe_sort_kernel(const uint16_t* __restrict__ eids, int* __restrict__ eoff,
                                                              uint16_t* __restrict__ plist, uint32_t* __restrict__ items,
                                                              uint32_t* __restrict__ nitp, int np) {
  __shared__ int tot[kE];         // pairs of expert e, all chunks
  __shared__ int pre[kE];         // pairs of expert e in the chunks before this one
  __shared__ int cw[4][kE];       // pairs of expert e in each wave of this chunk
  __shared__ int wsum[4][2];      // per-wave totals of the expert scans
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int c0 = (int)blockIdx.x * kSortChunk;
  tot[t] = 0;
  pre[t] = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) cw[w][t] = 0;
  __syncthreads();
  // ---- count all keys (4 per thread and step; the tail key by key)
  const int nq = np >> 2;
  for (int q = t; q < nq; q += kSortChunk) {
    const uint2 k4 = reinterpret_cast<const uint2*>(eids)[q];
    const uint32_t ks[4] = {k4.x & 0xFFu, (k4.x >> 16) & 0xFFu, k4.y & 0xFFu, (k4.y >> 16) & 0xFFu};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      atomicAdd(&tot[ks[j]], 1);
      if (4 * q + j < c0) atomicAdd(&pre[ks[j]], 1);
    }
  }
  for (int i = 4 * nq + t; i < np; i += kSortChunk) {
    const uint32_t k = eids[i] & 0xFFu;
    atomicAdd(&tot[k], 1);
    if (i < c0) atomicAdd(&pre[k], 1);
  }
  // ---- this chunk's pairs: wave w's step, the lanes of each key and their ranks
  const int idx = c0 + t;
  const bool valid = idx < np;
  const uint32_t key = valid ? (eids[idx] & 0xFFu) : 0u;   // ids are < 256 by contract
  uint64_t same = same_key_mask(key) & __ballot(valid);      // every lane takes part in the ballots
  const uint64_t below = (1ull << lane) - 1ull;
  const int rank = __builtin_popcountll(same & below);
  if (valid && rank == 0) cw[wave][key] = __builtin_popcountll(same);
  __syncthreads();
  // ---- expert e = t: exclusive scans over the experts of the pair counts and of the item counts
  const int tok = moe_item_tok(np);
  const int c = tot[t], ni = (c + tok - 1) / tok;
  int sc = c, si = ni;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int pc = __shfl_up(sc, o, 64), pi = __shfl_up(si, o, 64);
    if (lane >= o) { sc += pc; si += pi; }
  }
  if (lane == 63) { wsum[wave][0] = sc; wsum[wave][1] = si; }
  __syncthreads();
  int bc = sc - c, bi = si - ni;
  for (int w = 0; w < wave; ++w) { bc += wsum[w][0]; bi += wsum[w][1]; }
  if (blockIdx.x == 0) {
    eoff[t] = bc;
    for (int j = 0; j < ni; ++j) items[bi + j] = ((uint32_t)t << 16) | (uint32_t)(tok * j);
    if (t == kE - 1) {
      eoff[kE] = bc + c;
      *nitp = (uint32_t)(bi + ni);
    }
  }
  // bin e's slots for this chunk's waves: after the bin start, the earlier chunks and waves
  int run = bc + pre[t];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int n = cw[w][t];
    cw[w][t] = run;
    run += n;
  }
  __syncthreads();
  if (valid) plist[cw[wave][key] + rank] = (uint16_t)idx;
}

// ------------------------------------------------------------------ grouped IQ4_XS GEMM
enum MoeKind { MOE_UP = 0, MOE_DN = 1, MOE_DN_DENSE = 2, MOE_UP_DENSE = 3 };

// K: reduction length
template <int KIND> struct MoeShape;
template <> struct MoeShape<MOE_UP> { static constexpr int K = kHid; };
template <> struct MoeShape<MOE_UP_DENSE> { static constexpr int K = kHid; };
template <> struct MoeShape<MOE_DN> { static constexpr int K = kFf; };
template <> struct MoeShape<MOE_DN_DENSE> { static constexpr int K = kFf; };

__device__ __forceinline__ h8_t splat8h(_Float16 v) { return h8_t{v, v, v, v, v, v, v, v}; }

using gbyte = const __attribute__((address_space(1))) uint8_t;

// ------------------------------------------------------------------ grouped IQ4_XS GEMM (prefill)
// Work unit: one item (up to 96 of an expert's sorted pairs: at uniform routing all of them, so
// the expert's weights are streamed once) x one stripe of weight rows (FFN: 256 gate rows + the
// matching 256 up rows; down: 512 rows).  8 waves, two per SIMD; wave w owns four 16-row tiles
// (FFN: gate tiles 2w, 2w + 1 of the stripe and the two matching up tiles; down: tiles 4w..4w+3)
// over the whole K, so no reduction across waves.  K runs in stages of 128 (half an IQ4_XS
// block): in stage h = 2 kb + sb, lane (col, kq) of a wave holds row col's sub-block 4 sb + kq of
// block kb, i.e. 16 quant bytes and the block header.
//   * weights go straight from memory to registers, RING - 1 stages ahead (buffer loads: the
//     stage offset is a scalar, the lane's row offset a fixed register), and are decoded there:
//     each quant byte is looked up in a byte -> (kv[lo], kv[hi]) fp16 table kept once per lane
//     (64 copies, copy l in bank l), so the wave's 64 lookups never collide in a bank;
//   * activations: per stage the item's token rows are loaded (a stage ahead, rows through the
//     sorted pair list), converted to fp16 once, and stored in LDS already in the MFMA k order
//     (the 8 halves of piece p = 4 kq + c are x[k0 + 32 kq + 4c + {0, 16, 1, 17, 2, 18, 3, 19}],
//     the order the byte table pairs the weights in) with piece p of token row t at slot
//     p ^ (t & 15): the 16 lanes of a fragment read hit 16 distinct 16-B slots;
//   * per stage: issue the next stage's activation loads and the weight loads RING - 1 stages
//     ahead, 4 x (NG groups x 4 tiles) MFMAs on this stage, then store the next stage's
//     activations and one barrier;
//   * blockIdx -> (item, stripe) keeps the stripes of an item on one XCD (workgroups are
//     dispatched round-robin over the 8 XCDs), so its activations are read from that L2.
constexpr int kPfTiles = 4;   // 16-row tiles per wave
constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * TLX_WAVE;

struct __attribute__((aligned(16))) MoePfLds {
  uint32_t lut[256 * TLX_WAVE];   // [quant byte][lane]: (kv[lo], kv[hi]) fp16
  u4_t a[2][kPfTok * 16];         // 128-k stages of the item's activations, fp16, [row][swizzled piece]
  int xrow[kPfTok];               // activation row of token slot t
  int orow[kPfTok];               // output row of token slot t
};

template <int KIND>
constexpr int moe_pf_stripes() {
  return (KIND == MOE_UP || KIND == MOE_UP_DENSE) ? kFf / (16 * 2 * kPfWaves) : kHid / (16 * kPfTiles * kPfWaves);
}

// buffer resource over n bytes at p (raw dword-granular buffer; no format conversion)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t moe_rsrc(const void* p, uint32_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000);
}

// weight registers of one stage: per tile the lane's 16 quant bytes and its row's block header
struct MoeWs {
  u4_t q[kPfTiles];
  u2_t h[kPfTiles];
};

template <int KIND, int NG, bool TL>
__device__ __forceinline__ void moe_pf_tile(MoePfLds& L, const void* base, const float* __restrict__ xs,
                                            const float* __restrict__ iq4nl, void* __restrict__ out, int ntok,
                                            int stripe, int wave, int lane) {
  using S = MoeShape<KIND>;
  constexpr bool kUp = KIND == MOE_UP || KIND == MOE_UP_DENSE;
  constexpr int kNb = S::K / 256;
  constexpr int kH = 2 * kNb;                       // 128-k stages
  constexpr int kRowBytes = kNb * 136;
  constexpr uint32_t kSlab = kUp ? 2u * kGateBytes : (uint32_t)kHid * kRowBytes;
  // weight ring depth (stages RING - 1 ahead) as the accumulators leave room: deeper rings at
  // more groups spill
  constexpr int RING = NG <= 2 ? 4 : 2;
  constexpr int NI = (NG + 1) / 2;                  // activation pieces (x 2 float4) per thread
  const int col = lane & 15, kq = lane >> 4, t = threadIdx.x;
  // the wave's tiles: FFN gate tiles 2 * (kPfWaves * stripe + wave) + {0, 1}, then the same up
  // tiles; down tiles 4 * (kPfWaves * stripe + wave) + {0..3}
  const int tb = kPfWaves * stripe + wave;
  const __amdgpu_buffer_rsrc_t rw = moe_rsrc(base, kSlab);
  // tile j's first byte in the slab (wave-uniform): GGUF rows and tiled records alike
  int ts[kPfTiles];
#pragma unroll
  for (int j = 0; j < kPfTiles; ++j) {
    if constexpr (kUp)
      ts[j] = (j >= 2 ? kGateBytes : 0) + 16 * (2 * tb + (j & 1)) * kRowBytes;
    else
      ts[j] = 16 * (4 * tb + j) * kRowBytes;
  }
  // stage h's weights (block kb = h / 2, sub-block 4 (h & 1) + kq of row col): GGUF rows -- the
  // header at row col's 136 kb, the quant bytes at + 8 + 64 (h & 1) + 16 kq; tiled -- the
  // header at record (tile, kb) + 8 col, the quant bytes at + 128 + 1024 (h & 1) + 16 lane
  const int vh = TL ? 8 * col : col * kRowBytes;
  const int vq = TL ? 128 + 16 * lane : col * kRowBytes + 8 + 16 * kq;
  auto load_w = [&](MoeWs& w, int h) {
    const int so = TL ? 2176 * (h >> 1) : 136 * (h >> 1);
    const int sq = so + (TL ? 1024 : 64) * (h & 1);
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) {
      w.h[j] = __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(rw, vh, ts[j] + so, 0));
      w.q[j] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, vq, ts[j] + sq, 0));
    }
  };
  // activations: thread t, piece i covers row min(32 i + (t >> 4), 16 NG - 1), piece p = t & 15
  // (a row past the item's groups repeats the last one: stored twice with the same bytes)
  const __amdgpu_buffer_rsrc_t rx = moe_rsrc(xs, 0x7FFFFFFFu);
  const int p = t & 15;
  int xo[NI], ao[NI];   // the piece's source byte offset at k0 = 0, and its LDS slot
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = min(32 * i + (t >> 4), 16 * NG - 1);
    xo[i] = 4 * (32 * (p >> 2) + 4 * (p & 3));   // + the row's offset once xrow is visible
    ao[i] = row * 16 + (p ^ (row & 15));
  }
  // activations two stages ahead, in two register sets: stage h's are stored into LDS at the end
  // of stage h - 1
  float4 xa[2][NI][2];
  auto load_a = [&](int set, int h) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      xa[set][i][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i], 512 * h, 0));
      xa[set][i][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i] + 64, 512 * h, 0));
    }
  };
  auto store_a = [&](int set, u4_t* buf) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float4 v0 = xa[set][i][0], v1 = xa[set][i][1];
      const h8_t hv = {(_Float16)v0.x, (_Float16)v1.x, (_Float16)v0.y, (_Float16)v1.y,
                       (_Float16)v0.z, (_Float16)v1.z, (_Float16)v0.w, (_Float16)v1.w};
      buf[ao[i]] = __builtin_bit_cast(u4_t, hv);
    }
  };

  f4_t acc[NG][kPfTiles];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) acc[g][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // entry (quant byte i of qw) of this lane's copy: byte offset 256 * byte + 4 * lane, assembled by
  // one byte permute (result bytes: [4 * lane, byte i, 0, 0])
  const uint8_t* lut0 = reinterpret_cast<const uint8_t*>(L.lut);
  const uint32_t lane4 = 4u * (uint32_t)lane;
  auto lut = [&](uint32_t qw, int i) {
    const uint32_t off = __builtin_amdgcn_perm(qw, lane4, 0x0C0C0000u | ((4u + (uint32_t)i) << 8));
    return *reinterpret_cast<const uint32_t*>(lut0 + off);
  };

  MoeWs W[RING];
  // Stage h: weights from W[h % RING], activations from LDS buffer h & 1.  Loads are unconditional
  // and clamped at the end (a load under a branch makes the wait counts assume the worst; the
  // repeats past the end reload the last stage).  The memory counter completes in issue order, so
  // the order of the stage's two requests keeps either wait from draining the other's prefetch:
  // with RING > 2 the activations go first (the wait for stage h + 1's activations at the end of
  // stage h then covers only weights up to stage h + 1), with RING == 2 the weights (the wait for
  // stage h + 1's weights then covers only activations up to stage h + 1).
  auto stage = [&](int h, MoeWs& w, MoeWs& wnext) {
    // (with the deep ring the requests are fenced at the stage's start: the scheduler would
    // otherwise sink them to its end, and a small-NG stage is too short to cover their latency;
    // measured: P = 512, 1-2 groups, 150 -> 81 us.  At 3+ groups the fences cost 7%.)
    if constexpr (RING > 2) __builtin_amdgcn_sched_barrier(0);
    if constexpr (RING > 2) load_a(h & 1, min(h + 2, kH - 1));
    load_w(wnext, min(h + RING - 1, kH - 1));
    if constexpr (RING == 2) load_a(h & 1, min(h + 2, kH - 1));
    if constexpr (RING > 2) __builtin_amdgcn_sched_barrier(0);
    const u4_t* arow = L.a[h & 1] + 16 * col;   // + 256 * g: token row 16g + col (slot p ^ col)
    const int ib = 4 * (h & 1) + kq;             // the lane's sub-block of block h / 2
    _Float16 dh[kPfTiles];
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) {
      const uint32_t sh = w.h[j].x >> 16;
      const uint32_t ls = ((w.h[j].y >> (4 * ib)) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4);
      dh[j] = (_Float16)(tlx_h2f((uint16_t)w.h[j].x) * (float)((int)ls - 32));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      h8_t B[kPfTiles];
#pragma unroll
      for (int j = 0; j < kPfTiles; ++j) {
        const uint32_t qw = w.q[j][c];
        const u4_t w4 = {lut(qw, 0), lut(qw, 1), lut(qw, 2), lut(qw, 3)};
        B[j] = __builtin_bit_cast(h8_t, w4) * splat8h(dh[j]);
      }
      const int pc = 4 * kq + c;   // 16-B piece: k0 = 128 h + 32 kq + 4c (and + 16)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const h8_t A = __builtin_bit_cast(h8_t, arow[256 * g + (pc ^ col)]);
        // weights as the MFMA's first operand: the output lane (col, kq) then holds weight rows
        // 4 kq .. 4 kq + 3 of the tile for token col (4 consecutive outputs, one wide store)
#pragma unroll
        for (int j = 0; j < kPfTiles; ++j)
          acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(B[j], A, acc[g][j], 0, 0, 0);
      }
    }
    // (waits for its loads; stage h - 1's buffer is free: every wave passed the last barrier)
    store_a((h + 1) & 1, L.a[(h + 1) & 1]);
    __syncthreads();
  };

  // the first stages' weights first: the byte table is built while they are in flight
#pragma unroll
  for (int r = 0; r < RING - 1; ++r) load_w(W[r], min(r, kH - 1));
  {   // the byte table, one copy per lane: entry b of copy l at [b][l]; wave w writes the entries
      // b = w + 8i, whose two table values are wave-uniform (scalar loads)
#pragma unroll
    for (int i = 0; i < 256 / kPfWaves; ++i) {
      const int b = wave + kPfWaves * i;
      const _Float16 lo = (_Float16)iq4nl[b & 15], hi = (_Float16)iq4nl[b >> 4];
      L.lut[b * TLX_WAVE + lane] =
          (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
  }
  __syncthreads();   // xrow / orow (written by the kernel before the tile) are visible
#pragma unroll
  for (int i = 0; i < NI; ++i) xo[i] += L.xrow[min(32 * i + (t >> 4), 16 * NG - 1)] * (S::K * 4);
  load_a(0, 0);
  load_a(1, 1);
  store_a(0, L.a[0]);
  __syncthreads();   // stage 0's activations and the byte table are visible
  // stages in rounds of U (a multiple of the ring depth and of the two activation sets), then the
  // rest; stage h uses ring entry h % RING, a compile-time index in both loops
  constexpr int U = RING % 2 ? 2 * RING : RING;
  int h0 = 0;
  for (; h0 + U <= kH; h0 += U) {
#pragma unroll
    for (int r = 0; r < U; ++r) stage(h0 + r, W[r % RING], W[(r + RING - 1) % RING]);
  }
#pragma unroll
  for (int r = 0; r < kH % U; ++r) stage(h0 + r, W[r % RING], W[(r + RING - 1) % RING]);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // the clamped tail loads

  // lane (col, kq) holds rows 16 tile + 4 kq + r of token 16 g + col
  static_assert(kUp, "the down projection runs moe_pd_kernel");
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int slot = 16 * g + col;
    if (slot >= ntok) continue;
    const int o = L.orow[slot];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f4_t v;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gv = acc[g][j][r], uv = acc[g][j + 2][r];
        v[r] = gv / (1.f + expf(-gv)) * uv;
      }
      const int n = 16 * (2 * tb + j) + 4 * kq;
      *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(out) + (size_t)o * kFf + n) = v;
    }
  }
}

// workgroup id (of this kind's part of the grid, a multiple of 8 from the grid's start)
template <int KIND, bool TL>
__device__ __forceinline__ void moe_pf_body(MoePfLds& L, const uint64_t* __restrict__ ptbl,
                                            const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
                                            const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp,
                                            const float* __restrict__ xs, const float* __restrict__ iq4nl,
                                            void* __restrict__ out, int P, int id) {
  constexpr bool kDense = KIND == MOE_DN_DENSE || KIND == MOE_UP_DENSE;
  constexpr bool kUp = KIND == MOE_UP || KIND == MOE_UP_DENSE;
  constexpr int kS = moe_pf_stripes<KIND>();
  const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  // XCD x = id % 8 runs the kS stripes of items x, x + 8, ... one item after another
  const int l = id >> 3;
  const int stripe = l % kS, item = (l / kS) * 8 + (id & 7);

  int m0, ntok;
  const void* base;
  if constexpr (kDense) {   // the shared expert: chunks of kDenseTok positions
    m0 = item * kDenseTok;
    if (m0 >= P) return;
    ntok = min(kDenseTok, P - m0);
    base = (const void*)(ptbl[0]);
  } else {
    if (item >= (int)*nitp) return;
    const uint32_t it = items[item];
    const int e = (int)(it >> 16);
    m0 = (int)(it & 0xFFFFu);
    const int eb0 = eoff[e];
    ntok = min(kPfTok, eoff[e + 1] - eb0 - m0);
    m0 += eb0;
    base = (const void*)(ptbl[e]);
  }
  if (t < kPfTok) {
    const int slot = min(t, ntok - 1);   // padded slots repeat the last pair; never stored
    if constexpr (kDense) {
      L.xrow[t] = m0 + slot;
      L.orow[t] = m0 + slot;
    } else {
      const int pair = plist[m0 + slot];
      L.xrow[t] = kUp ? (pair >> 3) : pair;
      L.orow[t] = pair;
    }
  }
  // workgroup-uniform (the tile's first barrier publishes xrow / orow); dense chunks have <= 32
  switch ((ntok + 15) >> 4) {
    case 1: moe_pf_tile<KIND, 1, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
    case 2: moe_pf_tile<KIND, 2, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
    case 3: if constexpr (!kDense) moe_pf_tile<KIND, 3, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
    case 4: if constexpr (!kDense) moe_pf_tile<KIND, 4, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
    case 5: if constexpr (!kDense) moe_pf_tile<KIND, 5, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
    default: if constexpr (!kDense) moe_pf_tile<KIND, 6, TL>(L, base, xs, iq4nl, out, ntok, stripe, wave, lane); break;
  }
}

template <int KIND, bool TL>
__global__ __launch_bounds__(kPfThreads, 1) void moe_pf_kernel(
    const uint64_t* __restrict__ ptbl, const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
    const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp, const float* __restrict__ xs,
    const float* __restrict__ iq4nl, void* __restrict__ out, int P) {
  __shared__ MoePfLds L;
  moe_pf_body<KIND, TL>(L, ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P, (int)blockIdx.x);
}

// The grouped gate+up and the shared expert's gate+up in one launch: workgroups below nrb run the
// routed items, the rest the shared expert's dense chunks (after the routed ones: they fill the
// last, partial round of routed workgroups).  Each part is its own launch's code, so the outputs
// are the separate launches' bit for bit.
template <bool TL>
__global__ __launch_bounds__(kPfThreads, 1) void moe_pf_sh_kernel(
    const uint64_t* __restrict__ ptbl, const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
    const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp, const float* __restrict__ xs,
    const float* __restrict__ iq4nl, void* __restrict__ out, const uint64_t* __restrict__ ptbl_sh,
    float* __restrict__ sact, int P, int nrb) {
  __shared__ MoePfLds L;
  const int id = (int)blockIdx.x;
  if (id < nrb)
    moe_pf_body<MOE_UP, TL>(L, ptbl, eoff, plist, items, nitp, xs, iq4nl, out, 0, id);
  else
    moe_pf_body<MOE_UP_DENSE, TL>(L, ptbl_sh, nullptr, nullptr, nullptr, nullptr, xs, iq4nl, sact, P, id - nrb);
}

// ------------------------------------------------------------------ grouped IQ4_XS down GEMM (prefill)
// The down projection's K (512) is short enough for an item's activations to stay in LDS: a
// workgroup stages its item's act rows once (fp16, MFMA k order, 96 KB at 96 tokens) and then
// streams all 2048 weight rows as 4 stripes of 512 -- wave w owns tiles 4 (8 s + w) .. + 3 of
// stripe s -- with no barrier after the staging: the 16 (stripe, stage) steps of a wave are one
// weight stream, loaded 3 steps ahead.  Stage h (128 k) of block h / 2: lane (col, kq) holds row
// col's sub-block 4 (h & 1) + kq, decoded as in the gate/up kernel.  One workgroup per item, so
// an expert's down weights are read once and its activations once.
constexpr int kPdPieces = kFf / 8;   // 16-B pieces per staged row (64)

struct __attribute__((aligned(16))) MoePdLds {
  uint32_t lut[256 * TLX_WAVE];   // [quant byte][lane]: (kv[lo], kv[hi]) fp16
  u4_t a[kPfTok * kPdPieces];     // the item's activations, fp16, [row][swizzled piece]
};

template <int KIND, int NG, bool TL>
__device__ __forceinline__ void moe_pd_tile(MoePdLds& L, const void* base, const float* __restrict__ xs,
                                            const float* __restrict__ iq4nl, void* __restrict__ out,
                                            const uint16_t* __restrict__ plist, int m0, int ntok, int wave,
                                            int lane, int dstripe) {
  constexpr bool kDense = KIND == MOE_DN_DENSE;
  constexpr int kNb = kFf / 256;                     // blocks per row (2)
  constexpr int kRowBytes = kNb * 136;
  constexpr int RING = NG <= 4 ? 4 : 2;               // weight steps in the ring (RING - 1 ahead)
  const int col = lane & 15, kq = lane >> 4, t = threadIdx.x;
  // slot s's pair (row of act / parts): the sorted pair list, or the dense chunk's position
  auto pair_of = [&](int slot) { return kDense ? m0 + slot : (int)plist[m0 + slot]; };

  const __amdgpu_buffer_rsrc_t rw = moe_rsrc(base, (uint32_t)kHid * kRowBytes);
  const int vh = TL ? 8 * col : col * kRowBytes;
  const int vq = TL ? 128 + 16 * lane : col * kRowBytes + 8 + 16 * kq;
  // step i = 4 s + h: stripe s, stage h; tile j of the wave: 4 (8 s + wave) + j
  auto load_w = [&](MoeWs& w, int i) {
    const int s = i >> 2, h = i & 3;
    const int t0 = 16 * 4 * (kPfWaves * s + wave) * kRowBytes;   // first tile's first byte
    const int so = t0 + (TL ? 2176 * (h >> 1) : 136 * (h >> 1));
    const int sq = so + (TL ? 1024 : 64) * (h & 1);
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) {
      w.h[j] = __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(rw, vh, so + 16 * j * kRowBytes, 0));
      w.q[j] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, vq, sq + 16 * j * kRowBytes, 0));
    }
  };

  // the stripes of this workgroup: all 4 (routed items), or dstripe (dense chunks)
  const int s0 = kDense ? dstripe : 0, s1 = kDense ? s0 + 1 : 4;
  MoeWs W[RING];
#pragma unroll
  for (int r = 0; r < RING - 1; ++r) load_w(W[r], 4 * s0 + r);   // first: in flight during the staging and the table
  // ---- stage the item's activations: piece p of row r (x[r][8 (p & ~3) + ...]: sub-block p / 4,
  // chunk p % 4, the halves k0 + {0, 16, 1, 17, 2, 18, 3, 19}) at slot p ^ (r & 15) of row r.
  // All of a thread's pieces are requested at once; the byte table is built while they (and the
  // first weights) are in flight.
  {
    const __amdgpu_buffer_rsrc_t rx = moe_rsrc(xs, 0x7FFFFFFFu);
    constexpr int kPer = 16 * NG * kPdPieces / kPfThreads;   // pieces per thread (2 NG)
    float4 v[kPer][2];
    int dst[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int q = j * kPfThreads + t;   // piece index q = row * 64 + p
      const int row = q >> 6, p = q & 63;
      const int src = pair_of(min(row, ntok - 1)) * (kFf * 4) + 4 * (32 * (p >> 2) + 4 * (p & 3));
      v[j][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, src, 0, 0));
      v[j][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, src + 64, 0, 0));
      dst[j] = row * kPdPieces + (p ^ (row & 15));
    }
    // the byte table, one copy per lane (as the gate/up kernel)
#pragma unroll
    for (int i = 0; i < 256 / kPfWaves; ++i) {
      const int b = wave + kPfWaves * i;
      const _Float16 lo = (_Float16)iq4nl[b & 15], hi = (_Float16)iq4nl[b >> 4];
      L.lut[b * TLX_WAVE + lane] =
          (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const h8_t hv = {(_Float16)v[j][0].x, (_Float16)v[j][1].x, (_Float16)v[j][0].y, (_Float16)v[j][1].y,
                       (_Float16)v[j][0].z, (_Float16)v[j][1].z, (_Float16)v[j][0].w, (_Float16)v[j][1].w};
      L.a[dst[j]] = __builtin_bit_cast(u4_t, hv);
    }
  }
  __syncthreads();   // activations and table visible; no barrier after this

  const uint8_t* lut0 = reinterpret_cast<const uint8_t*>(L.lut);
  const uint32_t lane4 = 4u * (uint32_t)lane;
  auto lut = [&](uint32_t qw, int i) {
    const uint32_t off = __builtin_amdgcn_perm(qw, lane4, 0x0C0C0000u | ((4u + (uint32_t)i) << 8));
    return *reinterpret_cast<const uint32_t*>(lut0 + off);
  };
  const u4_t* arow = L.a + kPdPieces * col;   // + 1024 g: token row 16 g + col

  f4_t acc[NG][kPfTiles];
  static_assert(4 % RING == 0, "stage h of a stripe uses ring entry h % RING");
#pragma nounroll
  for (int s = s0; s < s1; ++s) {
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) acc[g][j] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int i = 4 * s + h;
    // (scheduling fences: one per stage -- with no barrier in the loop the scheduler would
    // otherwise interleave the stages' table lookups and decodes and run out of registers -- and
    // one after the stage's weight requests, which it would otherwise sink to the stage's end,
    // where the next stage waits for them at once)
    __builtin_amdgcn_sched_barrier(0);
    load_w(W[(h + RING - 1) % RING], min(i + RING - 1, 4 * s1 - 1));   // clamped: repeats the last step
    __builtin_amdgcn_sched_barrier(0);
    const MoeWs& w = W[h % RING];
    const int ib = 4 * (h & 1) + kq;
    _Float16 dh[kPfTiles];
#pragma unroll
    for (int j = 0; j < kPfTiles; ++j) {
      const uint32_t sh = w.h[j].x >> 16;
      const uint32_t ls = ((w.h[j].y >> (4 * ib)) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4);
      dh[j] = (_Float16)(tlx_h2f((uint16_t)w.h[j].x) * (float)((int)ls - 32));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      h8_t B[kPfTiles];
#pragma unroll
      for (int j = 0; j < kPfTiles; ++j) {
        const uint32_t qw = w.q[j][c];
        const u4_t w4 = {lut(qw, 0), lut(qw, 1), lut(qw, 2), lut(qw, 3)};
        B[j] = __builtin_bit_cast(h8_t, w4) * splat8h(dh[j]);
      }
      const int pc = 16 * h + 4 * kq + c;   // piece of k = 128 h + 32 kq + 4 c
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const h8_t A = __builtin_bit_cast(h8_t, arow[1024 * g + (pc ^ col)]);
        // weights as the MFMA's first operand: the output lane (col, kq) then holds weight rows
        // 4 kq .. 4 kq + 3 of the tile for token col (4 consecutive outputs, one wide store)
#pragma unroll
        for (int j = 0; j < kPfTiles; ++j)
          acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(B[j], A, acc[g][j], 0, 0, 0);
      }
    }
    if (h == 3) {   // stripe s done: lane (col, kq) holds rows 16 tile + 4 kq + r of token 16 g + col
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int slot = 16 * g + col;
        if (slot >= ntok) continue;
        const int o = pair_of(slot);
#pragma unroll
        for (int j = 0; j < kPfTiles; ++j) {
          const int n = 16 * (4 * (kPfWaves * s + wave) + j) + 4 * kq;
          const f4_t v = acc[g][j];
          if constexpr (KIND == MOE_DN) {
            const h4_t hv = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            *reinterpret_cast<h4_t*>(reinterpret_cast<uint16_t*>(out) + (size_t)o * kHid + n) = hv;
          } else {
            *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(out) + (size_t)o * kHid + n) = v;
          }
        }
      }
    }
  }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);   // the clamped tail loads
}

// one workgroup per item (routed: all 4 stripes) or per (kDenseTok-position chunk, stripe) (dense)
template <int KIND, bool TL>
__device__ __forceinline__ void moe_pd_body(MoePdLds& L, const uint64_t* __restrict__ ptbl,
                                            const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
                                            const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp,
                                            const float* __restrict__ xs, const float* __restrict__ iq4nl,
                                            void* __restrict__ out, int P, int tok, int item, int dstripe) {
  constexpr bool kDense = KIND == MOE_DN_DENSE;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  int m0, ntok;
  const void* base;
  if constexpr (kDense) {
    m0 = item * kDenseTok;
    if (m0 >= P) return;
    ntok = min(kDenseTok, P - m0);
    base = (const void*)(ptbl[0]);
  } else {
    if (item >= (int)*nitp) return;
    const uint32_t it = items[item];
    const int e = (int)(it >> 16);
    m0 = (int)(it & 0xFFFFu);
    const int eb0 = eoff[e];
    ntok = min(tok, eoff[e + 1] - eb0 - m0);   // tok: the sort's item size (64 or 96 pairs)
    m0 += eb0;
    base = (const void*)(ptbl[e]);
  }
  switch ((ntok + 15) >> 4) {   // workgroup-uniform; dense chunks have <= 32 positions
    case 1: moe_pd_tile<KIND, 1, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, dstripe); break;
    case 2: moe_pd_tile<KIND, 2, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, dstripe); break;
    case 3: if constexpr (!kDense) moe_pd_tile<KIND, 3, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, 0); break;
    case 4: if constexpr (!kDense) moe_pd_tile<KIND, 4, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, 0); break;
    case 5: if constexpr (!kDense) moe_pd_tile<KIND, 5, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, 0); break;
    default: if constexpr (!kDense) moe_pd_tile<KIND, 6, TL>(L, base, xs, iq4nl, out, plist, m0, ntok, wave, lane, 0); break;
  }
}

template <int KIND, bool TL>
__global__ __launch_bounds__(kPfThreads, 1) void moe_pd_kernel(
    const uint64_t* __restrict__ ptbl, const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
    const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp, const float* __restrict__ xs,
    const float* __restrict__ iq4nl, void* __restrict__ out, int P, int tok) {
  __shared__ MoePdLds L;
  moe_pd_body<KIND, TL>(L, ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P, tok, (int)blockIdx.x, (int)blockIdx.y);
}

// The grouped down and the shared expert's down in one launch: workgroups below nitems run the
// routed items, the rest the shared expert's (chunk, stripe) pairs, stripe fastest -- each part
// its own launch's code, so the outputs are the separate launches' bit for bit.
template <bool TL>
__global__ __launch_bounds__(kPfThreads, 1) void moe_pd_sh_kernel(
    const uint64_t* __restrict__ ptbl, const int* __restrict__ eoff, const uint16_t* __restrict__ plist,
    const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp, const float* __restrict__ act,
    const float* __restrict__ iq4nl, void* __restrict__ out, int tok, const uint64_t* __restrict__ ptbl_sh,
    const float* __restrict__ sact, float* __restrict__ shared, int P, int nitems) {
  __shared__ MoePdLds L;
  const int id = (int)blockIdx.x;
  if (id < nitems) {
    moe_pd_body<MOE_DN, TL>(L, ptbl, eoff, plist, items, nitp, act, iq4nl, out, 0, tok, id, 0);
  } else {
    const int d = id - nitems;
    moe_pd_body<MOE_DN_DENSE, TL>(L, ptbl_sh, nullptr, nullptr, nullptr, nullptr, sact, iq4nl, shared, P, 0, d >> 2,
                                  d & 3);
  }
}

// ------------------------------------------------------------------ grouped IQ4_XS GEMV
// The small-batch (decode / verify) form of the same products.  With a few tokens per expert
// there is too little work per weight to stage anything; here a workgroup owns one 16-row output
// tile (FFN: 16 gate + the matching 16 up rows; down: two tiles) of one work item, its waves
// split the tile's K blocks, every wave issues all of its loads at once, and the waves reduce
// through LDS in a fixed order.
//   * lane (col, kq) of a wave holds weight row col's sub-blocks kq and kq + 4 of each of its
//     blocks (the 4 lanes of a row read 64 contiguous bytes per load) and the block header; a
//     sub-block's 4-byte chunk c gives the 8
//     weights j = 4c..4c+3 (low nibbles) and 16 + 4c.. (high nibbles), decoded by 4 lookups of
//     the byte -> (kv[lo], kv[hi]) fp16 table and scaled by fp16(d * (ls - 32)) -- the same
//     operand values as the GEMM -- then one v_mfma_f32_16x16x32_f16 per chunk and 16-token group;
//   * the A operand is the matching activations, interleaved the same way, in groups of 16 of the
//     item's tokens (rows past the item repeat its last token and are never stored).
constexpr int kGvGroups = kTok / 16;

// waves per 16-row tile: the FFN tile (2 x 8 blocks per row) is split over 2 waves, a down tile
// (2 blocks per row) is one wave's
template <int KIND>
constexpr int moe_gv_wpt() { return (KIND == MOE_UP || KIND == MOE_UP_DENSE) ? 2 : 1; }

// One wave's share of a 16-row output tile for NG groups of 16 tokens.  NG is a template
// argument so that every activation load is unconditional: the compiler can then issue them
// ahead of their MFMAs instead of waiting on each one in turn.  red: the workgroup's
// [4 waves][kGvGroups][NMAT][64 lanes] reduction buffer.
template <int KIND, int NG, bool TL, bool XS>
__device__ __forceinline__ void moe_gv_tile(gbyte* base, const uint32_t* lut, const int* xrow, const int* orow,
                                            f4_t* red, const u4_t* xst, const float* __restrict__ xs,
                                            void* __restrict__ out, int ntok, int tile, int wave, int lane) {
  using S = MoeShape<KIND>;
  constexpr bool kUp = KIND == MOE_UP || KIND == MOE_UP_DENSE;
  constexpr int NMAT = kUp ? 2 : 1;
  constexpr int kNb = S::K / 256;                 // IQ4_XS blocks per row
  constexpr int kWpt = moe_gv_wpt<KIND>();        // waves per tile
  constexpr int kBpw = kNb / kWpt;                // blocks per wave
  constexpr int kRowBytes = kNb * 136;
  const int col = lane & 15, kq = lane >> 4;
  const int kb0 = (wave % kWpt) * kBpw;
  gbyte* wrow[NMAT];
  wrow[0] = base + (size_t)(16 * tile + col) * kRowBytes;
  if constexpr (NMAT == 2) wrow[1] = wrow[0] + kGateBytes;

  // all of the wave's weight loads first
  u2_t hdr[kBpw][NMAT];
  u4_t qv[kBpw][NMAT][2];
#pragma unroll
  for (int bb = 0; bb < kBpw; ++bb)
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
      if constexpr (TL) {   // record (tile, block): header at 8 col, quant bytes in lane order
        gbyte* rec = wrow[mi] - (size_t)col * kRowBytes + 2176 * (kb0 + bb);
        hdr[bb][mi] = *(const __attribute__((address_space(1))) u2_t*)(rec + 8 * col);
        qv[bb][mi][0] = *(const __attribute__((address_space(1))) u4_t*)(rec + 128 + 16 * lane);
        qv[bb][mi][1] = *(const __attribute__((address_space(1))) u4_t*)(rec + 1152 + 16 * lane);
      } else {
        gbyte* blk = wrow[mi] + 136 * (kb0 + bb);
        hdr[bb][mi] = *(const __attribute__((address_space(1))) u2_t*)(blk);
        qv[bb][mi][0] = *(const __attribute__((address_space(1))) u4_t*)(blk + 8 + 16 * kq);
        qv[bb][mi][1] = *(const __attribute__((address_space(1))) u4_t*)(blk + 72 + 16 * kq);
      }
    }
  const float* xr[NG];   // lane's activation row in group g, at its first k of a block
#pragma unroll
  for (int g = 0; g < NG; ++g) xr[g] = xs + (size_t)xrow[16 * g + col] * S::K + 256 * kb0 + 32 * kq;
  // staged (NG == 1): the lane's token row min(col, ntok - 1) of the staged copy
  const int xsrow = min(col, ntok - 1) * (S::K / 8 + 1);

  f4_t acc[NG][NMAT];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) acc[g][mi] = f4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int bb = 0; bb < kBpw; ++bb) {
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ib = kq + 4 * sb;   // the lane's sub-blocks kq, kq + 4
      _Float16 dh[NMAT];
#pragma unroll
      for (int mi = 0; mi < NMAT; ++mi) {
        const uint32_t sh = hdr[bb][mi].x >> 16;
        const uint32_t ls = ((hdr[bb][mi].y >> (4 * ib)) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4);
        dh[mi] = (_Float16)(tlx_h2f((uint16_t)hdr[bb][mi].x) * (float)((int)ls - 32));
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        h8_t B[NMAT];
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) {
          const uint32_t qw = qv[bb][mi][sb][c];
          const u4_t w4 = {lut[qw & 0xFF], lut[(qw >> 8) & 0xFF], lut[(qw >> 16) & 0xFF], lut[qw >> 24]};
          B[mi] = __builtin_bit_cast(h8_t, w4) * splat8h(dh[mi]);
        }
        const int k0 = 256 * bb + 128 * sb + 4 * c;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          h8_t A;
          if constexpr (XS) {   // staged: piece 32 (kb0 + bb) + 4 ib + c of the lane's token row
            A = __builtin_bit_cast(h8_t, xst[xsrow + 32 * (kb0 + bb) + 4 * ib + c]);
          } else {
            const float4 x0 = *reinterpret_cast<const float4*>(xr[g] + k0);
            const float4 x1 = *reinterpret_cast<const float4*>(xr[g] + k0 + 16);
            A = h8_t{(_Float16)x0.x, (_Float16)x1.x, (_Float16)x0.y, (_Float16)x1.y,
                     (_Float16)x0.z, (_Float16)x1.z, (_Float16)x0.w, (_Float16)x1.w};
          }
#pragma unroll
          for (int mi = 0; mi < NMAT; ++mi)
            acc[g][mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[mi], acc[g][mi], 0, 0, 0);
        }
      }
    }
  }

  // fixed-order reduction over the waves of a tile
  // slot of writer wave w (w % kWpt != 0): w / kWpt -- one per tile shared by two waves
  auto rslot = [&](int w, int g, int mi) -> f4_t& {
    return red[(((w / kWpt) * kGvGroups + g) * NMAT + mi) * 64 + lane];
  };
  if constexpr (kWpt > 1) {
    if (wave % kWpt != 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) rslot(wave, g, mi) = acc[g][mi];
    }
    __syncthreads();
    if (wave % kWpt != 0) return;
    for (int w = wave + 1; w < wave + kWpt; ++w)
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) acc[g][mi] += rslot(w, g, mi);
  }

  // lane (col, kq) holds tokens 16g + 4kq + r of row 16 * tile + col
  const int n = 16 * tile + col;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int slot = 16 * g + 4 * kq + r;
      if (slot >= ntok) continue;
      const int o = orow[slot];
      if constexpr (kUp) {
        const float gv = acc[g][0][r], uv = acc[g][1][r];
        reinterpret_cast<float*>(out)[(size_t)o * kFf + n] = gv / (1.f + expf(-gv)) * uv;
      } else if constexpr (KIND == MOE_DN) {
        reinterpret_cast<uint16_t*>(out)[(size_t)o * kHid + n] = tlx_f2h_bits(acc[g][0][r]);
      } else {
        reinterpret_cast<float*>(out)[(size_t)o * kHid + n] = acc[g][0][r];
      }
    }
  }
}

// Modes: dense (the shared expert, KIND *_DENSE: chunks of kTok positions); pair walk (eids:
// workgroup column x is pair x); pair walk fused with the shared expert (eids and ptbl_sh: columns
// x < 8 P are pairs, the rest the shared expert's chunks, which read xs_sh and write out_sh with
// the dense kind's epilogue); grouped (the sort's items).
template <int KIND, bool TL>
__global__ __launch_bounds__(256) void moe_gv_kernel(const uint64_t* __restrict__ ptbl, const int* __restrict__ eoff,
                                                     const uint16_t* __restrict__ plist,
                                                     const uint32_t* __restrict__ items, const uint32_t* __restrict__ nitp,
                                                     const uint16_t* __restrict__ eids, const float* __restrict__ xs,
                                                     const float* __restrict__ iq4nl, void* __restrict__ out, int P,
                                                     const uint64_t* __restrict__ ptbl_sh, const float* __restrict__ xs_sh,
                                                     void* __restrict__ out_sh, int swap) {
  // workgroup column (item, pair or chunk) and row (output tile group): swapped grids dispatch an
  // item's tile groups one after another (consecutive workgroups stream one expert slab)
  const uint32_t bx = swap ? blockIdx.y : blockIdx.x, by = swap ? blockIdx.x : blockIdx.y;
  constexpr bool kDense = KIND == MOE_DN_DENSE || KIND == MOE_UP_DENSE;
  constexpr int KD = KIND == MOE_UP ? MOE_UP_DENSE : KIND == MOE_DN ? MOE_DN_DENSE : KIND;   // the dense kind
  constexpr bool kUp = KIND == MOE_UP || KIND == MOE_UP_DENSE;
  constexpr int NMAT = kUp ? 2 : 1;
  constexpr int kTpw = 4 / moe_gv_wpt<KIND>();    // tiles per workgroup
  __shared__ uint32_t lut[256];
  __shared__ int xrow[kTok], orow[kTok];
  // reduction slots: one per tile shared by two waves (gate+up); the down tiles are one wave's
  // (16 KB: the workgroup's 30 KB of LDS leave residency to the register budget, 3 waves/SIMD)
  __shared__ f4_t red[(moe_gv_wpt<KIND>() > 1 ? 4 / moe_gv_wpt<KIND>() : 1) * kGvGroups * NMAT * 64];
  // Items of at most kGvStageRows tokens (decode: one or two) stage their token rows once, fp16
  // in the MFMA k order, row stride K / 8 + 1 pieces: read from global inside the decode loop,
  // each chunk's activations cost a serialized L2 round trip.
  constexpr int kK = MoeShape<KIND>::K, kPr = kK / 8 + 1;
  constexpr int kGvStageRows = 1024 / kPr;   // rows in 16 KB: 3 (gate+up, K = 2048), 15 (down)
  __shared__ u4_t xst[kGvStageRows * kPr];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;

  int m0, ntok;
  gbyte* base;
  // a shared-expert chunk of the fused pair walk (workgroup-uniform)
  const bool shc = !kDense && eids && ptbl_sh && (int)bx >= 8 * P;
  if (shc) {   // chunks of kShTok positions: one token group, the pair walk's register budget
    m0 = ((int)bx - 8 * P) * kShTok;
    ntok = min(kShTok, P - m0);
    base = (gbyte*)(ptbl_sh[0]);
    xs = xs_sh;
    out = out_sh;
  } else if constexpr (kDense) {
    m0 = (int)bx * kTok;
    ntok = min(kTok, P - m0);
    base = (gbyte*)(ptbl[0]);
  } else if (eids) {   // pair walk: workgroup column x is pair x, expert eids[x], no sort
    m0 = (int)bx;
    ntok = 1;
    base = (gbyte*)(ptbl[eids[m0]]);
  } else {
    if (bx >= *nitp) return;
    const uint32_t it = items[bx];
    const int e = (int)(it >> 16);
    m0 = (int)(it & 0xFFFFu);
    const int eb0 = eoff[e];
    ntok = min(kTok, eoff[e + 1] - eb0 - m0);
    m0 += eb0;
    base = (gbyte*)(ptbl[e]);
  }
  if (t < kTok) {
    const int slot = min(t, ntok - 1);
    if (kDense || shc) {
      xrow[t] = m0 + slot;
      orow[t] = m0 + slot;
    } else if (eids) {
      xrow[t] = kUp ? (m0 >> 3) : m0;
      orow[t] = m0;
    } else {
      const int pair = plist[m0 + slot];
      xrow[t] = kUp ? (pair >> 3) : pair;
      orow[t] = pair;
    }
  }
  {
    const _Float16 lo = (_Float16)iq4nl[t & 15], hi = (_Float16)iq4nl[t >> 4];
    lut[t] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  __syncthreads();
  const bool staged = ntok <= kGvStageRows;   // workgroup-uniform
  if (staged) {
    // piece q = row * (K / 8) + p: sub-block p / 4, chunk p % 4 -- x[32 (p / 4) + 4 (p % 4) + {0, 16, 1,
    // 17, 2, 18, 3, 19}]
    for (int q = t; q < ntok * (kK / 8); q += 256) {
      const int row = q / (kK / 8), p = q - row * (kK / 8);
      const float* src = xs + (size_t)xrow[row] * kK + 32 * (p >> 2) + 4 * (p & 3);
      const float4 v0 = *reinterpret_cast<const float4*>(src), v1 = *reinterpret_cast<const float4*>(src + 16);
      const h8_t hv = {(_Float16)v0.x, (_Float16)v1.x, (_Float16)v0.y, (_Float16)v1.y,
                       (_Float16)v0.z, (_Float16)v1.z, (_Float16)v0.w, (_Float16)v1.w};
      xst[row * kPr + p] = __builtin_bit_cast(u4_t, hv);
    }
    __syncthreads();
  }
  const int tile = (int)by * kTpw + wave / moe_gv_wpt<KIND>();   // 16-row output tile
  if constexpr (KIND == MOE_DN) {   // gate+up: the dense kind's tile is the routed one's code
    if (shc) {   // the dense kind's tile (the down projection's epilogue differs: f32 out)
      if (staged) moe_gv_tile<KD, 1, TL, true>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane);
      else moe_gv_tile<KD, 1, TL, false>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane);
      return;
    }
  }
  switch ((ntok + 15) >> 4) {   // workgroup-uniform
    case 1:
      if (staged) moe_gv_tile<KIND, 1, TL, true>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane);
      else moe_gv_tile<KIND, 1, TL, false>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane);
      break;
    case 2: moe_gv_tile<KIND, 2, TL, false>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane); break;
    case 3: moe_gv_tile<KIND, 3, TL, false>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane); break;
    default: moe_gv_tile<KIND, 4, TL, false>(base, lut, xrow, orow, red, xst, xs, out, ntok, tile, wave, lane); break;
  }
}

// ------------------------------------------------------------------ combine
// y = hres + (sum_r g_r * part_r (r ascending) + sg * shared), fp32; 8 elements per thread.
__global__ __launch_bounds__(64) void moe_combine_kernel(const uint16_t* __restrict__ parts, const float* __restrict__ gates,
                                                          const float* __restrict__ sg, const float* __restrict__ shared,
                                                          const float* __restrict__ hres, float* __restrict__ y) {
  // four one-wave workgroups a position (measured against one of four waves: P = 2048 18.3 ->
  // 17.3 us, P = 11 2.07 -> 1.95 us)
  const int p = blockIdx.x >> 2, i0 = 8 * (threadIdx.x + 64 * (blockIdx.x & 3));
  float g[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; ++r) g[r] = gates[p * kTopK + r];
  const float sgp = sg[p];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    const h8_t v = *reinterpret_cast<const h8_t*>(parts + ((size_t)p * kTopK + r) * kHid + i0);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = __builtin_fmaf(g[r], (float)v[k], acc[k]);
  }
  const float* sh = shared + (size_t)p * kHid + i0;
  const float* hr = hres + (size_t)p * kHid + i0;
  float* yo = y + (size_t)p * kHid + i0;
#pragma unroll
  for (int k = 0; k < 8; ++k) yo[k] = hr[k] + __builtin_fmaf(sgp, sh[k], acc[k]);
}

int moe_max_items(int np) { return (np + moe_item_tok(np) - 1) / moe_item_tok(np) + kE; }

}  // namespace

extern "C" int tlx_moe_topk(const float* logits, uint16_t* eids, float* gates, int P, void* stream) {
  TLX_RET_IF(P < 1, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(logits, 16), TLX_E_ALIGN);
  moe_topk_kernel<<<(P + 15) / 16, 256, 0, (hipStream_t)stream>>>(logits, eids, gates, P);
  return tlx_launch_status();
}

extern "C" int tlx_moe_route(const float* wrt, const float* wsh, const float* h, uint16_t* eids, float* gates,
                             float* sg, int P, void* stream) {
  TLX_RET_IF(P < 1, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(wrt, 16) || !tlx_aligned(h, 16) || !tlx_aligned(wsh, 8), TLX_E_ALIGN);
  moe_route_kernel<<<P, 256, 0, (hipStream_t)stream>>>(wrt, wsh, h, eids, gates, sg);
  return tlx_launch_status();
}

extern "C" int tlx_moe_sort(const uint16_t* eids, int* eoff, uint16_t* plist, uint32_t* items, uint32_t* nitp,
                            int np, void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(eids, 8), TLX_E_ALIGN);
  moe_sort_kernel<<<(np + kSortChunk - 1) / kSortChunk, kSortChunk, 0, (hipStream_t)stream>>>(eids, eoff, plist,
                                                                                            items, nitp, np);
  return tlx_launch_status();
}

extern "C" int tlx_moe_max_items(int np) { return moe_max_items(np); }

// work items the sort can produce for np pairs: at most ceil(np / 64) + 256 (one partial
// chunk per expert), and at most np (every item holds a pair) -- the small-batch grids use both
int moe_gv_items(int np) { return min(np, moe_max_items(np)); }

// items (expert chunks) rounded up to a multiple of 8 (one per XCD), times the stripes
template <int KIND>
int moe_pf_grid(int nitems) { return (nitems + 7) / 8 * 8 * moe_pf_stripes<KIND>(); }

// Grids of at least kGvSwapCols columns run swapped (measured: 2% faster at 512 pairs, 17% at
// 2048; at decode widths the column-major order is as fast or faster).
constexpr int kGvSwapCols = 128;
template <int KIND>
dim3 moe_gv_grid(int nx) {
  constexpr int kWpt = moe_gv_wpt<KIND>(), kTpw = 4 / kWpt;
  constexpr int kRows = (KIND == MOE_UP || KIND == MOE_UP_DENSE) ? kFf : kHid;
  return nx >= kGvSwapCols ? dim3(kRows / 16 / kTpw, nx) : dim3(nx, kRows / 16 / kTpw);
}

// launch helpers: the layout picks the kernel instantiation (GGUF rows or tiled records)
template <int KIND>
void moe_gv_launch(bool tl, dim3 grid, hipStream_t st, const uint64_t* ptbl, const int* eoff, const uint16_t* plist,
                   const uint32_t* items, const uint32_t* nitp, const uint16_t* eids, const float* xs,
                   const float* iq4nl, void* out, int P, const uint64_t* ptbl_sh = nullptr,
                   const float* xs_sh = nullptr, void* out_sh = nullptr) {
  constexpr int kTiles = ((KIND == MOE_UP || KIND == MOE_UP_DENSE) ? kFf : kHid) / 16 / (4 / moe_gv_wpt<KIND>());
  const int swap = grid.x == (unsigned)kTiles && grid.y >= (unsigned)kGvSwapCols;
  if (tl)
    moe_gv_kernel<KIND, true><<<grid, 256, 0, st>>>(ptbl, eoff, plist, items, nitp, eids, xs, iq4nl, out, P, ptbl_sh,
                                                     xs_sh, out_sh, swap);
  else
    moe_gv_kernel<KIND, false><<<grid, 256, 0, st>>>(ptbl, eoff, plist, items, nitp, eids, xs, iq4nl, out, P, ptbl_sh,
                                                      xs_sh, out_sh, swap);
}

template <int KIND>
void moe_pf_launch(bool tl, int nitems, hipStream_t st, const uint64_t* ptbl, const int* eoff, const uint16_t* plist,
                   const uint32_t* items, const uint32_t* nitp, const float* xs, const float* iq4nl, void* out, int P) {
  const int grid = moe_pf_grid<KIND>(nitems);
  if (tl)
    moe_pf_kernel<KIND, true><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P);
  else
    moe_pf_kernel<KIND, false><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P);
}

template <int KIND>
void moe_pd_launch(bool tl, int nitems, hipStream_t st, const uint64_t* ptbl, const int* eoff, const uint16_t* plist,
                   const uint32_t* items, const uint32_t* nitp, const float* xs, const float* iq4nl, void* out, int P,
                   int tok = kPfTok) {
  const dim3 grid(nitems, KIND == MOE_DN_DENSE ? 4 : 1);   // dense: one stripe per workgroup
  if (tl)
    moe_pd_kernel<KIND, true><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P, tok);
  else
    moe_pd_kernel<KIND, false><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, out, P, tok);
}

bool moe_layout_ok(int layout) { return layout == TLX_LAYOUT_RAW || layout == TLX_LAYOUT_TILED; }

extern "C" int tlx_moe_up4(const uint64_t* ptbl, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                           const uint16_t* plist, const float* xs, const float* iq4nl, float* ys, int np, int layout,
                           void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(xs, 16) || !tlx_aligned(ys, 16), TLX_E_ALIGN);
  const bool tl = layout == TLX_LAYOUT_TILED;
  const hipStream_t st = (hipStream_t)stream;
  if (np <= kGvUpMaxPairs)
    moe_gv_launch<MOE_UP>(tl, moe_gv_grid<MOE_UP>(moe_gv_items(np)), st, ptbl, eoff, plist, items, nitp, nullptr, xs,
                          iq4nl, ys, 0);
  else
    moe_pf_launch<MOE_UP>(tl, moe_max_items(np), st, ptbl, eoff, plist, items, nitp, xs, iq4nl, ys, 0);
  return tlx_launch_status();
}

extern "C" int tlx_moe_dn4(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                           const uint16_t* plist, const float* act, const float* iq4nl, uint16_t* parts, int np,
                           int layout, void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(act, 16) || !tlx_aligned(parts, 16), TLX_E_ALIGN);
  const bool tl = layout == TLX_LAYOUT_TILED;
  const hipStream_t st = (hipStream_t)stream;
  if (np <= kGvDnMaxPairs)
    moe_gv_launch<MOE_DN>(tl, moe_gv_grid<MOE_DN>(moe_gv_items(np)), st, ptbl_dn, eoff, plist, items, nitp, nullptr,
                          act, iq4nl, parts, 0);
  else
    moe_pd_launch<MOE_DN>(tl, moe_max_items(np), st, ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts, 0,
                          moe_item_tok(np));
  return tlx_launch_status();
}

extern "C" int tlx_moe_up4_pairs(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* iq4nl,
                                 float* ys, int np, int layout, void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(xs, 16), TLX_E_ALIGN);
  moe_gv_launch<MOE_UP>(layout == TLX_LAYOUT_TILED, moe_gv_grid<MOE_UP>(np), (hipStream_t)stream, ptbl, nullptr,
                        nullptr, nullptr, nullptr, eids, xs, iq4nl, ys, 0);
  return tlx_launch_status();
}

extern "C" int tlx_moe_dn4_pairs(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, const float* iq4nl,
                                 uint16_t* parts, int np, int layout, void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(act, 16) || !tlx_aligned(parts, 16), TLX_E_ALIGN);
  moe_gv_launch<MOE_DN>(layout == TLX_LAYOUT_TILED, moe_gv_grid<MOE_DN>(np), (hipStream_t)stream, ptbl_dn, nullptr,
                        nullptr, nullptr, nullptr, eids, act, iq4nl, parts, 0);
  return tlx_launch_status();
}

extern "C" int tlx_moe_up4_pairs_sh(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* iq4nl,
                                    float* ys, const uint64_t* ptbl_sh, float* sact, int P, int layout, void* stream) {
  TLX_RET_IF(P < 1 || 8 * P > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(xs, 16) || !tlx_aligned(sact, 16), TLX_E_ALIGN);
  const dim3 g = moe_gv_grid<MOE_UP>(8 * P + (P + kShTok - 1) / kShTok);
  moe_gv_launch<MOE_UP>(layout == TLX_LAYOUT_TILED, g, (hipStream_t)stream, ptbl, nullptr, nullptr, nullptr, nullptr,
                        eids, xs, iq4nl, ys, P, ptbl_sh, xs, sact);
  return tlx_launch_status();
}

extern "C" int tlx_moe_dn4_pairs_sh(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act,
                                    const float* iq4nl, uint16_t* parts, const uint64_t* ptbl_sh_dn, const float* sact,
                                    float* shared, int P, int layout, void* stream) {
  TLX_RET_IF(P < 1 || 8 * P > kMaxPairs || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(act, 16) || !tlx_aligned(parts, 16) || !tlx_aligned(sact, 16) || !tlx_aligned(shared, 16),
             TLX_E_ALIGN);
  const dim3 g = moe_gv_grid<MOE_DN>(8 * P + (P + kShTok - 1) / kShTok);
  moe_gv_launch<MOE_DN>(layout == TLX_LAYOUT_TILED, g, (hipStream_t)stream, ptbl_dn, nullptr, nullptr, nullptr, nullptr,
                        eids, act, iq4nl, parts, P, ptbl_sh_dn, sact, shared);
  return tlx_launch_status();
}

// the shared expert's gate+up (act) and down (out) alone: GEMV forms up to kGvSharedMaxP positions
int moe_shared_up(bool tl, int P, hipStream_t st, const uint64_t* ptbl_sh, const float* xs, const float* iq4nl,
                  float* act) {
  if (P <= kGvSharedMaxP)
    moe_gv_launch<MOE_UP_DENSE>(tl, moe_gv_grid<MOE_UP_DENSE>((P + kTok - 1) / kTok), st, ptbl_sh, nullptr, nullptr,
                                nullptr, nullptr, nullptr, xs, iq4nl, act, P);
  else
    moe_pf_launch<MOE_UP_DENSE>(tl, (P + kDenseTok - 1) / kDenseTok, st, ptbl_sh, nullptr, nullptr, nullptr, nullptr,
                                xs, iq4nl, act, P);
  return tlx_launch_status();
}

int moe_shared_dn(bool tl, int P, hipStream_t st, const uint64_t* ptbl_sh_dn, const float* act, const float* iq4nl,
                  float* out) {
  if (P <= kGvSharedMaxP)
    moe_gv_launch<MOE_DN_DENSE>(tl, moe_gv_grid<MOE_DN_DENSE>((P + kTok - 1) / kTok), st, ptbl_sh_dn, nullptr,
                                nullptr, nullptr, nullptr, nullptr, act, iq4nl, out, P);
  else
    moe_pd_launch<MOE_DN_DENSE>(tl, (P + kDenseTok - 1) / kDenseTok, st, ptbl_sh_dn, nullptr, nullptr, nullptr,
                                nullptr, act, iq4nl, out, P);
  return tlx_launch_status();
}

extern "C" int tlx_moe_shared(const uint64_t* ptbl_sh, const float* xs, const float* iq4nl, float* act, float* out,
                              int P, int layout, void* stream) {
  TLX_RET_IF(P < 1 || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(xs, 16) || !tlx_aligned(act, 16) || !tlx_aligned(out, 16), TLX_E_ALIGN);
  const bool tl = layout == TLX_LAYOUT_TILED;
  const hipStream_t st = (hipStream_t)stream;
  const int rc = moe_shared_up(tl, P, st, ptbl_sh, xs, iq4nl, act);
  TLX_RET_IF(rc != TLX_OK, rc);
  return moe_shared_dn(tl, P, st, ptbl_sh + 1, act, iq4nl, out);
}

extern "C" int tlx_moe_up4_sh(const uint64_t* ptbl, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                              const uint16_t* plist, const float* xs, const float* iq4nl, float* ys, int np,
                              const uint64_t* ptbl_sh, float* sact, int P, int layout, void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(xs, 16) || !tlx_aligned(ys, 16) || !tlx_aligned(sact, 16), TLX_E_ALIGN);
  const bool tl = layout == TLX_LAYOUT_TILED;
  const hipStream_t st = (hipStream_t)stream;
  if (np <= kGvUpMaxPairs || P <= kGvSharedMaxP) {   // a GEMV form on either side: the two launches
    const int rc = tlx_moe_up4(ptbl, items, nitp, eoff, plist, xs, iq4nl, ys, np, layout, stream);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared_up(tl, P, st, ptbl_sh, xs, iq4nl, sact);
  }
  const int nrb = moe_pf_grid<MOE_UP>(moe_max_items(np));
  const int grid = nrb + moe_pf_grid<MOE_UP_DENSE>((P + kDenseTok - 1) / kDenseTok);
  if (tl)
    moe_pf_sh_kernel<true><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, ys, ptbl_sh, sact,
                                                       P, nrb);
  else
    moe_pf_sh_kernel<false><<<grid, kPfThreads, 0, st>>>(ptbl, eoff, plist, items, nitp, xs, iq4nl, ys, ptbl_sh, sact,
                                                        P, nrb);
  return tlx_launch_status();
}

extern "C" int tlx_moe_dn4_sh(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                              const uint16_t* plist, const float* act, const float* iq4nl, uint16_t* parts, int np,
                              const uint64_t* ptbl_sh_dn, const float* sact, float* shared, int P, int layout,
                              void* stream) {
  TLX_RET_IF(np < 1 || np > kMaxPairs || P < 1 || !moe_layout_ok(layout), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(act, 16) || !tlx_aligned(parts, 16) || !tlx_aligned(sact, 16) || !tlx_aligned(shared, 16),
             TLX_E_ALIGN);
  const bool tl = layout == TLX_LAYOUT_TILED;
  const hipStream_t st = (hipStream_t)stream;
  if (np <= kGvDnMaxPairs || P <= kGvSharedMaxP) {
    const int rc = tlx_moe_dn4(ptbl_dn, items, nitp, eoff, plist, act, iq4nl, parts, np, layout, stream);
    TLX_RET_IF(rc != TLX_OK, rc);
    return moe_shared_dn(tl, P, st, ptbl_sh_dn, sact, iq4nl, shared);
  }
  const int nitems = moe_max_items(np);
  const int grid = nitems + 4 * ((P + kDenseTok - 1) / kDenseTok);
  if (tl)
    moe_pd_sh_kernel<true><<<grid, kPfThreads, 0, st>>>(ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts,
                                                       moe_item_tok(np), ptbl_sh_dn, sact, shared, P, nitems);
  else
    moe_pd_sh_kernel<false><<<grid, kPfThreads, 0, st>>>(ptbl_dn, eoff, plist, items, nitp, act, iq4nl, parts,
                                                        moe_item_tok(np), ptbl_sh_dn, sact, shared, P, nitems);
  return tlx_launch_status();
}

// ------------------------------------------------------------------ tiled slab repacker
// One thread per 8 output bytes: record u = (tile, block) word w -- w < 16: row 16 tile + w's
// block header; else lane region (w - 16) / 128 (sub-blocks kq, then kq + 4), lane l, half q:
// row 16 tile + (l & 15)'s quant bytes 64 region + 16 (l >> 4) + 8 q.  All reads are 8-B aligned
// (block starts are multiples of 8 bytes).
__global__ __launch_bounds__(256) void pack_iq4_tiled_kernel(const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst, long nwords, int nb) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= nwords) return;
  const long u = i / 272;
  const int w = (int)(i - u * 272);
  const long tile = u / nb;
  const int b = (int)(u - tile * nb);
  const long rb = 136L * nb;
  long off;
  if (w < 16) {
    off = (tile * 16 + w) * rb + 136L * b;
  } else {
    const int o = 8 * (w - 16), reg = o >> 10, l = (o & 1023) >> 4, q = (o >> 3) & 1;
    off = (tile * 16 + (l & 15)) * rb + 136L * b + 8 + 64 * reg + 16 * (l >> 4) + 8 * q;
  }
  reinterpret_cast<u2_t*>(dst)[i] = *reinterpret_cast<const u2_t*>(src + off);
}

extern "C" int tlx_pack_iq4_tiled(const void* src, void* tiled, int N, int K, void* stream) {
  TLX_RET_IF(N < 16 || (N % 16) || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(src, 8) || !tlx_aligned(tiled, 8), TLX_E_ALIGN);
  const long nwords = (long)(N / 16) * (K / 256) * 272;
  pack_iq4_tiled_kernel<<<(unsigned)((nwords + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)src, (uint8_t*)tiled, nwords, K / 256);
  return tlx_launch_status();
}

extern "C" int tlx_moe_combine(const uint16_t* parts, const float* gates, const float* sg, const float* shared,
                               const float* hres, float* y, int P, void* stream) {
  TLX_RET_IF(P < 1, TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(parts, 16), TLX_E_ALIGN);
  moe_combine_kernel<<<4 * P, 64, 0, (hipStream_t)stream>>>(parts, gates, sg, shared, hres, y);
  return tlx_launch_status();
}
