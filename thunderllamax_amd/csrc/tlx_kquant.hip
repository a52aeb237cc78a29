// K-quant decode GEMVs for gfx950 with fp16 activations: Q6_K (raw 210-B and padded 212-B
// blocks), fp16 outputs.  The q-branch of the fused attention projections and the Q6_K head.
//
// Design (one kernel for every M that fits the LDS budget; larger M runs in row groups):
//   * the activation block X[M][K] is staged once per workgroup in LDS with a row stride of
//     2K+16 bytes, so the 8 lanes of one LDS read phase fall on distinct 16-B slots;
//   * a workgroup owns a contiguous range of 16-row tiles, and its (tile, block) items are
//     split into 8 equal contiguous ranges, one per wave: every wave streams the same number
//     of weight bytes whatever the tile count;
//   * weights are read with quad-coalesced 16-B loads (4 lanes cover 64 contiguous bytes of
//     one row), written to a per-wave LDS staging tile in row order and read back in MFMA
//     fragment order (lane (col, kq) receives row col's bytes for its k-quarter);
//   * decode: q = ql nibble | (qh 2 bits) << 4 for 4 weights per dword, fp16 pairs 1 + q/1024
//     by v_perm with 0x3C bytes, minus 33/32 gives (q-32)/1024 exactly, times the int8 group
//     scale gives fp16(sc*(q-32))/1024 with one rounding (the size of the reference's own fp16
//     weight rounding); v_mfma_f32_16x16x32_f16 accumulates in fp32 and d*1024 is applied
//     once per block;
//   * tiles split between waves are combined through LDS in wave order after the main loop,
//     so results do not depend on scheduling.
#include "tlx_common.h"

#include <mutex>

namespace {

constexpr int kWaves = 8;
constexpr int kStgRow = 240;            // staging bytes per weight row (16 x odd: conflict-free)
constexpr int kStgItem = 16 * kStgRow;  // one item: 16 rows x one 256-weight block
constexpr int kSlot = 64 * 16;          // one wave's 16x16 fp32 partial tile
constexpr int kLdsMax = 160 * 1024;
constexpr int kPrefetch = 2;          // items in flight per wave (even: fragments ping-pong)

struct Q6Geo {
  int bs, qoff, scoff, doff;  // block bytes; offsets of ql (qh follows), scales, d
};
__host__ __device__ constexpr Q6Geo q6_geo(int layout) {
  return layout == TLX_LAYOUT_RAW ? Q6Geo{210, 0, 192, 208} : Q6Geo{212, 20, 4, 2};
}

struct KqArgs {
  const uint8_t* w;    // N rows x nb blocks
  const _Float16* x;   // [M][K]
  uint16_t* out;       // [M][N] fp16
  int M, N, K;
  int tw;              // tiles per workgroup
};

struct Q6Ld {  // one lane's share of an item as loaded: 48 B of ql/qh, a scale dword, d
  u4_t q[3];
  uint32_t sc, d;
};

struct Q6Frag {  // one lane's share in fragment order: 32 ql bytes, 32 qh bytes, 8 scales, d
  u4_t ql[2], qh[2];
  u2_t sc;
  uint32_t d;
};

// `off` is the block's 32-bit byte offset from the matrix base (scalar base + vector offset)
template <int LAYOUT>
__device__ __forceinline__ void q6_load(Q6Ld& L, const uint8_t* w, uint32_t off, int c) {
  constexpr Q6Geo G = q6_geo(LAYOUT);
#pragma unroll
  for (int j = 0; j < 3; ++j) L.q[j] = tlx_ldu<u4_t>(w + (off + G.qoff + 64 * j + 16 * c));
  L.sc = tlx_ldu<uint32_t>(w + (off + G.scoff + 4 * c));
  L.d = tlx_ldu<uint16_t>(w + (off + G.doff));
}

// staging row r: [ql 128][qh 64][sc 16][d 2][pad]
__device__ __forceinline__ void q6_stage(uint8_t* stg, const Q6Ld& L, int r, int c) {
  uint8_t* s = stg + r * kStgRow;
#pragma unroll
  for (int j = 0; j < 3; ++j) *reinterpret_cast<u4_t*>(s + 64 * j + 16 * c) = L.q[j];
  *reinterpret_cast<uint32_t*>(s + 192 + 4 * c) = L.sc;
  if (c == 0) *reinterpret_cast<uint16_t*>(s + 208) = (uint16_t)L.d;
}

// lane (col, kq = 2h + e) owns the elements k = 128h + 32g + l with g in {e, e + 2}: ql bytes
// [64h + 32e, +32), qh bytes [32h, +32), scales sc[8h .. 8h + 8).
__device__ __forceinline__ void q6_frag(Q6Frag& F, const uint8_t* stg, int col, int h, int e) {
  const uint8_t* f = stg + col * kStgRow;
  F.ql[0] = *reinterpret_cast<const u4_t*>(f + 64 * h + 32 * e);
  F.ql[1] = *reinterpret_cast<const u4_t*>(f + 64 * h + 32 * e + 16);
  F.qh[0] = *reinterpret_cast<const u4_t*>(f + 128 + 32 * h);
  F.qh[1] = *reinterpret_cast<const u4_t*>(f + 144 + 32 * h);
  F.sc = *reinterpret_cast<const u2_t*>(f + 192 + 8 * h);
  F.d = *reinterpret_cast<const uint16_t*>(f + 208);
}

// fp16 pairs (1 + q/1024) of bytes 0,1 (sel 0x04010400) or 2,3 (sel 0x04030402) of q
__device__ __forceinline__ h2_t q6_pair(uint32_t q, uint32_t sel) {
  return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x3C3C3C3Cu, q, sel));
}

// MFMA o = 4*nib + u covers, for lane (col, 2h + e), the 8 elements
// k = 128h + 32(e + 2nib) + 8u + i: ql bytes 8u..8u+7 (nibble nib), qh bytes 8u..8u+7
// (bits 2e + 4nib), scale byte (u >> 1) + 2e + 4nib of the lane's 8.  A[o] holds the
// matching 8 activations of the lane's row.
__device__ __forceinline__ f4_t q6_block(const Q6Frag& F, const h8_t* A, int e) {
  f4_t D = {0.f, 0.f, 0.f, 0.f};
  const h2_t off = {(_Float16)-1.03125f, (_Float16)-1.03125f};
#pragma unroll
  for (int nib = 0; nib < 2; ++nib) {
    const int sh = 2 * e + 4 * nib;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sb = (u >> 1) + 2 * e + 4 * nib;
      const uint32_t sw = sb < 4 ? F.sc.x : F.sc.y;
      const _Float16 s = (_Float16)(float)(int8_t)(uint8_t)(sw >> (8 * (sb & 3)));
      const h2_t sp = {s, s};
      const u4_t& L4 = F.ql[u >> 1];
      const u4_t& H4 = F.qh[u >> 1];
      const uint32_t l0 = (u & 1) ? L4.z : L4.x, l1 = (u & 1) ? L4.w : L4.y;
      const uint32_t g0 = (u & 1) ? H4.z : H4.x, g1 = (u & 1) ? H4.w : H4.y;
      const uint32_t q0 = ((l0 >> (4 * nib)) & 0x0F0F0F0Fu) | (((g0 >> sh) & 0x03030303u) << 4);
      const uint32_t q1 = ((l1 >> (4 * nib)) & 0x0F0F0F0Fu) | (((g1 >> sh) & 0x03030303u) << 4);
      const h2_t p0 = (q6_pair(q0, 0x04010400u) + off) * sp;
      const h2_t p1 = (q6_pair(q0, 0x04030402u) + off) * sp;
      const h2_t p2 = (q6_pair(q1, 0x04010400u) + off) * sp;
      const h2_t p3 = (q6_pair(q1, 0x04030402u) + off) * sp;
      const h8_t B = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
      D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[4 * nib + u], B, D, 0, 0, 0);
    }
  }
  return D;
}

__device__ __forceinline__ int kq_range(int I, int w) { return (int)((int64_t)I * w / kWaves); }

template <int LAYOUT>
__global__ __launch_bounds__(kWaves * TLX_WAVE) void q6_gemv16_kernel(const KqArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr Q6Geo G = q6_geo(LAYOUT);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int M = a.M, N = a.N, K = a.K, nb = K >> 8;
  const int XS = K + 8;  // halves per staged activation row
  const int xbytes = max(M * XS * 2, kWaves * 2 * kSlot);
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  uint8_t* stg = lds + xbytes + wave * kStgItem;

  const int T = (N + 15) >> 4;
  const int t0 = (int)blockIdx.x * a.tw;
  const int I = min(a.tw, T - t0) * nb;
  const int lo = kq_range(I, wave), hi = kq_range(I, wave + 1);

  const int r = lane >> 2, c = lane & 3;       // load role: row r, 16-B piece c of each 64 B
  const int col = lane & 15, kq = lane >> 4;   // MFMA role
  const int h = kq >> 1, e = kq & 1;
  const uint32_t rowb = (uint32_t)G.bs * nb;
  auto blk_of = [&](int i) -> uint32_t {
    const int t = t0 + i / nb, b = i - (i / nb) * nb;
    const int n = min(16 * t + r, N - 1);  // tail tile: clamp the loads, mask the stores
    return (uint32_t)n * rowb + (uint32_t)b * G.bs;
  };

  // Every load, staging write and fragment read below is unconditional (item indices are
  // clamped to the wave's last item), so the loop body is straight-line and the compiler's
  // wait counts stay exact.
  const int last = hi - 1;
  Q6Ld g[kPrefetch];  // ring: item i sits in g[(i - lo) % kPrefetch] until it is staged
  if (lo < hi) {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) q6_load<LAYOUT>(g[p], a.w, blk_of(min(lo + p, last)), c);
  }

  // activations: 1-KB LDS-DMA pieces (row m, halves [512j, 512j + 512)), in flight together
  // with the weight prefetch; when K % 512 == 256 a row's last piece is half a wave wide
  {
    const int pr = (K + 511) >> 9;
    for (int p = wave; p < M * pr; p += kWaves) {
      const int m = p / pr, j = p - m * pr;
      if (512 * j + 8 * lane < K)
        __builtin_amdgcn_global_load_lds(
            (const void*)(a.x + (size_t)m * K + 512 * j + 8 * lane),
            (__attribute__((address_space(3))) void*)(xs + m * XS + 512 * j), 16, 0, 0);
    }
  }
  __syncthreads();

  // activation rows >= M feed output rows that are never stored: read a valid row instead
  const _Float16* xa = xs + min(col, M - 1) * XS + 128 * h + 32 * e;

  auto store = [&](const f4_t& v, int t) {
    const int n = 16 * t + col;
    if (n >= N) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 4 * kq + j;
      if (m < M) a.out[(size_t)m * N + n] = tlx_f2h_bits(v[j]);
    }
  };

  f4_t acc = {0.f, 0.f, 0.f, 0.f}, accFirst = acc, accLast = acc;
  Q6Frag F[2];  // item i's fragments in F[(i - lo) & 1]
  if (lo < hi) {
    q6_stage(stg, g[0], r, c);
    q6_frag(F[0], stg, col, h, e);
    q6_load<LAYOUT>(g[0], a.w, blk_of(min(lo + kPrefetch, last)), c);
  }
  int seg = lo;
  for (int i0 = lo; i0 < hi; i0 += kPrefetch) {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int i = i0 + p;  // i >= hi: padding steps of the last round, computed and discarded
      const int ic = min(i, last);
      const int tl = ic / nb, b = ic - tl * nb;
      h8_t A[8];
#pragma unroll
      for (int o = 0; o < 8; ++o)
        A[o] = *reinterpret_cast<const h8_t*>(xa + 256 * b + 64 * (o >> 2) + 8 * (o & 3));
      // item i+1 goes through the single staging tile after item i's fragment reads were
      // issued (LDS executes a wave's instructions in order); its ring slot is then refilled
      q6_stage(stg, g[(p + 1) % kPrefetch], r, c);
      q6_frag(F[(p + 1) & 1], stg, col, h, e);
      const f4_t D = q6_block(F[p & 1], A, e);
      q6_load<LAYOUT>(g[(p + 1) % kPrefetch], a.w, blk_of(min(i + 1 + kPrefetch, last)), c);
      if (i < hi) {
        acc += (tlx_h2f((uint16_t)F[p & 1].d) * 1024.0f) * D;
        if (b == nb - 1 || i == hi - 1) {  // end of a tile segment
          if (seg - tl * nb == 0 && b == nb - 1) store(acc, t0 + tl);
          else if (tl == lo / nb) accFirst = acc;
          else accLast = acc;
          acc = f4_t{0.f, 0.f, 0.f, 0.f};
          seg = i + 1;
        }
      }
    }
  }

  // ---- tiles shared by consecutive waves: partial sums through LDS, combined in wave order
  __syncthreads();  // every wave is done with the staged activations and its staging tile
  float* slots = reinterpret_cast<float*>(lds);
  const int tf = lo / nb, tlast = (hi - 1) / nb;
  const bool firstPartial = lo < hi && !(lo % nb == 0 && (tf + 1) * nb <= hi);
  const bool lastPartial = lo < hi && tlast != tf && hi % nb != 0;
  if (firstPartial) *reinterpret_cast<f4_t*>(slots + ((wave * 2 + 0) * 64 + lane) * 4) = accFirst;
  if (lastPartial) *reinterpret_cast<f4_t*>(slots + ((wave * 2 + 1) * 64 + lane) * 4) = accLast;
  __syncthreads();
  // the wave holding a tile's last item combines it when the tile began in an earlier wave
  if (lo < hi && lo % nb != 0 && (tf + 1) * nb <= hi) {
    f4_t sum = {0.f, 0.f, 0.f, 0.f};
    for (int v = 0; v < wave; ++v) {
      const int lov = kq_range(I, v), hiv = kq_range(I, v + 1);
      if (lov >= hiv || hiv <= tf * nb) continue;
      const int slot = lov / nb == tf ? 0 : 1;
      sum += *reinterpret_cast<const f4_t*>(slots + ((v * 2 + slot) * 64 + lane) * 4);
    }
    sum += accFirst;
    store(sum, t0 + tf);
  }
}

inline size_t q6_lds_bytes(int M, int K) {
  const size_t xb = std::max((size_t)M * (K + 8) * 2, (size_t)kWaves * 2 * kSlot);
  return xb + (size_t)kWaves * kStgItem;
}

// largest row group whose staged activations fit the LDS budget
inline int q6_rows_per_pass(int M, int K) {
  int mc = M;
  while (mc > 1 && q6_lds_bytes(mc, K) > (size_t)kLdsMax) --mc;
  return mc;
}

template <int LAYOUT>
int q6_gemv16_launch(const uint8_t* w, const _Float16* x, uint16_t* out, int M, int N, int K,
                     hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&q6_gemv16_kernel<LAYOUT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
  });
  if (attr != hipSuccess) return (int)attr;
  const int T = (N + 15) / 16;
  const int mc = q6_rows_per_pass(M, K);
  if (q6_lds_bytes(mc, K) > (size_t)kLdsMax) return TLX_E_ARG;
  for (int m0 = 0; m0 < M; m0 += mc) {
    KqArgs a{w, x + (size_t)m0 * K, out + (size_t)m0 * N, std::min(mc, M - m0), N, K, 0};
    const size_t lds = q6_lds_bytes(a.M, K);
    int grid = std::min(T, tlx_cu_count());  // one resident workgroup per CU (VGPR-bound)
    a.tw = (T + grid - 1) / grid;
    grid = (T + a.tw - 1) / a.tw;
    q6_gemv16_kernel<LAYOUT><<<grid, kWaves * TLX_WAVE, lds, st>>>(a);
    const int rc = tlx_launch_status();
    if (rc != TLX_OK) return rc;
  }
  return TLX_OK;
}

int q6_check(const void* w, const void* x, const void* out, int M, int N, int K, int layout) {
  if (M < 1 || M > TLX_MAX_M || N < 1 || K < 256 || (K & 255)) return TLX_E_ARG;
  if (layout != TLX_LAYOUT_RAW && layout != TLX_LAYOUT_PACKED) return TLX_E_ARG;
  // 32-bit byte offsets inside the matrix
  if ((size_t)N * q6_geo(layout).bs * (K >> 8) > 0xFFFFFFFFull) return TLX_E_ARG;
  if (!tlx_aligned(w, 2) || !tlx_aligned(x, 16) || !tlx_aligned(out, 2)) return TLX_E_ALIGN;
  return TLX_OK;
}

int q6_gemv16(const void* w, const uint16_t* x, uint16_t* out, int M, int N, int K, int layout,
              hipStream_t st) {
  return layout == TLX_LAYOUT_RAW
             ? q6_gemv16_launch<TLX_LAYOUT_RAW>((const uint8_t*)w, (const _Float16*)x, out, M, N, K, st)
             : q6_gemv16_launch<TLX_LAYOUT_PACKED>((const uint8_t*)w, (const _Float16*)x, out, M, N,
                                                   K, st);
}

}  // namespace

extern "C" int tlx_q6k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                              int K, int layout, void* stream) {
  const int rc = q6_check(w, x_f16, out_f16, M, N, K, layout);
  TLX_RET_IF(rc != TLX_OK, rc);
  return q6_gemv16(w, x_f16, out_f16, M, N, K, layout, (hipStream_t)stream);
}

extern "C" int tlx_aq6k8(const void* wq, const void* wk, const void* wv, const float* gridf,
                         const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                         uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, int layout,
                         void* stream) {
  // q: Q6_K in the padded 212-B blocks (layout PACKED) or raw 210-B blocks; k and v: IQ3_XXS
  // packed rows, through the IQ3 GEMV (two launches on the same stream).
  int rc = q6_check(wq, xh_f16, qrow_f16, M, Nq, K, layout);
  if (rc == TLX_OK)
    rc = tlx_iq3_kv(wk, wv, gridf, xh_f16, krow_f16, vrow_f16, M, Nk, Nv, K, false, stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  rc = tlx_iq3_kv(wk, wv, gridf, xh_f16, krow_f16, vrow_f16, M, Nk, Nv, K, true, stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  return q6_gemv16(wq, xh_f16, qrow_f16, M, Nq, K, layout, (hipStream_t)stream);
}
