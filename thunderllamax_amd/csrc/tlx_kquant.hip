// K-quant kernels for gfx950 with fp16 activations: decode GEMVs for Q6_K (raw 210-B and padded
// 212-B blocks), Q5_K (176 B) and Q4_K (144 B) with fp16 outputs -- the q-branch of the fused
// attention projections, the Q4_K v rows and the Q5_K / Q6_K heads -- and bit-exact Q4_K / Q5_K
// dequantization.
//
// GEMV design (one kernel per format for every M that fits the LDS budget; larger M runs in
// row groups):
//   * the activation block X[M][K] is staged once per workgroup in LDS (LDS-DMA) with a row
//     stride of 2K+16 bytes, so the 8 lanes of one LDS read phase fall on distinct 16-B slots;
//   * a workgroup owns a contiguous range of 16-row tiles, and its (tile, block) items are
//     split into 8 equal contiguous ranges, one per wave: every wave streams the same number
//     of weight bytes whatever the tile count;
//   * weights are read with quad-coalesced 16-B loads (4 lanes cover 64 contiguous bytes of
//     one row), written to a per-wave LDS staging tile in row order and read back in MFMA
//     fragment order (lane (col, kq) receives row col's bytes for its k-quarter);
//   * Q6_K decode: q = ql nibble | (qh 2 bits) << 4 for 4 weights per dword, fp16 pairs
//     1 + q/1024 by v_perm with 0x3C bytes, minus 33/32 gives (q-32)/1024 exactly, times the
//     int8 group scale gives fp16(sc*(q-32))/1024 with one rounding (the size of the
//     reference's own fp16 weight rounding); d*1024 is applied once per block;
//   * Q4_K / Q5_K decode: w = (d*sc)*q - dmin*m splits into d * (sc*q), with sc*q <= 63*31 an
//     exact fp16 integer (v_perm with 0x64 bytes gives 1024 + q, one packed fma with sc and
//     -1024*sc gives sc*q), and the min term dmin * sum_s m_s * S_s, where S_s is the fp32 sum
//     of the 32 activations of sub-block s (computed once per workgroup): two fp32 MFMAs
//     (16x16x4) per block;
//   * v_mfma_f32_16x16x32_f16 accumulates in fp32; tiles split between waves are combined
//     through LDS in wave order after the main loop, so results do not depend on scheduling.
#include "tlx_common.h"

#include <mutex>

namespace {

enum KFmt { KF_Q6R = 0, KF_Q6P = 1, KF_Q4K = 2, KF_Q5K = 3 };

constexpr int kWaves = 8;
constexpr int kSlot = 64 * 16;          // one wave's 16x16 fp32 partial tile
constexpr int kLdsMax = 160 * 1024;
constexpr int kPrefetch = 2;            // items in flight per wave (even: fragments ping-pong)

struct KGeo {
  int bs;      // block bytes
  int qoff;    // Q6_K: ql/qh bytes (192) start; Q4_K/Q5_K: qs start
  int scoff;   // Q6_K scales
  int doff;    // Q6_K d
  int pieces;  // Q4_K/Q5_K: 16-B pieces per block
  int rs;      // staging bytes per weight row (16 x odd: conflict-free fragment reads)
};
__host__ __device__ constexpr KGeo kgeo(int f) {
  return f == KF_Q6R   ? KGeo{210, 0, 192, 208, 0, 240}
         : f == KF_Q6P ? KGeo{212, 20, 4, 2, 0, 240}
         : f == KF_Q4K ? KGeo{144, 16, 0, 0, 9, 208}
                       : KGeo{176, 48, 0, 0, 11, 208};
}
__host__ __device__ constexpr bool is_q6(int f) { return f == KF_Q6R || f == KF_Q6P; }

struct KqArgs {
  const uint8_t* w;    // N rows x nb blocks
  const _Float16* x;   // [M][K]
  uint16_t* out;       // [M][N] fp16
  int M, N, K;
  int tw;              // tiles per workgroup
};

struct KLd {  // one lane's share of an item as loaded
  u4_t q[3];           // Q6_K: 48 B of ql/qh; Q4_K/Q5_K: pieces c, c+4, c+8 of the block
  uint32_t sc, d;      // Q6_K only: a scale dword and d
};

struct KFrag {  // one lane's share in fragment order
  u4_t lo[2];          // Q6_K: 32 ql bytes; Q4_K/Q5_K: 32 qs bytes
  u4_t hi[2];          // Q6_K: 32 qh bytes; Q5_K: the 32 qh bytes
  u4_t hdr;            // Q6_K: .xy = 8 scales, .z = d; Q4_K/Q5_K: d, dmin, 12 scale bytes
};

// `off` is the block's 32-bit byte offset from the matrix base (scalar base + vector offset)
template <int F>
__device__ __forceinline__ void k_load(KLd& L, const uint8_t* w, uint32_t off, int c) {
  constexpr KGeo G = kgeo(F);
  if constexpr (is_q6(F)) {
#pragma unroll
    for (int j = 0; j < 3; ++j) L.q[j] = tlx_ldu<u4_t>(w + (off + G.qoff + 64 * j + 16 * c));
    L.sc = tlx_ldu<uint32_t>(w + (off + G.scoff + 4 * c));
    L.d = tlx_ldu<uint16_t>(w + (off + G.doff));
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j)  // pieces past the block re-read its last piece (not staged)
      L.q[j] = *reinterpret_cast<const u4_t*>(w + (off + 16 * min(c + 4 * j, G.pieces - 1)));
  }
}

// staging row r.  Q6_K: [ql 128][qh 64][sc 16][d 2][pad]; Q4_K/Q5_K: the block as stored.
template <int F>
__device__ __forceinline__ void k_stage(uint8_t* stg, const KLd& L, int r, int c) {
  constexpr KGeo G = kgeo(F);
  uint8_t* s = stg + r * G.rs;
  if constexpr (is_q6(F)) {
#pragma unroll
    for (int j = 0; j < 3; ++j) *reinterpret_cast<u4_t*>(s + 64 * j + 16 * c) = L.q[j];
    *reinterpret_cast<uint32_t*>(s + 192 + 4 * c) = L.sc;
    if (c == 0) *reinterpret_cast<uint16_t*>(s + 208) = (uint16_t)L.d;
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (c + 4 * j < G.pieces) *reinterpret_cast<u4_t*>(s + 16 * (c + 4 * j)) = L.q[j];
  }
}

// Q6_K: lane (col, kq = 2h + e) owns the elements k = 128h + 32g + l with g in {e, e + 2}:
// ql bytes [64h + 32e, +32), qh bytes [32h, +32), scales sc[8h .. 8h + 8).
// Q4_K / Q5_K: lane (col, kq) owns k = 64kq + 0..63: qs bytes [32kq, +32) (low nibbles are
// sub-block 2kq, high nibbles 2kq+1), all 32 qh bytes (bits 2kq, 2kq+1), the 16-B header.
template <int F>
__device__ __forceinline__ void k_frag(KFrag& R, const uint8_t* stg, int col, int kq) {
  constexpr KGeo G = kgeo(F);
  const uint8_t* f = stg + col * G.rs;
  if constexpr (is_q6(F)) {
    const int h = kq >> 1, e = kq & 1;
    R.lo[0] = *reinterpret_cast<const u4_t*>(f + 64 * h + 32 * e);
    R.lo[1] = *reinterpret_cast<const u4_t*>(f + 64 * h + 32 * e + 16);
    R.hi[0] = *reinterpret_cast<const u4_t*>(f + 128 + 32 * h);
    R.hi[1] = *reinterpret_cast<const u4_t*>(f + 144 + 32 * h);
    const u2_t sc = *reinterpret_cast<const u2_t*>(f + 192 + 8 * h);
    R.hdr = u4_t{sc.x, sc.y, *reinterpret_cast<const uint16_t*>(f + 208), 0u};
  } else {
    R.lo[0] = *reinterpret_cast<const u4_t*>(f + G.qoff + 32 * kq);
    R.lo[1] = *reinterpret_cast<const u4_t*>(f + G.qoff + 32 * kq + 16);
    if constexpr (F == KF_Q5K) {
      R.hi[0] = *reinterpret_cast<const u4_t*>(f + 16);
      R.hi[1] = *reinterpret_cast<const u4_t*>(f + 32);
    }
    R.hdr = *reinterpret_cast<const u4_t*>(f);
  }
}

// fp16 pairs of bytes 0,1 (sel 0x04010400) or 2,3 (sel 0x04030402) of q, high bytes from hb4
__device__ __forceinline__ h2_t k_pair(uint32_t q, uint32_t hb4, uint32_t sel) {
  return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(hb4, q, sel));
}

// Q6_K block: MFMA o = 4*nib + u covers, for lane (col, 2h + e), the 8 elements
// k = 128h + 32(e + 2nib) + 8u + i: ql bytes 8u..8u+7 (nibble nib), qh bytes 8u..8u+7
// (bits 2e + 4nib), scale byte (u >> 1) + 2e + 4nib of the lane's 8.  Returns the block's
// contribution d * sum_k x*w.
__device__ __forceinline__ f4_t q6_block(const KFrag& F, const h8_t* A, int kq) {
  const int e = kq & 1;
  f4_t D = {0.f, 0.f, 0.f, 0.f};
  const h2_t off = {(_Float16)-1.03125f, (_Float16)-1.03125f};
#pragma unroll
  for (int nib = 0; nib < 2; ++nib) {
    const int sh = 2 * e + 4 * nib;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sb = (u >> 1) + 2 * e + 4 * nib;
      const uint32_t sw = sb < 4 ? F.hdr.x : F.hdr.y;
      const _Float16 s = (_Float16)(float)(int8_t)(uint8_t)(sw >> (8 * (sb & 3)));
      const h2_t sp = {s, s};
      const u4_t& L4 = F.lo[u >> 1];
      const u4_t& H4 = F.hi[u >> 1];
      const uint32_t l0 = (u & 1) ? L4.z : L4.x, l1 = (u & 1) ? L4.w : L4.y;
      const uint32_t g0 = (u & 1) ? H4.z : H4.x, g1 = (u & 1) ? H4.w : H4.y;
      const uint32_t q0 = ((l0 >> (4 * nib)) & 0x0F0F0F0Fu) | (((g0 >> sh) & 0x03030303u) << 4);
      const uint32_t q1 = ((l1 >> (4 * nib)) & 0x0F0F0F0Fu) | (((g1 >> sh) & 0x03030303u) << 4);
      const h2_t p0 = (k_pair(q0, 0x3C3C3C3Cu, 0x04010400u) + off) * sp;
      const h2_t p1 = (k_pair(q0, 0x3C3C3C3Cu, 0x04030402u) + off) * sp;
      const h2_t p2 = (k_pair(q1, 0x3C3C3C3Cu, 0x04010400u) + off) * sp;
      const h2_t p3 = (k_pair(q1, 0x3C3C3C3Cu, 0x04030402u) + off) * sp;
      const h8_t B = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
      D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[4 * nib + u], B, D, 0, 0, 0);
    }
  }
  return (tlx_h2f((uint16_t)F.hdr.z) * 1024.0f) * D;
}

// 6-bit scale (sm = 0) or min (sm = 1) of sub-block 4*hi + j from the 12 scale bytes
// (header dwords 1..3): ggml get_scale_min_k4.
__device__ __forceinline__ uint32_t k4_field(const u4_t& hdr, int hi, int j, int sm) {
  const uint32_t a = ((sm ? hdr.z : hdr.y) >> (8 * j)) & 0xFFu;  // q[j] (scale) or q[j+4] (min)
  const uint32_t c = (hdr.w >> (8 * j)) & 0xFFu;                  // q[j+8]
  return hi == 0 ? (a & 63u) : (((sm ? c >> 4 : c) & 0xFu) | ((a >> 6) << 4));
}

// Q4_K / Q5_K block.  MFMA o = 4*nib + u covers, for lane (col, kq), the 8 elements
// k = 64kq + 32nib + 8u + i of sub-block 2kq + nib: qs bytes 8u..8u+7 of the lane's 32
// (nibble nib), qh bytes 8u..8u+7 (bit 2kq + nib).  The min term uses two fp32 MFMAs whose
// k index is the sub-block 4i + kq; S[4i] is the lane row's fp32 sum over that sub-block.
template <int F>
__device__ __forceinline__ f4_t k4_block(const KFrag& R, const h8_t* A, const float* S, int kq) {
  f4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nib = 0; nib < 2; ++nib) {
    const int s = 2 * kq + nib;
    const _Float16 sc = (_Float16)(float)k4_field(R.hdr, s >> 2, s & 3, 0);
    const h2_t sp = {sc, sc};
    const h2_t mp = {(_Float16)(-1024.0f) * sc, (_Float16)(-1024.0f) * sc};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u4_t& L4 = R.lo[u >> 1];
      const uint32_t l0 = (u & 1) ? L4.z : L4.x, l1 = (u & 1) ? L4.w : L4.y;
      uint32_t q0 = (l0 >> (4 * nib)) & 0x0F0F0F0Fu, q1 = (l1 >> (4 * nib)) & 0x0F0F0F0Fu;
      if constexpr (F == KF_Q5K) {
        const u4_t& H4 = R.hi[u >> 1];
        const uint32_t g0 = (u & 1) ? H4.z : H4.x, g1 = (u & 1) ? H4.w : H4.y;
        q0 |= ((g0 >> s) & 0x01010101u) << 4;
        q1 |= ((g1 >> s) & 0x01010101u) << 4;
      }
      // (1024 + q) * sc - 1024 * sc = sc * q, exact: one rounding of an exact integer
      const h2_t p0 = __builtin_elementwise_fma(k_pair(q0, 0x64646464u, 0x04010400u), sp, mp);
      const h2_t p1 = __builtin_elementwise_fma(k_pair(q0, 0x64646464u, 0x04030402u), sp, mp);
      const h2_t p2 = __builtin_elementwise_fma(k_pair(q1, 0x64646464u, 0x04010400u), sp, mp);
      const h2_t p3 = __builtin_elementwise_fma(k_pair(q1, 0x64646464u, 0x04030402u), sp, mp);
      const h8_t B = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
      D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[4 * nib + u], B, D, 0, 0, 0);
    }
  }
  const float d = tlx_h2f((uint16_t)(R.hdr.x & 0xFFFFu));
  const float dmin = tlx_h2f((uint16_t)(R.hdr.x >> 16));
  f4_t Dm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 2; ++i)
    Dm = __builtin_amdgcn_mfma_f32_16x16x4f32(S[4 * i], dmin * (float)k4_field(R.hdr, i, kq, 1),
                                              Dm, 0, 0, 0);
  return d * D - Dm;
}

__device__ __forceinline__ int kq_range(int I, int w) { return (int)((int64_t)I * w / kWaves); }

__host__ __device__ inline size_t k_x_bytes(int M, int K) {
  const size_t xb = (size_t)M * (K + 8) * 2;
  return xb > (size_t)kWaves * 2 * kSlot ? xb : (size_t)kWaves * 2 * kSlot;
}

// LDS: [staged X (the partial-tile slots after the main loop)][Q4_K/Q5_K: S[M][K/32] fp32]
//      [8 staging tiles]
__host__ __device__ inline size_t k_lds_bytes(int F, int M, int K) {
  return k_x_bytes(M, K) + (is_q6(F) ? 0 : (size_t)M * (K / 32) * 4) +
         (size_t)kWaves * 16 * kgeo(F).rs;
}

template <int F>
__global__ __launch_bounds__(kWaves * TLX_WAVE) void kq_gemv16_kernel(const KqArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr KGeo G = kgeo(F);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int M = a.M, N = a.N, K = a.K, nb = K >> 8, ng = K >> 5;
  const int XS = K + 8;  // halves per staged activation row
  const size_t xbytes = k_x_bytes(M, K);
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  float* ssum = reinterpret_cast<float*>(lds + xbytes);
  uint8_t* stg = lds + xbytes + (is_q6(F) ? 0 : (size_t)M * ng * 4) + wave * 16 * G.rs;

  const int T = (N + 15) >> 4;
  const int t0 = (int)blockIdx.x * a.tw;
  const int I = min(a.tw, T - t0) * nb;
  const int lo = kq_range(I, wave), hi = kq_range(I, wave + 1);

  const int r = lane >> 2, c = lane & 3;      // load role: row r, 16-B piece c of each 64 B
  const int col = lane & 15, kq = lane >> 4;  // MFMA role
  const uint32_t rowb = (uint32_t)G.bs * nb;
  // Every load, staging write and fragment read below is unconditional (item indices are
  // clamped to the wave's last item), so the loop body is straight-line and the compiler's
  // wait counts stay exact.  The load cursor (the next item to load, as a block offset that
  // steps by one block and jumps to the next tile's rows) stops at the last item, whose loads
  // then repeat.
  const int last = hi - 1;
  uint32_t loff = 0;
  int lb = 0, lt = 0, lleft = 0;
  auto tile_off = [&](int t) {  // tail tile: clamp the loads, mask the stores
    return (uint32_t)min(16 * t + r, N - 1) * rowb;
  };
  auto load_next = [&](KLd& L) {
    k_load<F>(L, a.w, loff, c);
    if (lleft > 0) {
      --lleft;
      if (++lb == nb) {
        lb = 0;
        loff = tile_off(++lt);
      } else {
        loff += G.bs;
      }
    }
  };
  KLd g[kPrefetch];  // ring: item i sits in g[(i - lo) % kPrefetch] until it is staged
  if (lo < hi) {
    lt = t0 + lo / nb;
    lb = lo - (lo / nb) * nb;
    lleft = last - lo;
    loff = tile_off(lt) + (uint32_t)lb * G.bs;
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) load_next(g[p]);
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
  if constexpr (!is_q6(F)) {
    // fp32 sums of the 32 activations of every sub-block, summed in k order
    for (int v = threadIdx.x; v < M * ng; v += kWaves * TLX_WAVE) {
      const int m = v / ng, gi = v - m * ng;
      const _Float16* p = xs + m * XS + 32 * gi;
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const h8_t h = *reinterpret_cast<const h8_t*>(p + 8 * q);
#pragma unroll
        for (int z = 0; z < 8; ++z) sum += (float)h[z];
      }
      ssum[v] = sum;
    }
    __syncthreads();
  }

  // activation rows >= M feed output rows that are never stored: read a valid row instead
  const int am = min(col, M - 1);
  const _Float16* xa = xs + am * XS + (is_q6(F) ? 128 * (kq >> 1) + 32 * (kq & 1) : 64 * kq);
  const float* sa = ssum + am * ng + kq;

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
  KFrag R[2];  // item i's fragments in R[(i - lo) & 1]
  if (lo < hi) {
    k_stage<F>(stg, g[0], r, c);
    k_frag<F>(R[0], stg, col, kq);
    load_next(g[0]);
  }
  int seg = lo;
  int tl = lo / nb, b = lo - (lo / nb) * nb;  // compute cursor (tile local to the workgroup)
  for (int i0 = lo; i0 < hi; i0 += kPrefetch) {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const int i = i0 + p;  // i >= hi: padding steps of the last round, computed and discarded
      h8_t A[8];
#pragma unroll
      for (int o = 0; o < 8; ++o)
        A[o] = *reinterpret_cast<const h8_t*>(xa + 256 * b + (is_q6(F) ? 64 : 32) * (o >> 2) +
                                              8 * (o & 3));
      float S[8];
      if constexpr (!is_q6(F)) {
#pragma unroll
        for (int z = 0; z < 8; z += 4) S[z] = sa[8 * b + z];
      }
      // item i+1 goes through the single staging tile after item i's fragment reads were
      // issued (LDS executes a wave's instructions in order); its ring slot is then refilled
      k_stage<F>(stg, g[(p + 1) % kPrefetch], r, c);
      k_frag<F>(R[(p + 1) & 1], stg, col, kq);
      f4_t D;
      if constexpr (is_q6(F)) D = q6_block(R[p & 1], A, kq);
      else D = k4_block<F>(R[p & 1], A, S, kq);
      load_next(g[(p + 1) % kPrefetch]);
      if (i < hi) {
        acc += D;
        if (b == nb - 1 || i == hi - 1) {  // end of a tile segment
          if (seg - tl * nb == 0 && b == nb - 1) store(acc, t0 + tl);
          else if (tl == lo / nb) accFirst = acc;
          else accLast = acc;
          acc = f4_t{0.f, 0.f, 0.f, 0.f};
          seg = i + 1;
        }
        if (i + 1 < hi && ++b == nb) {
          b = 0;
          ++tl;
        }
      }
    }
  }

  // ---- tiles shared by consecutive waves: partial sums through LDS, combined in wave order
  __syncthreads();  // every wave is done with the staged activations and its staging tile
  f4_t* slots = reinterpret_cast<f4_t*>(lds);
  const int tf = lo / nb, tlast = (hi - 1) / nb;
  const bool firstPartial = lo < hi && !(lo % nb == 0 && (tf + 1) * nb <= hi);
  const bool lastPartial = lo < hi && tlast != tf && hi % nb != 0;
  if (firstPartial) slots[(wave * 2 + 0) * 64 + lane] = accFirst;
  if (lastPartial) slots[(wave * 2 + 1) * 64 + lane] = accLast;
  __syncthreads();
  // the wave holding a tile's last item combines it when the tile began in an earlier wave
  if (lo < hi && lo % nb != 0 && (tf + 1) * nb <= hi) {
    f4_t sum = {0.f, 0.f, 0.f, 0.f};
    for (int v = 0; v < wave; ++v) {
      const int lov = kq_range(I, v), hiv = kq_range(I, v + 1);
      if (lov >= hiv || hiv <= tf * nb) continue;
      sum += slots[(v * 2 + (lov / nb == tf ? 0 : 1)) * 64 + lane];
    }
    sum += accFirst;
    store(sum, t0 + tf);
  }
}

// largest row group whose staged activations fit the LDS budget
inline int k_rows_per_pass(int F, int M, int K) {
  int mc = M;
  while (mc > 1 && k_lds_bytes(F, mc, K) > (size_t)kLdsMax) --mc;
  return mc;
}

// One-time kernel set-up: the dynamic LDS limit above 64 KB (done once per process, by the first
// call or by tlx_attach_workspace, so that calls made under stream capture do no set-up).
template <int F>
hipError_t kq_attr_once() {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&kq_gemv16_kernel<F>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
  });
  return attr;
}

template <int F>
int kq_gemv16_launch(const uint8_t* w, const _Float16* x, uint16_t* out, int M, int N, int K,
                     hipStream_t st) {
  const hipError_t attr = kq_attr_once<F>();
  if (attr != hipSuccess) return (int)attr;
  const int T = (N + 15) / 16;
  const int mc = k_rows_per_pass(F, M, K);
  if (k_lds_bytes(F, mc, K) > (size_t)kLdsMax) return TLX_E_ARG;
  for (int m0 = 0; m0 < M; m0 += mc) {
    KqArgs a{w, x + (size_t)m0 * K, out + (size_t)m0 * N, std::min(mc, M - m0), N, K, 0};
    int grid = std::min(T, tlx_cu_count());  // one resident workgroup per CU (VGPR-bound)
    a.tw = (T + grid - 1) / grid;
    grid = (T + a.tw - 1) / a.tw;
    kq_gemv16_kernel<F><<<grid, kWaves * TLX_WAVE, k_lds_bytes(F, a.M, K), st>>>(a);
    const int rc = tlx_launch_status();
    if (rc != TLX_OK) return rc;
  }
  return TLX_OK;
}

}  // namespace

int tlx_kq_setup() {
  const hipError_t e[4] = {kq_attr_once<0>(), kq_attr_once<1>(), kq_attr_once<2>(), kq_attr_once<3>()};
  for (hipError_t x : e)
    if (x != hipSuccess) return (int)x;
  return TLX_OK;
}

namespace {

int kq_check(int F, const void* w, const void* x, const void* out, int M, int N, int K) {
  if (M < 1 || M > TLX_MAX_M || N < 1 || K < 256 || (K & 255)) return TLX_E_ARG;
  // 32-bit byte offsets inside the matrix
  if ((size_t)N * kgeo(F).bs * (K >> 8) > 0xFFFFFFFFull) return TLX_E_ARG;
  // Q4_K / Q5_K blocks are read as whole 16-B pieces
  if (!tlx_aligned(w, is_q6(F) ? 2 : 16) || !tlx_aligned(x, 16) || !tlx_aligned(out, 2))
    return TLX_E_ALIGN;
  return TLX_OK;
}

int kq_gemv16(int F, const void* w, const uint16_t* x, uint16_t* out, int M, int N, int K,
              hipStream_t st) {
  const uint8_t* wb = (const uint8_t*)w;
  const _Float16* xh = (const _Float16*)x;
  switch (F) {
    case KF_Q6R: return kq_gemv16_launch<KF_Q6R>(wb, xh, out, M, N, K, st);
    case KF_Q6P: return kq_gemv16_launch<KF_Q6P>(wb, xh, out, M, N, K, st);
    case KF_Q4K: return kq_gemv16_launch<KF_Q4K>(wb, xh, out, M, N, K, st);
    default: return kq_gemv16_launch<KF_Q5K>(wb, xh, out, M, N, K, st);
  }
}

int q6_fmt(int layout) {
  return layout == TLX_LAYOUT_RAW ? KF_Q6R : layout == TLX_LAYOUT_PACKED ? KF_Q6P : -1;
}

// ------------------------------------------------------------------ Q4_K / Q5_K dequantization
// One thread per (block, lane l in 0..31): the 8 outputs k = 8l + j, in the order and rounding
// of ggml's dequantize_row_q{4,5}_K: (d*sc)*q - dmin*m, no fused multiply-add.
template <bool FIVE>
__global__ __launch_bounds__(256) void k4_dequant_kernel(const uint8_t* __restrict__ w,
                                                         void* __restrict__ out, int64_t nblk,
                                                         int out_f16) {
#pragma clang fp contract(off)
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nblk * 32) return;
  const int64_t bi = t >> 5;
  const int l = (int)(t & 31);
  const uint8_t* blk = w + bi * (FIVE ? 176 : 144);
  const float d = tlx_h2f(tlx_ldu<uint16_t>(blk));
  const float dmin = tlx_h2f(tlx_ldu<uint16_t>(blk + 2));
  const int s = l >> 2;  // sub-block
  const uint8_t* q = blk + 4;
  uint32_t sc, mn;
  if (s < 4) {
    sc = q[s] & 63;
    mn = q[s + 4] & 63;
  } else {
    sc = (q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4);
    mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
  }
  const float d1 = d * (float)sc, m1 = dmin * (float)mn;
  const uint8_t* qs = blk + (FIVE ? 48 : 16) + 32 * (l >> 3) + 8 * (l & 3);
  const int nsh = 4 * ((l >> 2) & 1);
  const int64_t k0 = bi * 256 + 8 * l;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int qv = (qs[j] >> nsh) & 0xF;
    if constexpr (FIVE) qv += ((blk[16 + 8 * (l & 3) + j] >> s) & 1) << 4;
    const float v = d1 * (float)qv - m1;
    if (out_f16)
      reinterpret_cast<uint16_t*>(out)[k0 + j] = tlx_f2h_bits(v);
    else
      reinterpret_cast<float*>(out)[k0 + j] = v;
  }
}

template <bool FIVE>
int k4_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16, void* stream) {
  TLX_RET_IF(rows < 1 || kdim < 256 || (kdim & 255), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(w, 2) || !tlx_aligned(out, 4), TLX_E_ALIGN);
  const int64_t nblk = rows * (kdim >> 8);
  const int64_t grid = (nblk * 32 + 255) / 256;
  TLX_RET_IF(grid > 0x7fffffff, TLX_E_ARG);
  k4_dequant_kernel<FIVE><<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>((const uint8_t*)w, out,
                                                                          nblk, out_f16);
  return tlx_launch_status();
}

}  // namespace

int tlx_kq_gemv(int fmt, const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                int K, bool launch, void* stream) {
  TLX_RET_IF(fmt < KF_Q6R || fmt > KF_Q5K, TLX_E_ARG);
  const int rc = kq_check(fmt, w, x_f16, out_f16, M, N, K);
  TLX_RET_IF(rc != TLX_OK || !launch, rc);
  return kq_gemv16(fmt, w, x_f16, out_f16, M, N, K, (hipStream_t)stream);
}

extern "C" int tlx_q6k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                              int K, int layout, void* stream) {
  const int f = q6_fmt(layout);
  TLX_RET_IF(f < 0, TLX_E_ARG);
  const int rc = kq_check(f, w, x_f16, out_f16, M, N, K);
  TLX_RET_IF(rc != TLX_OK, rc);
  return kq_gemv16(f, w, x_f16, out_f16, M, N, K, (hipStream_t)stream);
}

extern "C" int tlx_q4k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                              int K, void* stream) {
  const int rc = kq_check(KF_Q4K, w, x_f16, out_f16, M, N, K);
  TLX_RET_IF(rc != TLX_OK, rc);
  return kq_gemv16(KF_Q4K, w, x_f16, out_f16, M, N, K, (hipStream_t)stream);
}

extern "C" int tlx_q5k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N,
                              int K, void* stream) {
  const int rc = kq_check(KF_Q5K, w, x_f16, out_f16, M, N, K);
  TLX_RET_IF(rc != TLX_OK, rc);
  return kq_gemv16(KF_Q5K, w, x_f16, out_f16, M, N, K, (hipStream_t)stream);
}

extern "C" int tlx_head8(const void* wq5, const uint16_t* xh_f16, uint16_t* logits_f16, int M,
                         int vocab, int K, void* stream) {
  return tlx_q5k_gemv16(wq5, xh_f16, logits_f16, M, vocab, K, stream);
}

extern "C" int tlx_q4k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16,
                               void* stream) {
  return k4_dequant<false>(w, out, rows, kdim, out_f16, stream);
}

extern "C" int tlx_q5k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16,
                               void* stream) {
  return k4_dequant<true>(w, out, rows, kdim, out_f16, stream);
}
