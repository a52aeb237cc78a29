/*
 * tlx.h -- C ABI of libtlx_hip.so, the gfx950 (MI355X) quantized-weight matmul library.
 *
 * Every entry point:
 *   - takes device pointers and plain sizes (no HIP or torch types; `stream` is a
 *     hipStream_t passed as void*, NULL = the default stream);
 *   - keeps the reference kernel's positional argument order, then appends the sizes the
 *     reference bakes into kernel names / #defines (M, N, K) and a layout flag;
 *   - is asynchronous on `stream` and never aborts;
 *   - allocates nothing, ever.  Scratch device memory is the caller's: query the sizes with
 *     tlx_workspace_size and attach buffers per device with tlx_attach_workspace (the host owns
 *     every buffer, as the reference's boot-time Bufs: engine/engine0.py:85-95).  The GEMV
 *     workspace is required by the IQ3_XXS decode GEMVs over TLX_LAYOUT_TILED records (ffn8,
 *     ffn8_hh, down8, iq3_gemv, iq3_gemv_multi and the IQ3_XXS segments of the attention
 *     projections, at every M: shared partial tiles and arrival counters; TLX_E_NOWS without
 *     one) and used by the packed-row forms at M >= 6 (the tile-ordered activation copy; without
 *     a workspace they read the activations directly).  The GEMM workspace lets the prefill
 *     GEMMs (tlx_pfg3_*) split the last partial round of tiles; without one they run whole tiles.
 *     Calls that use a workspace must not overlap in time on one device (order them on one
 *     stream); attach outside stream capture, after which every call is capture-safe;
 *   - returns TLX_OK, a negative TLX_E_* code for a rejected argument (nothing launched),
 *     or a positive hipError_t from the launch.
 *
 * Activations and outputs named *_f16 hold IEEE binary16 bit patterns (uint16_t).
 */
#ifndef TLX_H
#define TLX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TLX_OK 0
#define TLX_E_ARG (-1)     /* size / M / layout out of range */
#define TLX_E_ALIGN (-2)   /* a pointer or row stride is not aligned as the layout needs */
#define TLX_E_NODEV (-3)   /* no usable gfx950 device */
#define TLX_E_NOMEM (-4)   /* reserved (the library allocates no device memory) */
#define TLX_E_TRUNC (-5)   /* tlx_gguf_parse: the image ends inside the header; pass more bytes */
#define TLX_E_NOWS (-6)    /* the call needs the GEMV workspace and none is attached on this device */

/* Weight layouts (row-major over output rows). */
#define TLX_LAYOUT_RAW 0     /* GGUF blocks as stored in the file */
#define TLX_LAYOUT_PACKED 1  /* IQ3_XXS: pack_w1c regions [qs 64NB][sw 32NB][d 2NB];
                                Q6_K: pack_w1c 212-B blocks [pad2][d2][sc16][lo128][qh64] */
#define TLX_LAYOUT_PACK7 2   /* IQ3_XXS packed7 (engine/pack_w7.py:7-21): [N/8 groups][K/128
                                chunks][32 units r*4+c][16 B: q u16 x4, sw u32, d u16, pad] */
#define TLX_LAYOUT_TILED 3   /* IQ3_XXS tile-major streaming layout of this library (no reference
                                counterpart; built by tlx_pack_iq3_tiled): [ceil(N/16) tiles]
                                [K/256 blocks] 1632-B records (tlx_iq3_tiled_bytes gives the size):
                                [0,1024) slot L = 16*kq + r, 16 B: bits 0..127 of its index stream;
                                [1024,1536) slot L, 8 B: bits 128..191; [1536,1600) row r, u32: the
                                8 sub-block scale nibbles; [1600,1632) row r, u16: d.  The stream of
                                slot (kq, r) holds weights 64kq..64kq+63 of row r as 16 12-bit table
                                indices (sign nibble with the parity bit folded in, grid byte);
                                rows >= N are zero */

#define TLX_MAX_M 16         /* decode GEMVs accept 1..16 activation rows */

int tlx_version(void);
const char* tlx_strerror(int code);

/* ------------------------------------------------------------------ workspaces
 * No reference counterpart (the reference's GEMVs need no scratch; its host allocates every
 * buffer once at boot: engine/engine0.py:85-95).  tlx_workspace_size reports the bytes of the
 * GEMV workspace (a few MB) and of the prefill GEMM's split workspace (128 MB; smaller works,
 * with fewer split tiles).  tlx_attach_workspace binds caller-owned device buffers (256-B
 * aligned; either may be NULL) to the current device, replacing any earlier ones, zeroes the
 * GEMV workspace's counters on `stream` with a kernel, and does the library's one-time set-up
 * (kernel attributes), so that every later call may be made under stream capture.  The buffers
 * must outlive every call that uses them. */
int tlx_workspace_size(uint64_t* gemv_bytes, uint64_t* gemm_bytes);
int tlx_attach_workspace(void* gemv_ws, uint64_t gemv_bytes, void* gemm_ws, uint64_t gemm_bytes,
                         void* stream);

/* ------------------------------------------------------------------ dequantization
 * Oracle-parity kernels: decode `rows` x `kdim` weights.  out_f16 = 0 writes float32 (the
 * exact GGUF value), 1 writes fp16 bits (the value the reference's GEMVs consume).
 * No reference counterpart (the reference dequantizes on the CPU in numpy:
 * engine/pack_w4.py:39-68, engine/mm/MM_P2_ports.py:21-45,
 * engine/mm/MM_P0_d2_repack.py:78-93).
 */
int tlx_iq3xxs_dequant(const void* w, const float* gridf, void* out, int64_t rows, int64_t kdim,
                       int layout, int out_f16, void* stream);
int tlx_q6k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int layout, int out_f16,
                    void* stream);
/* Q4_K / Q5_K dequantization, bit-exact with ggml's dequantize_row_q4_K / q5_K (the order the
 * reference's row bodies use: engine/aq3k8.cu:44-53, engine/head8.cu:70-89):
 * y = (d*sc)*q - dmin*m in fp32.  out: float32 or (out_f16 != 0) fp16 [rows][kdim]. */
int tlx_q4k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16, void* stream);
int tlx_q5k_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16, void* stream);
int tlx_iq4xs_dequant(const void* w, const float* iq4nl, float* out, int64_t rows, int64_t kdim,
                      void* stream);

/* ------------------------------------------------------------------ decode / spec-verify GEMVs */

/* Fused IQ3_XXS FFN gate+up GEMV + SwiGLU:
 *   gact[m][n] = silu16(half(Wg[n]·x[m])) * half(Wu[n]·x[m])
 * Replaces ffn8 / ffn8v{3..11} (engine/ffn8.cu:134-185, engine/ffn8v11.cu:88-133):
 * ffn8(wg, wu, gridf, hhx, gact).  wg, wu: N rows x 98*(K/256) B (layout PACKED rows,
 * RAW blocks, or TILED records), or the prefill GEMM's PACK7 units (N % 8 == 0, 16-B aligned):
 * then it replaces the r7 twins ffn8r7 / ffn8v{3,8,11}r7 that read the packed7 plane
 * (engine/ffn8v11r7.cu:4-16,261; engine/trunk_w1c.py:20-25), bit for bit the packed-row results;
 * gridf: float[1024]; hhx_f16: [M][K]; gact_f16: [M][N]. */
int tlx_ffn8(const void* wg, const void* wu, const float* gridf, const uint16_t* hhx_f16,
             uint16_t* gact_f16, int M, int N, int K, int layout, void* stream);

/* IQ3_XXS down GEMV + residual:  y[m][n] = hh[m][n] + float(half(Wd[n]·gact[m]))
 * Replaces down8 / down8nw32_{3..11} (engine/down8.cu:134-144,
 * engine/down8nw32_11.cu:88-125): down8(wd, gridf, gact, hh, y); with TLX_LAYOUT_PACK7 the r7
 * twins down8r7 / down8nw32v{3,8,11}r7 (engine/down8nw32v11r7.cu:261).  Layouts as tlx_ffn8. */
int tlx_down8(const void* wd, const float* gridf, const uint16_t* gact_f16, const float* hh,
              float* y, int M, int N, int K, int layout, void* stream);

/* Plain IQ3_XXS GEMV with fp16 output: out[m][n] = half(W[n]·x[m]).  The per-segment body
 * of the fused attention / GDN projections (IQ3ROWP, engine/aq3k8.cu:99-131).  Layouts as
 * tlx_ffn8 (PACKED, RAW, PACK7 or TILED). */
int tlx_iq3_gemv(const void* w, const float* gridf, const uint16_t* x_f16, uint16_t* out_f16,
                 int M, int N, int K, int layout, void* stream);

/* Up to four IQ3_XXS matrices that share the activations, one launch: out[s][m][r] =
 * half(W_s[r]·x[m]), W_s of n[s] rows (w, out, n: host arrays of nseg entries; layout PACKED rows,
 * RAW blocks or TILED records, the same for all).  With GGUF IQ3_XXS tensors this replaces the
 * GDN block's separate projection launches k1_q5 / k1_iq3 / k1_ab
 * (engine/gdn_block.cu:44-148: qkv, gate, alpha, beta all read the same normed x). */
int tlx_iq3_gemv_multi(const void* const* w, uint16_t* const* out, const int* n, int nseg,
                       const float* gridf, const uint16_t* x_f16, int M, int K, int layout, void* stream);

/* Fused attention q/k/v projections (one entry per reference kernel; one launch per quant
 * format on `stream`; all arguments are validated before any launch):
 *   tlx_aq3k8: q, k (and v) IQ3_XXS in `layout` (PACKED rows, RAW blocks or TILED records); v is IQ3_XXS
 *     (the benchmark's dense configuration) unless `layout` has TLX_V_Q4K, then GGUF Q4_K (the reference's
 *     wv4).  Replaces aq3k8 / aq3k8v{4..11} (engine/aq3k8.cu:134-145, engine/aq3k8v11.cu:88-180):
 *     aq3k8(wq, wk, wv4, gridf, xh, qrow, krow, vrow).
 *   tlx_aq6k8: q Q6_K (layout PACKED = padded 212-B blocks, RAW = 210-B), k (and v) IQ3_XXS
 *     packed rows, v Q4_K with TLX_V_Q4K.  Replaces aq6k8 (engine/aq6k8.cu:134-173).
 *   tlx_a_qkv_iq3: q, k IQ3_XXS GGUF blocks, v Q4_K.  Replaces a_qkv_iq3
 *     (engine/a_qkv_iq3.cu:88-127).
 *   tlx_a_qkv_q6: q Q6_K 210-B blocks, k IQ3_XXS GGUF blocks, v Q4_K.  Replaces a_qkv_q6
 *     (engine/a_qkv_q6.cu:88-125).
 * xh_f16: [M][K]; qrow/krow/vrow: fp16 [M][Nq|Nk|Nv]. */
#define TLX_V_Q4K 0x100  /* or-ed into `layout`: v rows are GGUF Q4_K */
/* Or-ed into the `layout` of tlx_ffn8 / tlx_iq3_gemv (TLX_LAYOUT_TILED only): the fp16 output is
 * written in the tile-ordered activation form [N/8][16][8] (N * 32 bytes; slot r of column group
 * n/8 holds row r, rows M..15 repeat row M-1) instead of [M][N] -- the form in which the next
 * IQ3_XXS GEMV reads its activations without a copy launch.  No reference counterpart (the
 * reference's GEMVs take row-major activations); the values are those of the row-major output. */
#define TLX_OUT_TILEORD 0x200
/* Or-ed into the `layout` of tlx_ffn8 / tlx_down8 / tlx_iq3_gemv: the activations are already in
 * the tile-ordered form [K/8][16][8] (e.g. written by a TLX_OUT_TILEORD call); results are bit
 * for bit those of the row-major activations. */
#define TLX_IN_TILEORD 0x400
int tlx_aq3k8(const void* wq, const void* wk, const void* wv, const float* gridf,
              const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16, uint16_t* vrow_f16,
              int M, int Nq, int Nk, int Nv, int K, int layout, void* stream);
int tlx_aq6k8(const void* wq, const void* wk, const void* wv, const float* gridf,
              const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16, uint16_t* vrow_f16,
              int M, int Nq, int Nk, int Nv, int K, int layout, void* stream);
int tlx_a_qkv_iq3(const void* wq, const void* wk, const void* wv4, const float* gridf,
                  const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                  uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, void* stream);
int tlx_a_qkv_q6(const void* wq, const void* wk, const void* wv4, const float* gridf,
                 const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                 uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, void* stream);

/* Q6_K GEMV, fp32 activations and outputs: y[n] = sum_k ((d*sc)*(q-32))[n][k] * x[k].
 * The contract of h6k2048 (engine/mm/MM_P34_h6k2048.cu:8-52): h6k2048(w, x, y, rows),
 * generalised to any K (multiple of 256, at most 15360: x is staged in 64 KB of LDS) and to the
 * raw 210-B / padded 212-B layouts. */
int tlx_q6k_gemv(const void* w, const float* x, float* y, int rows, int K, int layout,
                 void* stream);

/* Q6_K GEMV with fp16 activations and fp16 outputs: out[m][n] = half(sum_k W[n][k]*x[m][k]),
 * W = (d*sc)*(q-32) per GGUF Q6_K block; layout TLX_LAYOUT_RAW (210-B blocks) or
 * TLX_LAYOUT_PACKED (the padded 212-B blocks [pad2][d2][sc16][ql128][qh64] of
 * engine/pack_w1c.py:33-45).  The q-branch body of aq6k8 (engine/aq6k8.cu:141-173) and
 * a_qkv_q6 (engine/a_qkv_q6.cu:95-124), and the Q6_K lm_head.  M in 1..16; M rows whose
 * activations do not fit the LDS budget run as consecutive row groups. */
int tlx_q6k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N, int K,
                   int layout, void* stream);

/* Q4_K / Q5_K GEMV with fp16 activations and fp16 outputs: out[m][n] = half(sum_k W[n][k]*x[m][k])
 * with W = (d*sc)*q - dmin*m per GGUF block (144 B / 176 B raw, 16-B aligned rows).  The Q4_K
 * body is the v-row body of the fused attention projections (KVBODY8, engine/aq3k8.cu:27-61);
 * the Q5_K body is the dense lm_head's Q5ROW (engine/head8.cu:65-96).  M in 1..16. */
int tlx_q4k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N, int K,
                   void* stream);
int tlx_q5k_gemv16(const void* w, const uint16_t* x_f16, uint16_t* out_f16, int M, int N, int K,
                   void* stream);

/* Dense lm_head, Q5_K: logits[m][v] = half(W[v]·xh[m]).
 * Replaces head8 / head8v{M} (engine/head8.cu:134-141, engine/head8v11.cu:88-121):
 * head8(wq5, xh, logits); the vocabulary size and K are explicit. */
int tlx_head8(const void* wq5, const uint16_t* xh_f16, uint16_t* logits_f16, int M, int vocab,
              int K, void* stream);


/* ---- prefill dequant-GEMM (M rows of a prompt chunk, MFMA fp16 x fp16 -> fp32) ----
 * x16 is M x K fp16 row-major; W is N IQ3_XXS rows in the packed7 layout (TLX_LAYOUT_PACK7,
 * the layout the reference's pf_gemm3 REPACK=1 kernels read).  M % 256 == 0, K % 128 == 0,
 * 16-byte aligned buffers.  Each output element is one fp32 MFMA sum over k of
 * x[m][k] * half(W[n][k]); its k order differs from the reference's mma.sync order, so
 * results agree to rounding (relative error <= 1e-3), not bitwise. */

/* FFN gate+up fused with SwiGLU: out16[m][n] = hsilu(half(g)) * half(u), N % 128 == 0.
 * Replaces pf_gemm3 with FFN=1 (engine/pf_gemm3.cu:313-323, epilogue :415-420):
 * kernel(w1, w2, gridf, x16, out16). */
int tlx_pfg3_ffn(const void* wg, const void* wu, const float* gridf, const uint16_t* x16,
                 uint16_t* out16, int M, int N, int K, int layout, void* stream);

/* Residual GEMM (down / o projection): out32[m][n] = res[m][n] + acc, N % 256 == 0.
 * Replaces pf_gemm3 with RES=1 (engine/pf_gemm3.cu:313-323, epilogue :410-414):
 * kernel(w1, gridf, x16, res16, out32). */
int tlx_pfg3_iq3d(const void* w, const float* gridf, const uint16_t* x16, const float* res,
                  float* out32, int M, int N, int K, int layout, void* stream);

/* Plain GEMM with fp16 output: out16[m][n] = half(acc), N % 256 == 0.
 * Replaces pf_gemm3 with FFN=0, RES=0 (engine/pf_gemm3.cu:313-323, epilogue :421-423). */
int tlx_pfg3_iq3o(const void* w, const float* gridf, const uint16_t* x16, uint16_t* out16,
                  int M, int N, int K, int layout, void* stream);

/* Merged multi-segment prefill GEMM: up to three weight matrices of different formats that share
 * the activations, one launch, plain fp16 epilogue: out_s[m][r] = half(sum_k x16[m][k] * half(W_s[r][k])),
 * half(W) the reference's fp16 operand (IQ3_XXS fp16(db*g); Q4_K / Q5_K fp16((d*sc)*q - dmin*m);
 * Q6_K fp16((d*sc)*(q-32)), each computed in fp32 and rounded once).  Replaces pf_gemm3m
 * (engine/pf_gemm3m.cu:1-16,229; its builds engine/build_p7b.py:58-77: attention q/k/v with an
 * IQ3_XXS or Q6_K q, IQ3_XXS k and Q4_K v; GDN qkv Q5_K with the IQ3_XXS gate):
 * kernel(wA, wB[, wC], gridf, x16, outA, outB[, outC]) as arrays of nseg entries.  Per segment
 * (w, out, n rows, type, layout): type a ggml type code, with its layout
 *   TLX_TYPE_IQ3_XXS + TLX_LAYOUT_PACK7 (the packed7 units the IQ3_XXS GEMMs read),
 *   TLX_TYPE_Q4_K / TLX_TYPE_Q5_K + TLX_LAYOUT_RAW (GGUF 144-B / 176-B blocks),
 *   TLX_TYPE_Q6_K + TLX_LAYOUT_PACKED (the padded 212-B blocks of engine/pack_w1c.py:33-45);
 * n % 256 == 0, M % 256 == 0, K % 256 == 0, 16-byte aligned buffers.  out_s is fp16 [M][n_s]. */
#define TLX_TYPE_Q4_K 12
#define TLX_TYPE_Q5_K 13
#define TLX_TYPE_Q6_K 14
#define TLX_TYPE_IQ3_XXS 18
int tlx_pfg3m(const void* const* w, uint16_t* const* out, const int* n, const int* type, const int* layout,
              int nseg, const float* gridf, const uint16_t* x16, int M, int K, void* stream);

/* ---- int8-activation (W4A8) prefill branch.
 * Activation quantizer, replaces pfk_q8 (engine/pfk_q8.cu:25-59, kernel(x, xq, sx, rs)):
 * per (row, 128-k chunk) s = max(absmax, 1e-6) * (1/127), xq = rint(x / s) clamped to
 * +-127, rs = sum of the chunk's xq.  x16 [M][K] fp16, xq [M][K] int8, sx / rs [M][K/128];
 * K % 128 == 0.  Bit-identical to the reference. */
int tlx_p8_quant(const uint16_t* x16, int8_t* xq, float* sx, int32_t* rs, int M, int K, void* stream);

/* Fused W4A8 gate+up + SwiGLU, replaces p8w4ffn7 (engine/p8_w4ffn7.cu:169-257,
 * kernel(w1u, w2u, lut8, xq, sx, out16)): the packed7 IQ3_XXS weights (TLX_LAYOUT_PACK7)
 * with each grid magnitude replaced by its linearized level lut8[4g + j] (int8[1024]: 1..15)
 * and the sub-block scale d * ((sw >> 28) + 0.5) * 0.5 * 4.0507, times the int8 activations
 * xq * sx of tlx_p8_quant; out16 = silu16(half(g)) * half(u).  M % 128 == 0, N % 64 == 0,
 * K % 256 == 0. */
int tlx_p8w4_ffn(const void* w1u, const void* w2u, const int8_t* lut8, const int8_t* xq, const float* sx,
                 uint16_t* out16, int M, int N, int K, int layout, void* stream);

/* ---- Activation producers either side of the GEMVs (fp32 residual stream, fp16 GEMV input).
 * RMSNorm, replaces k0n{M} / k0_norm (engine/k0n11.cu:88-103, engine/gdn_block.cu:30-40):
 * xh[m] = half((x[m] * r) * nw), r = rsqrt(sum(x[m]^2) / D + 1e-6).  D % 8 == 0. */
int tlx_rms_f16(const float* x, const float* nw, uint16_t* xh, int M, int D, void* stream);
/* Residual add + RMSNorm, replaces hh{M} / k3m_hh (engine/hh11.cu:88-107,
 * engine/gdn_block.cu:258-276): hh = x + float(a) (fp32, exact), hhx = half((hh * r) * nw). */
int tlx_add_rms_f16(const float* x, const uint16_t* a, const float* nw, float* hh, uint16_t* hhx, int M,
                    int D, void* stream);
/* tlx_ffn8 that allocates nothing and needs no attached workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels and results
 * (bit for bit) as tlx_ffn8; the scratch is the library's own fixed device array (about 3 MB per
 * device, held until the process ends), so K <= 65536 (larger K: TLX_E_ARG).  Every call on a
 * device shares that device's scratch: calls that overlap in time on one device race (order them
 * on one stream).  Each call first clears the scratch's counters with a small kernel. */
int tlx_ffn8_noalloc(const void* wg, const void* wu, const float* gridf, const uint16_t* hhx_f16,
                     uint16_t* gact_f16, int M, int N, int K, int layout, void* stream);

/* hh{M} fused with ffn8: tlx_add_rms_f16(x, attn_out, nw2, hh, hhx) then tlx_ffn8(wg, wu, gridf,
 * hhx, gact) with the same results bit for bit; from M = 6 on the producer also writes the
 * GEMV's tile-ordered activation copy, so the call is two launches instead of three.  Same
 * workspace rules as the IQ3_XXS GEMVs.  K is the model dimension D. */
int tlx_ffn8_hh(const void* wg, const void* wu, const float* gridf, const float* x, const uint16_t* attn_out,
                const float* nw2, float* hh, uint16_t* hhx_f16, uint16_t* gact_f16, int M, int N, int K,
                int layout, void* stream);

/* ---- On-disk formats.
 * GGUF v3 tensor table, replaces parse_gguf (engine/engine0.py:25-51) and tnbytes (:53-55):
 * parses the image head[0..len) of a file's start (magic, version, counts, the key/value
 * section skipped, the tensor table).  Fills *n_tensors, *data_start (the end of the tensor
 * table rounded up to 32 bytes, as the reference) and up to max_tensors entries of tensors
 * (tensors may be NULL to count only).  dims are in GGUF order: dims[0] is the row length
 * ("[in, out]").  nbytes is the reference's tnbytes, 0 for a type it does not know.  Host
 * only; TLX_E_TRUNC when the image is too short (read more of the file and call again),
 * TLX_E_ARG for a malformed file or a name longer than 127 bytes. */
#define TLX_GGUF_MAX_DIMS 4
typedef struct tlx_gguf_tensor {
  char name[128];
  int32_t type;       /* ggml type code (18 IQ3_XXS, 14 Q6_K, 13 Q5_K, 12 Q4_K, 23 IQ4_XS, ...) */
  uint32_t n_dims;
  uint64_t dims[TLX_GGUF_MAX_DIMS];
  uint64_t offset;    /* bytes from data_start */
  uint64_t nbytes;
} tlx_gguf_tensor;
int tlx_gguf_parse(const void* head, uint64_t len, uint64_t* data_start, int64_t* n_tensors,
                   tlx_gguf_tensor* tensors, int64_t max_tensors);

/* Repackers (device to device, byte permutations):
 * raw IQ3_XXS rows [N][K/256][98] -> packed rows [qs 64NB][sw 32NB][d 2NB], replaces pack_iq3
 * (engine/pack_w1c.py:20-31); */
int tlx_pack_iq3_rows(const void* raw, void* packed, int N, int K, void* stream);
/* raw Q6_K rows [N][K/256][210] -> padded blocks [pad2][d2][sc16][ql128][qh64], replaces pack_q6
 * (engine/pack_w1c.py:33-45, which fixes K = 5120); */
int tlx_pack_q6_pad(const void* raw, void* padded, int N, int K, void* stream);
/* packed IQ3_XXS rows -> packed7 units [N/8][K/128][32][16 B], replaces pack_tensor
 * (engine/pack_w7.py:40-75); N % 8 == 0. */
int tlx_pack_w7(const void* packed, void* p7, int N, int K, void* stream);
/* IQ3_XXS rows (src_layout TLX_LAYOUT_RAW blocks or TLX_LAYOUT_PACKED rows) -> TLX_LAYOUT_TILED
 * records, ceil(N/16) * (K/256) * 1632 B (= tlx_iq3_tiled_bytes(N, K); 0 for invalid sizes).  No reference counterpart: the decode GEMVs
 * (tlx_ffn8, tlx_ffn8_hh, tlx_down8, tlx_iq3_gemv) read it with every wave load one contiguous
 * run, the streaming form of the layout pack_w1c (engine/pack_w1c.py:20-31) makes for the
 * reference's GEMVs.  The GEMV results are bit-identical to those of the source layout. */
int tlx_pack_iq3_tiled(const void* src, void* tiled, int N, int K, int src_layout, void* stream);
uint64_t tlx_iq3_tiled_bytes(int N, int K);

/* ---- MoE grouped-expert path (256 routed experts + 1 shared, hidden 2048, expert FF 512,
 * top-8; IQ4_XS weights).  Pairs are position-major, rank ascending: pair = 8*pos + rank.
 * Expert e's gate/up slab at ptbl[e] (512 gate rows, then 512 up rows 557,056 B later; 1088 B
 * a row), its down slab at ptbl_dn[e] (2048 rows x 272 B).  ptbl / ptbl_dn are device arrays
 * of 256 device addresses.  layout (the expert GEMMs' trailing argument): TLX_LAYOUT_RAW for
 * slabs of GGUF rows as above, TLX_LAYOUT_TILED for slabs repacked by tlx_pack_iq4_tiled (same
 * size, same results bit for bit; faster: every wave load is one contiguous run). */

/* GGUF IQ4_XS rows u8[N][K/256*136] -> tiled records u8[N/16][K/256][2176] (N % 16 == 0,
 * K % 256 == 0; 8-B aligned buffers): per (16-row tile, 256-k block) the 16 rows' block headers
 * (8 B each, row order), then their quant bytes in MFMA lane order -- lane l = 16 kq + r holds row
 * r's bytes 16 kq .. 16 kq + 15, then (a second 1024 B) its bytes 64 + 16 kq .. .  A pure byte
 * permutation; an expert slab keeps its size and its up rows their offset.  No reference
 * counterpart: the reference reads GGUF rows (engine/mm/MM_P2_gx8e256up4.cu:23-39); this is the
 * load-time repack for the grouped GEMMs' layout argument. */
int tlx_pack_iq4_tiled(const void* src, void* tiled, int N, int K, void* stream);

/* Top-8 + renormalized softmax from router logits f32[P][256], 16-B aligned (the router epilogue of
 * engine/mm/MM_P1_rt8e256.cu:41-60: strict >, ties to the lower id).  eids u16[P][8],
 * gates f32[P][8].  No reference counterpart on its own: the benchmark's MoE configuration feeds logits. */
int tlx_moe_topk(const float* logits, uint16_t* eids, float* gates, int P, void* stream);

/* Router: logits = wrt[256][2048] . h[P][2048], top-8 + softmax, sg = sigmoid(wsh . h).
 * Replaces rt8e256 (engine/mm/MM_P1_rt8e256.cu:14-21): rt8e256(wrt, wsh, h, eids, gates, sg). */
int tlx_moe_route(const float* wrt, const float* wsh, const float* h, uint16_t* eids, float* gates,
                  float* sg, int P, void* stream);

/* Deterministic stable sort of the np = 8P pairs by expert (eids 8-B aligned): eoff i32[257] (exclusive bin
 * offsets), plist u16[np] (pair ids, pair order inside a bin), items u32[tlx_moe_max_items(np)]
 * (expert << 16 | first pair in bin, one per 64 pairs for np <= 512 and per 96 pairs above: the
 * grouped GEMMs' forms), nitp u32[1] (item count).  np <= 16384.
 * Replaces mmsort8 (engine/mm/MM_B_mmsort8.cu:22-31): mmsort8(eids, eoff, plist, items, nitp, np);
 * eoff / plist are the reference's, the item granularity is this library's own. */
int tlx_moe_sort(const uint16_t* eids, int* eoff, uint16_t* plist, uint32_t* items, uint32_t* nitp,
                 int np, void* stream);
int tlx_moe_max_items(int np);

/* Grouped gate+up + SwiGLU over the sorted pairs: ys[pair][512] = silu(Wg_e . x[pos]) * (Wu_e . x[pos]),
 * f32, pos = pair >> 3.  Replaces gxm_up4 (engine/mm/MM_B_gxm_up4.cu:20-28): gxm_up4(ptbl, items, nitp,
 * eoff, plist, xs f32[P][2048], iq4nlb f32[16], ys), same positional order; items / nitp are the
 * ones tlx_moe_sort wrote.  The fp16-MMA prefill form gxu_gm (engine/mm/MM_E_gxu_gm.cu:86-93) is
 * the same call: np > 512 runs the MFMA grouped GEMM. */
int tlx_moe_up4(const uint64_t* ptbl, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                const uint16_t* plist, const float* xs, const float* iq4nl, float* ys, int np, int layout,
                void* stream);

/* Grouped down over the sorted pairs: parts[pair][2048] = fp16(Wd_e . act[pair]).
 * Replaces gxm_dn / gxm_dnf (engine/mm/MM_B_gxm_dn.cu:15-23, engine/mm/MM_C_gxm_dnf.cu:22):
 * gxm_dn(ptbl, items, nitp, eoff, plist, xs = act f32[NPAIR][512], iq4nlb, parts), same order;
 * np > 160 runs the MFMA form (gxd_gm, engine/mm/MM_E_gxd_gm.cu:91-97). */
int tlx_moe_dn4(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                const uint16_t* plist, const float* act, const float* iq4nl, uint16_t* parts, int np,
                int layout, void* stream);

/* Pair-walk decode form of tlx_moe_up4 (no sort): pair p runs expert eids[p] on x[p >> 3].
 * Replaces gx8e256up4 (engine/mm/MM_P2_gx8e256up4.cu:8-14): gx8e256up4(ptbl, eids, xs, iq4nlb, ys)
 * launched over NPAIR = np blocks.  Bit-identical to tlx_moe_up4 on the same pairs. */
int tlx_moe_up4_pairs(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* iq4nl,
                      float* ys, int np, int layout, void* stream);

/* Pair-walk decode form of tlx_moe_dn4: pair p runs expert eids[p] on act[p].
 * Replaces gx8e256dn (engine/mm/MM_P2_gx8e256dn.cu:8-14): gx8e256dn(ptbl, eids, xs, iq4nlb, parts).
 * Bit-identical to tlx_moe_dn4 on the same pairs. */
int tlx_moe_dn4_pairs(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, const float* iq4nl,
                      uint16_t* parts, int np, int layout, void* stream);

/* The pair walk with the shared expert in the same launch (decode sizes: one launch per
 * projection instead of two).  No counterpart among the reference's entry points: its fused
 * decode sequence (engine/mm/MM_P7_lib.py:436-448, MM_FUSE2) merges launches of this layer the
 * same way.  P positions, 8 P pairs: tlx_moe_up4_pairs over the pairs plus tlx_moe_shared's
 * gate+up (ptbl_sh[0], into sact[P][512]); tlx_moe_dn4_pairs over the pairs plus the shared
 * down projection (ptbl_sh_dn[0] = the shared down slab, sact into shared[P][2048] f32).  The
 * outputs are those of the separate calls bit for bit.  sact and shared 16-B aligned. */
int tlx_moe_up4_pairs_sh(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* iq4nl,
                         float* ys, const uint64_t* ptbl_sh, float* sact, int P, int layout, void* stream);
int tlx_moe_dn4_pairs_sh(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, const float* iq4nl,
                         uint16_t* parts, const uint64_t* ptbl_sh_dn, const float* sact, float* shared, int P,
                         int layout, void* stream);

/* The grouped forms (tlx_moe_up4 / tlx_moe_dn4 over the sorted pairs) and the shared expert's
 * gate+up / down over the P positions in one launch each, where both sides run their MFMA forms
 * (np > 512 / 160 and P > 256; else the two launches): the shared expert's workgroups follow the
 * routed ones and fill the routed grid's last, partial round.  No counterpart in the reference
 * (its shared expert is separate launches, engine/mm/MM_P7_lib.py:449-511 sequences them); the
 * outputs are those of the separate calls bit for bit.  sact (f32 [P][512]) and shared (f32
 * [P][2048]) as tlx_moe_shared's act / out; ptbl_sh / ptbl_sh_dn one slab pointer each. */
int tlx_moe_up4_sh(const uint64_t* ptbl, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                   const uint16_t* plist, const float* xs, const float* iq4nl, float* ys, int np,
                   const uint64_t* ptbl_sh, float* sact, int P, int layout, void* stream);
int tlx_moe_dn4_sh(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                   const uint16_t* plist, const float* act, const float* iq4nl, uint16_t* parts, int np,
                   const uint64_t* ptbl_sh_dn, const float* sact, float* shared, int P, int layout, void* stream);

/* Shared expert over all P positions: act[P][512] (caller scratch) then out[P][2048] f32.
 * ptbl_sh = {gate/up slab, down slab}.  Replaces shgu32 / shdn32 (engine/mm/MM_P2_ports.py:195-201
 * restates them) with the IQ4_XS weights of the benchmark's MoE configuration. */
int tlx_moe_shared(const uint64_t* ptbl_sh, const float* xs, const float* iq4nl, float* act, float* out,
                   int P, int layout, void* stream);

/* y = hres + (sum_r gates[r] * parts[pos][r] + sg * shared), f32[P][2048].
 * Replaces cmbz2048 (engine/mm/MM_P34_cmbz2048.cu:6-13): cmbz2048(parts, gates, sg, shared, hres, y). */
int tlx_moe_combine(const uint16_t* parts, const float* gates, const float* sg, const float* shared,
                    const float* hres, float* y, int P, void* stream);

/* ---- The MoE weight classes of the reference's real checkpoint (Qwen3.6-35B-A3B): IQ3_S routed
 * gate/up, Q6_K routed down (3 of 40 layers), Q8_0 shared expert.  Operands are fp16 of the fp32
 * GGUF values, f32 accumulation (results within rel-err 1e-3 of the float64 products; the
 * reference's decode forms accumulate in fp32 FMA-free, its prefill forms in fp16 MMA).  Slabs as
 * the reference's: IQ3_S gate/up slab = 512 gate rows, then 512 up rows from byte 450,560, 880 B a
 * row (k = 2048); Q6_K down slab = 2048 rows of 420 B (raw 210-B blocks, k = 512); slab addresses
 * 2-B aligned.  gridf: the IQ3_S grid as float[512][4], passed at run time as by the reference.
 * np = number of pairs (8 per position), <= 16384; the sorted forms take tlx_moe_sort's eoff / plist.
 * layout (the routed forms' argument before the stream): TLX_LAYOUT_RAW for slabs of GGUF rows as
 * above, TLX_LAYOUT_TILED for slabs repacked by tlx_pack_iq3s_tiled / tlx_pack_q6k_tiled (same
 * size, same results bit for bit: every lane's bytes of a block are one contiguous run). */

/* GGUF IQ3_S rows u8[N][K/256*110] -> tiled records u8[N/16][K/256][1760]; GGUF Q6_K rows
 * u8[N][K/256*210] -> u8[N/16][K/256][3360] (N % 16 == 0, K % 256 == 0).  Record (tile, block), lane
 * l = 16 kq + r (row r of the tile): IQ3_S [qs: lane l's 16 B qs[16kq..] | signs: 8 B signs[8kq..] |
 * qh: 2 B qh[2kq..] | scale byte kq | 16 rows' d]; Q6_K [ql: lane l's 32 B ql[32kq..] | qh: row r's
 * 32 B qh[32h..] at 32 (16 h + r) | sc: 4 B sc[8h + 2c + {0,1,4,5}] (h = kq/2, c = kq%2) | 16 rows' d].
 * A pure byte permutation: an expert slab keeps its size and its up rows their offset.  No reference
 * counterpart (the reference reads GGUF rows, engine/mm/MM_E_gxu_gm.cu:86-93 and
 * engine/mm/MM_B_gxm_dn6.cu:18-25); the load-time repack for the layout argument above. */
int tlx_pack_iq3s_tiled(const void* src, void* tiled, int N, int K, void* stream);
int tlx_pack_q6k_tiled(const void* src, void* tiled, int N, int K, void* stream);

/* IQ3_S dequant (dq_iq3_s, engine/mm/MM_P0_d2_repack.py:95-120): 110-B blocks
 * [d f16][qs 64][qh 8][signs 32][scales 4]; out f32 or (out_f16) fp16 [rows][kdim], kdim % 256. */
int tlx_iq3s_dequant(const void* w, const float* gridf, void* out, int64_t rows, int64_t kdim, int out_f16,
                     void* stream);
/* Q8_0 dequant (dq_q8_0, engine/mm/MM_P2_ports.py:47-54): 34-B blocks [d f16][q i8 32], y = d * q;
 * kdim % 256. */
int tlx_q8_0_dequant(const void* w, void* out, int64_t rows, int64_t kdim, int out_f16, void* stream);

/* IQ3_S grouped gate+up + SwiGLU over the sorted pairs: ys[pair][512] f32 =
 * silu(Wg_e . x[pair >> 3]) * (Wu_e . x[pair >> 3]).  Replaces gxu_gm
 * (engine/mm/MM_E_gxu_gm.cu:86-93): gxu_gm(ptbl, eoff, plist, xs f32[P][2048], gridf, ys). */
int tlx_moe_up3s(const uint64_t* ptbl, const int* eoff, const uint16_t* plist, const float* xs,
                 const float* gridf, float* ys, int np, int layout, void* stream);
/* Pair-walk form (no sort): pair p runs expert eids[p].  Replaces gx8e256up
 * (engine/mm/MM_P1_gx8e256up.cu:15-20): gx8e256up(ptbl, eids, xs, gridf, ys).  The decode form:
 * weights go straight to registers, the grid's levels are read as fp16 (exact for the IQ3_S
 * grid's integers); the operands are tlx_moe_up3s's, summed in another k order (within 1e-5). */
int tlx_moe_up3s_pairs(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* gridf,
                       float* ys, int np, int layout, void* stream);
/* Q6_K grouped down over the sorted pairs: parts[pair][2048] = fp16(Wd_e . act[pair]).  Replaces
 * gxm_dn6 (engine/mm/MM_B_gxm_dn6.cu:18-25): gxm_dn6(ptbl, items, nitp, eoff, plist,
 * xs = act f32[NPAIR][512], parts), same positional order; items / nitp are accepted (may be null)
 * and not read: this form walks eoff / plist. */
int tlx_moe_dn6(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                const uint16_t* plist, const float* act, uint16_t* parts, int np, int layout, void* stream);
/* Pair-walk form: replaces gx8e256dn6 (engine/mm/MM_P2_gx8e256dn6.cu:9-13):
 * gx8e256dn6(ptbl, eids, xs = act, parts).  The decode form, as tlx_moe_up3s_pairs: tlx_moe_dn6's
 * operands summed in another k order. */
int tlx_moe_dn6_pairs(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, uint16_t* parts,
                      int np, int layout, void* stream);
/* The sorted forms (tlx_moe_up3s / tlx_moe_dn6) and the Q8_0 shared expert's gate+up / down
 * (tlx_moe_shared8's two launches) in one launch each above P = 16 (else the two launches): the
 * shared expert's workgroups follow the routed ones.  The down keeps two launches whenever parts
 * is 8-B aligned (the routed register-decode form and the shared expert's staged form have LDS
 * footprints one launch cannot share).  No counterpart in the reference (gxu_gm / gxm_dn6 and
 * shexp8 are separate launches); outputs those of the separate calls bit for bit.
 * sact f32 [P][512] (16-B aligned) and shared f32 [P][2048] as tlx_moe_shared8's act / y. */
int tlx_moe_up3s_sh(const uint64_t* ptbl, const int* eoff, const uint16_t* plist, const float* xs,
                    const float* gridf, float* ys, int np, const void* wg8, const void* wu8, float* sact, int P,
                    int layout, void* stream);
int tlx_moe_dn6_sh(const uint64_t* ptbl_dn, const uint32_t* items, const uint32_t* nitp, const int* eoff,
                   const uint16_t* plist, const float* act, uint16_t* parts, int np, const void* wd8,
                   const float* sact, float* shared, int P, int layout, void* stream);
/* The pair walks (tlx_moe_up3s_pairs / tlx_moe_dn6_pairs) and the Q8_0 shared expert's decode forms
 * (tlx_moe_shared8's two launches) in one launch each at P <= 16 (else the two launches): the shared
 * expert's workgroups follow the pairs' and read their token rows from memory (no LDS staging, so
 * the pair walk keeps its occupancy).  No counterpart in the reference (gx8e256up / gx8e256dn6 and
 * shexp8 are separate launches); outputs those of the separate calls bit for bit.  sact f32 [P][512]
 * (16-B aligned) and shared f32 [P][2048] as tlx_moe_shared8's act / y. */
int tlx_moe_up3s_pairs_sh(const uint64_t* ptbl, const uint16_t* eids, const float* xs, const float* gridf,
                          float* ys, int np, const void* wg8, const void* wu8, float* sact, int P, int layout,
                          void* stream);
int tlx_moe_dn6_pairs_sh(const uint64_t* ptbl_dn, const uint16_t* eids, const float* act, uint16_t* parts, int np,
                         const void* wd8, const float* sact, float* shared, int P, int layout, void* stream);
/* The Q8_0 shared expert over P positions: y[P][2048] f32 = Wd . (silu(Wg . x) * (Wu . x)), with act
 * f32[P][512] caller scratch (two launches on the stream; P <= 16 the decode form).  Replaces shexp8
 * (engine/mm/MM_P2_shexp8.cu:8-13): shexp8(wg [512][2176], wu [512][2176], wd [2048][544], x, y).
 * x and act 16-B aligned. */
int tlx_moe_shared8(const void* wg, const void* wu, const void* wd, const float* x, float* y, float* act, int P,
                    void* stream);

/* ---- Measurement.
 * HBM read-stream probe (the measured bandwidth ceiling the benchmark states GEMV throughput
 * against, beside the datasheet figure; the reference's counterpart is its read-stream tool
 * tools/w0_e4_bw.cu, not a hot-path kernel): reads nbytes of src once (nbytes a multiple of
 * tlx_stream_chunk_bytes()), writing 4 * nbytes / tlx_stream_chunk_bytes() words to sink. */
uint64_t tlx_stream_chunk_bytes(void);
int tlx_stream_read(const void* src, uint64_t nbytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TLX_H */
