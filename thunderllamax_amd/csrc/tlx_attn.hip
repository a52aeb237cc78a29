// Fused attention q/k/v projections: the reference's four warp-range kernels (aq3k8, aq6k8,
// a_qkv_iq3, a_qkv_q6) as one entry point each.  Segments of one quant format share a launch;
// a segment in another format (the Q6_K q, the Q4_K v) takes a launch of its own on the same
// stream.  Every argument is validated before anything is launched.
#include "tlx_common.h"

namespace {

constexpr int kQ6Raw = 0, kQ6Pad = 1, kQ4K = 2;  // tlx_kq_gemv formats

// q and k are IQ3_XXS in `layout`; v is IQ3_XXS in `layout`, or Q4_K when v4 is set.
int attn_iq3(const void* wq, const void* wk, const void* wv, const float* gridf, const uint16_t* xh,
             uint16_t* qrow, uint16_t* krow, uint16_t* vrow, int M, int Nq, int Nk, int Nv, int K,
             int layout, bool v4, void* stream) {
  const void* w[3] = {wq, wk, wv};
  uint16_t* out[3] = {qrow, krow, vrow};
  const int n[3] = {Nq, Nk, Nv};
  const int nseg = v4 ? 2 : 3;
  int rc = tlx_iq3_segments(w, out, n, nseg, gridf, xh, M, K, layout, false, stream);
  if (rc == TLX_OK && v4) rc = tlx_kq_gemv(kQ4K, wv, xh, vrow, M, Nv, K, false, stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  rc = tlx_iq3_segments(w, out, n, nseg, gridf, xh, M, K, layout, true, stream);
  if (rc == TLX_OK && v4) rc = tlx_kq_gemv(kQ4K, wv, xh, vrow, M, Nv, K, true, stream);
  return rc;
}

// q is Q6_K (fmt), k is IQ3_XXS in `klayout`; v is IQ3_XXS in `klayout`, or Q4_K when v4 is set.
int attn_q6(int fmt, const void* wq, const void* wk, const void* wv, const float* gridf,
            const uint16_t* xh, uint16_t* qrow, uint16_t* krow, uint16_t* vrow, int M, int Nq,
            int Nk, int Nv, int K, int klayout, bool v4, void* stream) {
  const void* w[2] = {wk, wv};
  uint16_t* out[2] = {krow, vrow};
  const int n[2] = {Nk, Nv};
  const int nseg = v4 ? 1 : 2;
  int rc = tlx_kq_gemv(fmt, wq, xh, qrow, M, Nq, K, false, stream);
  if (rc == TLX_OK) rc = tlx_iq3_segments(w, out, n, nseg, gridf, xh, M, K, klayout, false, stream);
  if (rc == TLX_OK && v4) rc = tlx_kq_gemv(kQ4K, wv, xh, vrow, M, Nv, K, false, stream);
  TLX_RET_IF(rc != TLX_OK, rc);
  rc = tlx_iq3_segments(w, out, n, nseg, gridf, xh, M, K, klayout, true, stream);
  if (rc == TLX_OK && v4) rc = tlx_kq_gemv(kQ4K, wv, xh, vrow, M, Nv, K, true, stream);
  if (rc == TLX_OK) rc = tlx_kq_gemv(fmt, wq, xh, qrow, M, Nq, K, true, stream);
  return rc;
}

}  // namespace

extern "C" int tlx_aq3k8(const void* wq, const void* wk, const void* wv, const float* gridf,
                         const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                         uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, int layout,
                         void* stream) {
  return attn_iq3(wq, wk, wv, gridf, xh_f16, qrow_f16, krow_f16, vrow_f16, M, Nq, Nk, Nv, K,
                  layout & ~TLX_V_Q4K, (layout & TLX_V_Q4K) != 0, stream);
}

extern "C" int tlx_aq6k8(const void* wq, const void* wk, const void* wv, const float* gridf,
                         const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                         uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, int layout,
                         void* stream) {
  const int base = layout & ~TLX_V_Q4K;
  TLX_RET_IF(base != TLX_LAYOUT_RAW && base != TLX_LAYOUT_PACKED, TLX_E_ARG);
  return attn_q6(base == TLX_LAYOUT_RAW ? kQ6Raw : kQ6Pad, wq, wk, wv, gridf, xh_f16, qrow_f16,
                 krow_f16, vrow_f16, M, Nq, Nk, Nv, K, TLX_LAYOUT_PACKED, (layout & TLX_V_Q4K) != 0,
                 stream);
}

extern "C" int tlx_a_qkv_iq3(const void* wq, const void* wk, const void* wv4, const float* gridf,
                             const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                             uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, void* stream) {
  return attn_iq3(wq, wk, wv4, gridf, xh_f16, qrow_f16, krow_f16, vrow_f16, M, Nq, Nk, Nv, K,
                  TLX_LAYOUT_RAW, true, stream);
}

extern "C" int tlx_a_qkv_q6(const void* wq, const void* wk, const void* wv4, const float* gridf,
                            const uint16_t* xh_f16, uint16_t* qrow_f16, uint16_t* krow_f16,
                            uint16_t* vrow_f16, int M, int Nq, int Nk, int Nv, int K, void* stream) {
  return attn_q6(kQ6Raw, wq, wk, wv4, gridf, xh_f16, qrow_f16, krow_f16, vrow_f16, M, Nq, Nk, Nv, K,
                 TLX_LAYOUT_RAW, true, stream);
}
