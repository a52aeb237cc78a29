// On-disk formats: the GGUF v3 tensor table (host) and the weight repackers (GPU).
//
// tlx_gguf_parse restates the reader contract of engine/engine0.py:25-51: header (magic,
// version, tensor count, key/value count), the key/value section skipped value by value
// (strings, nested arrays), the tensor table (name, dims in GGUF order -- dims[0] is the row
// length, "[in, out]" -- ggml type, offset), and data_start = the position after the table
// rounded up to 32 bytes.  Byte sizes follow the reference's tables (tnbytes,
// engine/engine0.py:20-22,53-55).  It reads a caller-provided image of the file's head and
// never touches the device.
//
// The repackers are byte (u16-word) permutations run on the GPU where the weights already
// live, one thread per output word (reads and writes coalesced along the output):
//   * tlx_pack_iq3_rows -- engine/pack_w1c.py:20-31: raw IQ3_XXS rows [N][NB][d2|qs64|sw32]
//     -> packed rows [qs 64NB][sw 32NB][d 2NB];
//   * tlx_pack_q6_pad   -- engine/pack_w1c.py:33-45: raw Q6_K rows [N][NB][ql128|qh64|sc16|d2]
//     -> padded blocks [pad2][d2][sc16][ql128][qh64];
//   * tlx_pack_w7       -- engine/pack_w7.py:40-75: packed IQ3_XXS rows -> packed7 units
//     [N/8][K/128][32][q u16 x4 | sw u32 | d u16 | pad u16], unit r*4 + c = row r of the group,
//     sub-block c of the 128-k chunk.
#include "tlx_common.h"

#include <cstring>

namespace {

// ------------------------------------------------------------------ GGUF reader
struct Cursor {
  const uint8_t* p;
  uint64_t len, pos;
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (pos + sizeof(T) > len) { ok = false; return v; }
    std::memcpy(&v, p + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  void skip(uint64_t n) {
    if (n > len - pos) { ok = false; pos = len; return; }
    pos += n;
  }
};

// bytes of a scalar key/value type (engine/engine0.py:23), 0 for string / array / unknown
uint64_t gguf_scalar_bytes(int32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;   // u8, i8, bool
    case 2: case 3: return 2;           // u16, i16
    case 4: case 5: case 6: return 4;   // u32, i32, f32
    case 10: case 11: case 12: return 8;   // u64, i64, f64
    default: return 0;
  }
}

// skip one value of type t; false on an unknown type (or nesting deeper than the reader allows)
bool gguf_skip_value(Cursor& c, int32_t t, int depth) {
  if (t == 8) {   // string: u64 length + bytes
    c.skip(c.get<uint64_t>());
    return c.ok;
  }
  if (t == 9) {   // array: element type, u64 count, elements
    if (depth > 8) return false;
    const int32_t et = c.get<int32_t>();
    const uint64_t n = c.get<uint64_t>();
    if (!c.ok) return false;
    const uint64_t eb = gguf_scalar_bytes(et);
    if (eb) {
      if (n > (c.len - c.pos) / eb) { c.ok = false; return true; }
      c.skip(n * eb);
      return c.ok;
    }
    for (uint64_t i = 0; i < n && c.ok; ++i)
      if (!gguf_skip_value(c, et, depth + 1)) return false;
    return true;
  }
  const uint64_t b = gguf_scalar_bytes(t);
  if (!b) return false;
  c.skip(b);
  return true;
}

// tnbytes (engine/engine0.py:20-22,53-55): elements per block and block bytes of the quantized
// types, element bytes of the plain ones; 0 for a type the reference does not know
uint64_t gguf_tensor_bytes(uint64_t ne, int32_t t) {
  switch (t) {
    case 0: return 4 * ne;  case 1: return 2 * ne;  case 24: return ne;      case 25: return 2 * ne;
    case 26: return 4 * ne; case 27: return 8 * ne; case 28: return 8 * ne;  case 30: return 2 * ne;
    case 2: return ne / 32 * 18;   case 3: return ne / 32 * 20;   case 6: return ne / 32 * 22;
    case 7: return ne / 32 * 24;   case 8: return ne / 32 * 34;   case 12: return ne / 256 * 144;
    case 13: return ne / 256 * 176; case 14: return ne / 256 * 210; case 18: return ne / 256 * 98;
    case 21: return ne / 256 * 110; case 22: return ne / 256 * 82; case 23: return ne / 256 * 136;
    case 39: return ne / 32 * 17;  case 41: return ne / 128 * 18;
    default: return 0;
  }
}

// ------------------------------------------------------------------ repack kernels
// raw IQ3_XXS block = 49 u16 words: d, qs[32], sw[16]
__global__ __launch_bounds__(256) void pack_iq3_rows_kernel(const uint16_t* __restrict__ raw, uint16_t* __restrict__ out,
                                                            long total, int nb) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;   // output word
  if (i >= total) return;
  const int rw = 49 * nb;                 // u16 words per row
  const long row = i / rw;
  const int w = (int)(i - row * rw);
  int b, src;                             // block, word within the raw block
  if (w < 32 * nb) { b = w >> 5; src = 1 + (w & 31); }                   // qs
  else if (w < 48 * nb) { b = (w - 32 * nb) >> 4; src = 33 + ((w - 32 * nb) & 15); }   // sw
  else { b = w - 48 * nb; src = 0; }                                    // d
  out[i] = raw[row * rw + 49 * b + src];
}

// raw Q6_K block = 105 u16 words: ql[64], qh[32], sc[8], d; padded = 106: pad, d, sc[8], ql[64], qh[32]
__global__ __launch_bounds__(256) void pack_q6_pad_kernel(const uint16_t* __restrict__ raw, uint16_t* __restrict__ out,
                                                          long total) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;   // output word
  if (i >= total) return;
  const long blk = i / 106;
  const int w = (int)(i - blk * 106);
  int src;
  if (w == 0) { out[i] = 0; return; }
  if (w == 1) src = 104;                  // d
  else if (w < 10) src = 96 + (w - 2);    // sc
  else if (w < 74) src = w - 10;          // ql
  else src = 64 + (w - 74);               // qh
  out[i] = raw[blk * 105 + src];
}

// packed7 unit word s of unit u = r * 4 + c in (group g, chunk ch): q words 0..3, sw lo / hi, d, pad
__global__ __launch_bounds__(256) void pack_w7_kernel(const uint16_t* __restrict__ rows, uint16_t* __restrict__ out,
                                                      long total, int nb, int nch) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;   // output word
  if (i >= total) return;
  const int s = (int)(i & 7), u = (int)((i >> 3) & 31);
  const long gc = i >> 8;                 // group * nch + chunk
  const long g = gc / nch;
  const int ch = (int)(gc - g * nch), r = u >> 2, c = u & 3;
  const int b = ch >> 1, h = ch & 1;
  const uint16_t* row = rows + (g * 8 + r) * (long)(49 * nb);
  uint16_t v;
  if (s < 4) v = row[32 * b + 16 * h + 4 * c + s];
  else if (s < 6) v = row[32 * nb + 2 * (8 * b + 4 * h + c) + (s - 4)];
  else if (s == 6) v = row[48 * nb + b];
  else v = 0;
  out[i] = v;
}

unsigned grid_of(long total) { return (unsigned)((total + 255) / 256); }

}  // namespace

extern "C" int tlx_gguf_parse(const void* head, uint64_t len, uint64_t* data_start, int64_t* n_tensors,
                              tlx_gguf_tensor* tensors, int64_t max_tensors) {
  TLX_RET_IF(head == nullptr || data_start == nullptr || n_tensors == nullptr, TLX_E_ARG);
  Cursor c{(const uint8_t*)head, len, 0};
  const uint32_t magic = c.get<uint32_t>();
  TLX_RET_IF(!c.ok, TLX_E_TRUNC);
  TLX_RET_IF(magic != 0x46554747u, TLX_E_ARG);   // "GGUF"
  (void)c.get<int32_t>();                        // version (not checked, as the reference)
  const int64_t nt = c.get<int64_t>(), nkv = c.get<int64_t>();
  TLX_RET_IF(!c.ok, TLX_E_TRUNC);
  TLX_RET_IF(nt < 0 || nkv < 0, TLX_E_ARG);
  for (int64_t i = 0; i < nkv; ++i) {
    c.skip(c.get<uint64_t>());                   // key
    const int32_t t = c.get<int32_t>();
    TLX_RET_IF(!c.ok, TLX_E_TRUNC);
    const bool known = gguf_skip_value(c, t, 0);
    TLX_RET_IF(!c.ok, TLX_E_TRUNC);
    TLX_RET_IF(!known, TLX_E_ARG);
  }
  for (int64_t i = 0; i < nt; ++i) {
    const uint64_t nlen = c.get<uint64_t>();
    TLX_RET_IF(!c.ok || nlen > c.len - c.pos, TLX_E_TRUNC);
    const char* name = (const char*)c.p + c.pos;
    c.skip(nlen);
    const uint32_t nd = c.get<uint32_t>();
    TLX_RET_IF(!c.ok, TLX_E_TRUNC);
    TLX_RET_IF(nd > TLX_GGUF_MAX_DIMS, TLX_E_ARG);
    uint64_t dims[TLX_GGUF_MAX_DIMS] = {0, 0, 0, 0};
    uint64_t ne = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      dims[d] = c.get<uint64_t>();
      ne *= dims[d];
    }
    const int32_t t = c.get<int32_t>();
    const uint64_t off = c.get<uint64_t>();
    TLX_RET_IF(!c.ok, TLX_E_TRUNC);
    if (tensors != nullptr && i < max_tensors) {
      TLX_RET_IF(nlen >= sizeof(tensors[i].name), TLX_E_ARG);
      tlx_gguf_tensor& o = tensors[i];
      std::memset(&o, 0, sizeof(o));
      std::memcpy(o.name, name, nlen);
      o.type = t;
      o.n_dims = nd;
      for (uint32_t d = 0; d < nd; ++d) o.dims[d] = dims[d];
      o.offset = off;
      o.nbytes = gguf_tensor_bytes(ne, t);
    }
  }
  *n_tensors = nt;
  *data_start = (c.pos + 31) / 32 * 32;
  return TLX_OK;
}

extern "C" int tlx_pack_iq3_rows(const void* raw, void* packed, int N, int K, void* stream) {
  TLX_RET_IF(N < 1 || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(raw, 2) || !tlx_aligned(packed, 2), TLX_E_ALIGN);
  const long total = (long)N * 49 * (K / 256);
  pack_iq3_rows_kernel<<<grid_of(total), 256, 0, (hipStream_t)stream>>>((const uint16_t*)raw, (uint16_t*)packed,
                                                                         total, K / 256);
  return tlx_launch_status();
}

extern "C" int tlx_pack_q6_pad(const void* raw, void* padded, int N, int K, void* stream) {
  TLX_RET_IF(N < 1 || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(raw, 2) || !tlx_aligned(padded, 2), TLX_E_ALIGN);
  const long total = (long)N * (K / 256) * 106;
  pack_q6_pad_kernel<<<grid_of(total), 256, 0, (hipStream_t)stream>>>((const uint16_t*)raw, (uint16_t*)padded, total);
  return tlx_launch_status();
}

extern "C" int tlx_pack_w7(const void* packed, void* p7, int N, int K, void* stream) {
  TLX_RET_IF(N < 8 || (N % 8) || K < 256 || (K % 256), TLX_E_ARG);
  TLX_RET_IF(!tlx_aligned(packed, 2) || !tlx_aligned(p7, 2), TLX_E_ALIGN);
  const long total = (long)(N / 8) * (K / 128) * 256;
  pack_w7_kernel<<<grid_of(total), 256, 0, (hipStream_t)stream>>>((const uint16_t*)packed, (uint16_t*)p7, total,
                                                                   K / 256, K / 128);
  return tlx_launch_status();
}
