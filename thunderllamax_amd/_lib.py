"""ctypes binding of libtlx_hip.so (the C ABI declared in include/tlx.h).

The library is loaded from this package directory only; there is no fallback: if it is
missing the import of any op raises, so a GPU run can never silently use another path.
torch is imported first so the process has exactly one HIP runtime (torch's), which the
library then binds to.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtlx_hip.so")

TLX_OK = 0
TLX_E_ARG = -1
TLX_E_ALIGN = -2
TLX_E_NODEV = -3
TLX_E_NOMEM = -4
TLX_E_TRUNC = -5
TLX_E_NOWS = -6
LAYOUT_RAW = 0
LAYOUT_PACKED = 1
LAYOUT_PACK7 = 2
LAYOUT_TILED = 3
V_Q4K = 0x100   # or-ed into the fused attention layout: v rows are GGUF Q4_K
OUT_TILEORD = 0x200   # or-ed into an IQ3_XXS GEMV layout: fp16 output in the tile-ordered form [N/8][16][8]
IN_TILEORD = 0x400    # or-ed into an IQ3_XXS GEMV layout: activations in the tile-ordered form [K/8][16][8]
MAX_M = 16
# ggml type codes of the weight classes the merged prefill GEMM (tlx_pfg3m) takes
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_IQ3_XXS = 18

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64

# name -> argument types (return type is int for all but tlx_strerror)
SIGNATURES = {
    "tlx_version": [],
    "tlx_strerror": [_i],
    "tlx_workspace_size": [_p, _p],
    "tlx_attach_workspace": [_p, ctypes.c_uint64, _p, ctypes.c_uint64, _p],
    "tlx_iq3_tiled_bytes": [_i, _i],
    "tlx_iq3xxs_dequant": [_p, _p, _p, _i64, _i64, _i, _i, _p],
    "tlx_q6k_dequant": [_p, _p, _i64, _i64, _i, _i, _p],
    "tlx_iq4xs_dequant": [_p, _p, _p, _i64, _i64, _p],
    "tlx_ffn8": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_ffn8_noalloc": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_down8": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_iq3_gemv": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_aq3k8": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "tlx_q6k_gemv": [_p, _p, _p, _i, _i, _i, _p],
    "tlx_q6k_gemv16": [_p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_a_qkv_iq3": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "tlx_a_qkv_q6": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "tlx_q4k_gemv16": [_p, _p, _p, _i, _i, _i, _p],
    "tlx_q5k_gemv16": [_p, _p, _p, _i, _i, _i, _p],
    "tlx_head8": [_p, _p, _p, _i, _i, _i, _p],
    "tlx_q4k_dequant": [_p, _p, _i64, _i64, _i, _p],
    "tlx_q5k_dequant": [_p, _p, _i64, _i64, _i, _p],
    "tlx_aq6k8": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p],
    "tlx_pfg3_ffn": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_pfg3_iq3d": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_pfg3_iq3o": [_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_pfg3m": [_p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _p],
    "tlx_p8_quant": [_p, _p, _p, _p, _i, _i, _p],
    "tlx_gguf_parse": [_p, ctypes.c_uint64, _p, _p, _p, _i64],
    "tlx_rms_f16": [_p, _p, _p, _i, _i, _p],
    "tlx_add_rms_f16": [_p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_ffn8_hh": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_pack_iq3_rows": [_p, _p, _i, _i, _p],
    "tlx_pack_q6_pad": [_p, _p, _i, _i, _p],
    "tlx_pack_w7": [_p, _p, _i, _i, _p],
    "tlx_iq3_gemv_multi": [_p, _p, _p, _i, _p, _p, _i, _i, _i, _p],
    "tlx_pack_iq3_tiled": [_p, _p, _i, _i, _i, _p],
    "tlx_p8w4_ffn": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "tlx_moe_topk": [_p, _p, _p, _i, _p],
    "tlx_moe_route": [_p, _p, _p, _p, _p, _p, _i, _p],
    "tlx_moe_sort": [_p, _p, _p, _p, _p, _i, _p],
    "tlx_moe_max_items": [_i],
    "tlx_moe_up4": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn4": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_up4_pairs": [_p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn4_pairs": [_p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_shared": [_p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_up4_pairs_sh": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn4_pairs_sh": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_up4_sh": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _p],
    "tlx_moe_dn4_sh": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p],
    "tlx_pack_iq4_tiled": [_p, _p, _i, _i, _p],
    "tlx_pack_iq3s_tiled": [_p, _p, _i, _i, _p],
    "tlx_pack_q6k_tiled": [_p, _p, _i, _i, _p],
    "tlx_moe_combine": [_p, _p, _p, _p, _p, _p, _i, _p],
    "tlx_iq3s_dequant": [_p, _p, _p, _i64, _i64, _i, _p],
    "tlx_q8_0_dequant": [_p, _p, _i64, _i64, _i, _p],
    "tlx_moe_up3s": [_p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_up3s_pairs": [_p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn6": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn6_pairs": [_p, _p, _p, _p, _i, _i, _p],
    "tlx_moe_up3s_pairs_sh": [_p, _p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn6_pairs_sh": [_p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p],
    "tlx_moe_shared8": [_p, _p, _p, _p, _p, _p, _i, _p],
    "tlx_moe_up3s_sh": [_p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p],
    "tlx_moe_dn6_sh": [_p, _p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p],
    "tlx_stream_chunk_bytes": [],
    "tlx_stream_read": [_p, ctypes.c_uint64, _p, _p],
}


class TlxError(RuntimeError):
    """A libtlx entry point returned a non-zero status."""

    def __init__(self, name, code, msg):
        super().__init__(f"{name}: {msg} (status {code})")
        self.code = code


_LIB = None


def lib():
    """The loaded library (loaded on first use; raises if it was never built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m thunderllamax_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = (ctypes.c_char_p if name == "tlx_strerror" else
                         ctypes.c_uint64 if name in ("tlx_iq3_tiled_bytes", "tlx_stream_chunk_bytes")
                         else ctypes.c_int)
        _LIB = L
    return _LIB


def call(name, *args):
    """Call entry point `name`; raise TlxError on a non-zero status."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != TLX_OK:
        raise TlxError(name, rc, L.tlx_strerror(rc).decode())
    return rc
