"""The C ABI: the built library loads, exports every entry point include/tlx.h declares,
the ctypes table matches the header, and argument validation rejects bad calls before any
device work (these calls return before touching the GPU, so they run on the CPU host)."""
import ctypes
import os
import re

import pytest

from thunderllamax_amd import _lib

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "tlx.h")


def _declared():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tlx_\w+)\s*\(", src)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_header_and_binding_argument_counts_agree():
    src = re.sub(r"/\*.*?\*/", "", open(HDR).read(), flags=re.S)
    for name, params in re.findall(r"\b(tlx_\w+)\s*\(([^)]*)\)\s*;", src):
        params = params.strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(_lib.SIGNATURES[name]), name


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(L, name), name


def test_version_and_strerror():
    L = _lib.lib()
    assert L.tlx_version() >= 1
    assert b"argument" in L.tlx_strerror(_lib.TLX_E_ARG)
    assert b"align" in L.tlx_strerror(_lib.TLX_E_ALIGN)


@pytest.mark.parametrize("M,N,K,layout,code", [
    (0, 64, 5120, 1, _lib.TLX_E_ARG),        # M below range
    (17, 64, 5120, 1, _lib.TLX_E_ARG),       # M above TLX_MAX_M
    (1, 64, 5000, 1, _lib.TLX_E_ARG),        # K not a multiple of 256
    (1, 60, 5120, 2, _lib.TLX_E_ARG),        # packed7 units come in 8-row groups
    (1, 64, 5120, 5, _lib.TLX_E_ARG),        # no such layout
    (1, 64, 256 * 21, 1, _lib.TLX_E_ALIGN),  # odd block count -> rows not dword aligned
])
def test_ffn8_argument_validation(M, N, K, layout, code):
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    p = (p + 15) & ~15
    rc = L.tlx_ffn8(p, p, p, p, p, M, N, K, layout, None)
    assert rc == code


def test_q6k_gemv_argument_validation():
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    assert L.tlx_q6k_gemv(p, p, p, 0, 5120, 0, None) == _lib.TLX_E_ARG
    assert L.tlx_q6k_gemv(p, p, p, 16, 5120, 7, None) == _lib.TLX_E_ARG
    assert L.tlx_q6k_gemv(p + 1, p, p, 16, 5120, 0, None) == _lib.TLX_E_ALIGN


def test_tiled_record_size_header_library_and_ops_agree():
    """The record size the header states, tlx_iq3_tiled_bytes and the Python size check agree
    (a caller sizing buffers from the header must not under-allocate)."""
    from thunderllamax_amd import ops
    src = open(HDR).read()
    stated = {int(v) for v in re.findall(r"(\d+)-B records", src)}
    assert stated == {1632}, stated
    assert "1632 B (= tlx_iq3_tiled_bytes(N, K)" in src
    L = _lib.lib()
    for N, K in ((1, 256), (16, 256), (17, 5120), (17408, 5120), (5120, 17408), (48, 5120)):
        want = -(-N // 16) * (K // 256) * 1632
        assert L.tlx_iq3_tiled_bytes(N, K) == want
        assert ops._iq3_w(N, K, _lib.LAYOUT_TILED) == want
    assert L.tlx_iq3_tiled_bytes(0, 256) == 0 and L.tlx_iq3_tiled_bytes(16, 300) == 0


def test_workspace_size_and_attach_validation():
    """Workspace sizes are queryable on the host; attach rejects a short or misaligned GEMV
    buffer before any device work."""
    L = _lib.lib()
    g, m = ctypes.c_uint64(), ctypes.c_uint64()
    assert L.tlx_workspace_size(ctypes.byref(g), ctypes.byref(m)) == 0
    assert 1 << 20 < g.value <= 8 << 20 and m.value == 128 << 20
    assert L.tlx_attach_workspace(0x1000, g.value - 1, None, 0, None) == _lib.TLX_E_ARG
    assert L.tlx_attach_workspace(0x1010, g.value, None, 0, None) == _lib.TLX_E_ALIGN
    assert L.tlx_attach_workspace(None, 0, 0x1010, m.value, None) == _lib.TLX_E_ALIGN
    assert b"workspace" in L.tlx_strerror(_lib.TLX_E_NOWS)


def test_no_device_allocation_in_library_sources():
    """The library allocates no device memory: no hipMalloc / hipFree / hipMemset in csrc/."""
    csrc = os.path.join(os.path.dirname(_lib.LIB_PATH), "csrc")
    for f in sorted(os.listdir(csrc)):
        text = re.sub(r"//[^\n]*", "", open(os.path.join(csrc, f)).read())
        for bad in ("hipMalloc", "hipFree", "hipMemset", "hipExtMalloc"):
            assert bad not in text, (f, bad)


def test_pfg3m_argument_validation():
    """The merged prefill GEMM rejects unsupported weight classes and shapes before any launch."""
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    P = ctypes.c_void_p * 3
    I = ctypes.c_int * 3
    w, o = P(p, p, p), P(p, p, p)

    def rc(n, types, layouts, nseg=3, M=256, K=512, x=p):
        return L.tlx_pfg3m(w, o, I(*n), I(*types), I(*layouts), nseg, p, x, M, K, None)

    ok_t, ok_l = (_lib.TYPE_IQ3_XXS, _lib.TYPE_Q6_K, _lib.TYPE_Q4_K), (_lib.LAYOUT_PACK7, _lib.LAYOUT_PACKED, _lib.LAYOUT_RAW)
    assert rc((256, 256, 256), ok_t, ok_l, nseg=0) == _lib.TLX_E_ARG
    assert rc((256, 256, 256), ok_t, ok_l, nseg=4) == _lib.TLX_E_ARG
    assert rc((256, 256, 128), ok_t, ok_l) == _lib.TLX_E_ARG                      # n % 256
    assert rc((256, 256, 256), ok_t, ok_l, M=128) == _lib.TLX_E_ARG               # M % 256
    assert rc((256, 256, 256), ok_t, ok_l, K=384) == _lib.TLX_E_ARG               # K % 256
    assert rc((256, 256, 256), ok_t, (_lib.LAYOUT_PACKED,) * 3) == _lib.TLX_E_ARG   # IQ3_XXS must be packed7
    assert rc((256, 256, 256), (_lib.TYPE_Q6_K,) * 3, (_lib.LAYOUT_RAW,) * 3) == _lib.TLX_E_ARG  # Q6_K: padded
    assert rc((256, 256, 256), (23,) * 3, (_lib.LAYOUT_RAW,) * 3) == _lib.TLX_E_ARG  # IQ4_XS: not a class
    assert rc((256, 256, 256), ok_t, ok_l, x=p + 2) == _lib.TLX_E_ALIGN


def test_moe_checkpoint_classes_argument_validation():
    """The IQ3_S / Q6_K / Q8_0 expert entry points and dequantizers reject bad sizes and alignment
    before any launch."""
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    R, T = _lib.LAYOUT_RAW, _lib.LAYOUT_TILED
    assert L.tlx_moe_up3s(p, p, p, p, p, p, 0, R, None) == _lib.TLX_E_ARG          # no pairs
    assert L.tlx_moe_up3s(p, p, p, p, p, p, 16385, R, None) == _lib.TLX_E_ARG      # more than the sort supports
    assert L.tlx_moe_up3s(p, p, p, p, p, p, 8, _lib.LAYOUT_PACKED, None) == _lib.TLX_E_ARG   # layout
    assert L.tlx_moe_up3s(p, p, p, p + 4, p, p, 8, T, None) == _lib.TLX_E_ALIGN    # xs 16-B aligned
    assert L.tlx_moe_up3s_pairs(p, p, p, p + 8, p, 8, R, None) == _lib.TLX_E_ALIGN # gridf 16-B aligned
    assert L.tlx_moe_up3s_pairs(p, p, p, p, p, 8, 7, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_dn6(p, None, None, p, p, p, p, 0, R, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_dn6(p, None, None, p, p, p, p, 8, _lib.LAYOUT_PACK7, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_dn6_pairs(p, p, p + 4, p, 8, T, None) == _lib.TLX_E_ALIGN
    assert L.tlx_pack_iq3s_tiled(p, p, 8, 256, None) == _lib.TLX_E_ARG            # N % 16
    assert L.tlx_pack_q6k_tiled(p, p, 16, 384, None) == _lib.TLX_E_ARG            # K % 256
    assert L.tlx_moe_shared8(p, p, p, p, p, p, 0, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_shared8(p, p, p, p, p, p + 4, 4, None) == _lib.TLX_E_ALIGN  # act 16-B aligned
    assert L.tlx_iq3s_dequant(p, p, p, 1, 384, 0, None) == _lib.TLX_E_ARG        # kdim % 256
    assert L.tlx_q8_0_dequant(p + 1, p, 1, 256, 0, None) == _lib.TLX_E_ALIGN


def test_moe_grouped_shared_fused_argument_validation():
    """The grouped forms with the shared expert in the same launch reject bad sizes, layouts and
    alignment before any launch."""
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    R = _lib.LAYOUT_RAW
    assert L.tlx_moe_up4_sh(p, p, p, p, p, p, p, p, 0, p, p, 4, R, None) == _lib.TLX_E_ARG       # no pairs
    assert L.tlx_moe_up4_sh(p, p, p, p, p, p, p, p, 32, p, p, 0, R, None) == _lib.TLX_E_ARG      # no positions
    assert L.tlx_moe_up4_sh(p, p, p, p, p, p, p, p, 32, p, p, 4, 7, None) == _lib.TLX_E_ARG      # layout
    assert L.tlx_moe_up4_sh(p, p, p, p, p, p, p, p, 32, p, p + 4, 4, R, None) == _lib.TLX_E_ALIGN   # sact
    assert L.tlx_moe_dn4_sh(p, p, p, p, p, p, p, p, 16385, p, p, p, 4, R, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_dn4_sh(p, p, p, p, p, p, p, p, 32, p, p, p + 4, 4, R, None) == _lib.TLX_E_ALIGN  # shared


def test_moe_checkpoint_fused_argument_validation():
    """The checkpoint-class sorted forms with the shared expert in the same launch reject bad
    sizes and alignment before any launch."""
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    R = _lib.LAYOUT_RAW
    assert L.tlx_moe_up3s_sh(p, p, p, p, p, p, 0, p, p, p, 4, R, None) == _lib.TLX_E_ARG          # no pairs
    assert L.tlx_moe_up3s_sh(p, p, p, p, p, p, 32, p, p, p, 0, R, None) == _lib.TLX_E_ARG         # no positions
    assert L.tlx_moe_up3s_sh(p, p, p, p, p, p, 32, p, p, p, 4, 5, None) == _lib.TLX_E_ARG         # layout
    assert L.tlx_moe_up3s_sh(p, p, p, p, p, p, 32, p, p, p + 4, 4, R, None) == _lib.TLX_E_ALIGN   # sact
    assert L.tlx_moe_up3s_sh(p, p, p, p + 4, p, p, 32, p, p, p, 4, R, None) == _lib.TLX_E_ALIGN   # xs
    assert L.tlx_moe_dn6_sh(p, None, None, p, p, p, p, 16385, p, p, p, 4, R, None) == _lib.TLX_E_ARG
    assert L.tlx_moe_dn6_sh(p, None, None, p, p, p, p, 32, p, p, p, 4, 9, None) == _lib.TLX_E_ARG   # layout
    assert L.tlx_moe_dn6_sh(p, None, None, p, p, p, p, 32, p + 1, p, p, 4, R, None) == _lib.TLX_E_ALIGN  # wd8
    assert L.tlx_moe_up3s_pairs_sh(p, p, p, p, p, 0, p, p, p, 1, R, None) == _lib.TLX_E_ARG          # no pairs
    assert L.tlx_moe_up3s_pairs_sh(p, p, p, p, p, 8, p, p, p, 1, 2, None) == _lib.TLX_E_ARG          # layout
    assert L.tlx_moe_up3s_pairs_sh(p, p, p, p, p, 8, p, p, p + 4, 1, R, None) == _lib.TLX_E_ALIGN    # sact
    assert L.tlx_moe_dn6_pairs_sh(p, p, p, p, 8, p, p, p, 0, R, None) == _lib.TLX_E_ARG              # no positions
    assert L.tlx_moe_dn6_pairs_sh(p, p, p, p, 8, p, p + 4, p, 1, R, None) == _lib.TLX_E_ALIGN        # sact
