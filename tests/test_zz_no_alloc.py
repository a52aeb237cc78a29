"""tlx_ffn8_noalloc (ffn8 on the library's own static scratch, no workspace, no allocation) called
through the C ABI against tlx_ffn8 on the same inputs: two calls in a row, the second with a
smaller input, on the tiled records (parts + counters of the scratch) and on the packed rows at
M >= 6 (the scratch's activation-copy region).  The kernels and their order are tlx_ffn8's, so the
outputs must be identical bit for bit (stricter than the path's rel-err 1e-3)."""
import numpy as np
import pytest
import torch

from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_TILED, TLX_E_ARG, call, lib

pytestmark = pytest.mark.gpu


def _mats(gpu, rng, N, K, tiled):
    out = []
    for _ in range(2):
        p = torch.from_numpy(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)).to(gpu)
        if tiled:
            t = torch.empty(-(-N // 16) * 16 * 102 * (K // 256), dtype=torch.uint8, device=gpu)
            ops.pack_iq3_tiled(p, t, N, K)
            p = t
        out.append(p)
    return out


def _noalloc(wg, wu, g, x, out, layout, stream):
    M, K, N = x.shape[0], x.shape[1], out.shape[1]
    call("tlx_ffn8_noalloc", wg.data_ptr(), wu.data_ptr(), g.data_ptr(), x.data_ptr(), out.data_ptr(),
         M, N, K, layout, stream)


@pytest.mark.parametrize("layout", [LAYOUT_TILED, LAYOUT_PACKED])
def test_ffn8_noalloc_equals_ffn8(gpu, layout):
    tiled = layout == LAYOUT_TILED
    rng = np.random.default_rng(77)
    g = formats.gridf_tensor(gpu)
    st = torch.cuda.current_stream().cuda_stream
    # first call: config 2's full size at M = 11; second: a smaller matrix and fewer rows
    for N, K, M in ((17408, 5120, 11), (1000, 2560, 7)):
        print(f"[case] ffn8_noalloc layout={layout} N={N} K={K} M={M}", flush=True)
        wg, wu = _mats(gpu, rng, N, K, tiled)
        x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
        a = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        _noalloc(wg, wu, g, x, a, layout, st)       # before any workspace use in this test
        torch.cuda.synchronize()
        b = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        ops.ffn8(wg, wu, g, x, b, layout=layout)
        torch.cuda.synchronize()
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_ffn8_noalloc_rejects_k_beyond_scratch(gpu):
    """K > 65536 does not fit the scratch's activation-copy region: rejected before any launch."""
    L = lib()
    x = torch.zeros(16, dtype=torch.float16, device=gpu)
    p = x.data_ptr()
    assert L.tlx_ffn8_noalloc(p, p, p, p, p, 1, 16, 65536 + 256, LAYOUT_TILED, None) == TLX_E_ARG
