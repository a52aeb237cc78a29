"""GPU dequantization kernels against the oracle: bit-exact (float32 and fp16 outputs)."""
import numpy as np
import pytest
import torch

from oracle import layouts, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW

pytestmark = pytest.mark.gpu


def _bits(t):
    a = t.cpu().numpy()
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("rows,kdim", [(1, 256), (37, 5120), (16, 17408)])
@pytest.mark.parametrize("layout", [LAYOUT_RAW, LAYOUT_PACKED])
def test_iq3xxs_dequant_bit_exact(gpu, rows, kdim, layout):
    print(f"[case] iq3xxs_dequant rows={rows} k={kdim} layout={layout}", flush=True)
    raw = synth.iq3xxs_raw(np.random.default_rng(rows * 7 + kdim), rows, kdim)
    host = raw if layout == LAYOUT_RAW else formats.iq3_pack_rows(raw, kdim)
    w = torch.from_numpy(host).to(gpu)
    gridf = formats.gridf_tensor(gpu)
    exact = quants.dequant_iq3xxs_blocks(raw.reshape(-1, 98)).reshape(rows, kdim)
    out32 = torch.empty(rows, kdim, dtype=torch.float32, device=gpu)
    out16 = torch.empty(rows, kdim, dtype=torch.float16, device=gpu)
    ops.iq3xxs_dequant(w, gridf, out32, kdim, layout)
    ops.iq3xxs_dequant(w, gridf, out16, kdim, layout)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out32), exact.view(np.uint32))
    ref16 = quants.dequant_iq3xxs_packed(formats.iq3_pack_rows(raw, kdim), kdim).astype(np.float16)
    assert np.array_equal(_bits(out16), ref16.view(np.uint16))


@pytest.mark.parametrize("rows,kdim", [(1, 256), (29, 5120)])
@pytest.mark.parametrize("layout", [LAYOUT_RAW, LAYOUT_PACKED])
def test_q6k_dequant_bit_exact(gpu, rows, kdim, layout):
    print(f"[case] q6k_dequant rows={rows} k={kdim} layout={layout}", flush=True)
    raw = synth.q6k_raw(np.random.default_rng(rows + kdim), rows, kdim)
    host = raw if layout == LAYOUT_RAW else layouts.pack_q6_pad(raw, kdim)
    w = torch.from_numpy(host).to(gpu)
    ref = quants.dequant_q6k(raw, kdim)
    out32 = torch.empty(rows, kdim, dtype=torch.float32, device=gpu)
    out16 = torch.empty(rows, kdim, dtype=torch.float16, device=gpu)
    ops.q6k_dequant(w, out32, kdim, layout)
    ops.q6k_dequant(w, out16, kdim, layout)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out32), ref.view(np.uint32))
    assert np.array_equal(_bits(out16), ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("rows,kdim", [(1, 256), (19, 2048), (64, 512)])
def test_iq4xs_dequant_bit_exact(gpu, rows, kdim):
    print(f"[case] iq4xs_dequant rows={rows} k={kdim}", flush=True)
    raw = synth.iq4xs_raw(np.random.default_rng(rows + 3 * kdim), rows, kdim)
    w = torch.from_numpy(raw).to(gpu)
    out = torch.empty(rows, kdim, dtype=torch.float32, device=gpu)
    ops.iq4xs_dequant(w, formats.iq4nl_tensor(gpu), out, kdim)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), quants.dequant_iq4xs(raw, kdim).view(np.uint32))
