"""Product packers (thunderllamax_amd.formats) against the oracle's restatement of the
reference packers, and both against their inverses."""
import numpy as np
import pytest

from oracle import layouts
from thunderllamax_amd import formats, synth


@pytest.mark.parametrize("rows,kdim", [(8, 256), (16, 512), (24, 5120)])
def test_iq3_packed_matches_reference_packer(rows, kdim):
    raw = synth.iq3xxs_raw(np.random.default_rng(rows + kdim), rows, kdim)
    p = formats.iq3_pack_rows(raw, kdim)
    assert np.array_equal(p, layouts.pack_iq3_w1c(raw, kdim))
    assert np.array_equal(layouts.unpack_iq3_w1c(p, kdim), raw)


@pytest.mark.parametrize("rows,kdim", [(8, 256), (16, 1024)])
def test_pack7_matches_reference_packer_and_inverts(rows, kdim):
    raw = synth.iq3xxs_raw(np.random.default_rng(7), rows, kdim)
    p = formats.iq3_pack_rows(raw, kdim)
    p7 = formats.iq3_pack7(p, kdim)
    assert np.array_equal(p7, layouts.pack_w7(p, kdim))
    assert np.array_equal(layouts.unpack_w7(p7, kdim, rows), p)
    assert np.all(p7[..., 14:16] == 0)


@pytest.mark.parametrize("rows,kdim", [(3, 256), (5, 1024)])
def test_q6_padded_matches_reference_packer(rows, kdim):
    raw = synth.q6k_raw(np.random.default_rng(3), rows, kdim)
    p = formats.q6_pad_rows(raw, kdim)
    assert np.array_equal(p, layouts.pack_q6_pad(raw, kdim))
    blk = p.reshape(rows, -1, 212)
    assert np.all(blk[:, :, 0:2] == 0)
    assert np.array_equal(blk[:, :, 20:212], raw.reshape(rows, -1, 210)[:, :, 0:192])


def test_bf16_to_f16_activation_rule():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.0e-5, 65504.0], dtype=np.float32)
    # bf16 keeps 8 significant bits, ties to even
    assert synth.bf16_round(x)[1] == np.float32(1.0)           # exact tie -> even
    assert synth.bf16_round(x)[2] == np.float32(1.0078125)
    f = synth.activations_f16(np.random.default_rng(0), 4, 256)
    assert f.dtype == np.float16 and np.all(np.isfinite(f))
