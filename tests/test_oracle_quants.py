"""Pin the oracle's dequantizers.

Two kinds of check, both independent of the code under test:
* known-answer blocks whose values are worked out by hand from the GGUF block definitions;
* agreement between independent restatements of one format taken from different places in
  the reference (numpy ports vs the CUDA kernels' per-lane decodes).
"""
import numpy as np
import pytest

from oracle import layouts, quants
from thunderllamax_amd import formats, synth

F16_ONE = np.array([1.0], np.float16).view(np.uint8)
F16_TWO = np.array([2.0], np.float16).view(np.uint8)


def _iq3_block(d_bytes, qs, sw):
    b = np.zeros(98, np.uint8)
    b[0:2] = d_bytes
    b[2:66] = qs
    b[66:98] = np.asarray(sw, "<u4").view(np.uint8)
    return b


# ----------------------------------------------------------------------------- IQ3_XXS
def test_iq3_known_answer_plain():
    # d=1, every grid index 0 (|4,4,4,4|), scale nibble 0 -> db = 1*0.5*0.5 -> all weights 1
    b = _iq3_block(F16_ONE, np.zeros(64, np.uint8), np.zeros(8))
    assert np.array_equal(quants.dequant_iq3xxs_blocks(b[None]), np.ones(256, np.float32))


def test_iq3_known_answer_scale_sign_parity_and_index():
    qs = np.zeros(64, np.uint8)
    qs[0] = 1                                  # chunk 0, first 4 weights: grid[1] = bytes 20,4,4,4
    sw = np.zeros(8, np.uint32)
    sw[0] = (15 << 28) | 1                     # db = 2*15.5*0.5 = 15.5; chunk 0 sign field = 1
    sw[2] = 0x7F << 21                         # sub-block 2, chunk 3: 7 sign bits + parity 1
    b = _iq3_block(F16_TWO, qs, sw)
    w = quants.dequant_iq3xxs_blocks(b[None])
    exp = np.full(256, 0.5, np.float32)        # other sub-blocks: db = 2*0.5*0.5 = 0.5, grid 4
    exp *= 4
    exp[0:32] = 62.0                           # sub-block 0: 15.5 * 4
    exp[0] = -310.0                            # 15.5 * 20, sign bit 0
    exp[7] = -62.0                             # parity(1) = 1 -> weight 7 negative
    exp[64 + 24:64 + 32] = -2.0                # sub-block 2, chunk 3 all negative
    assert np.array_equal(w, exp)


def test_iq3_fp16_rounding_of_packed_form():
    # d with a full mantissa makes db*g need more than 11 bits: the packed (engine) form
    # rounds once to fp16, the block form stays exact
    d = np.array([0.99951171875], np.float16).view(np.uint8)
    qs = np.full(64, 255, np.uint8)            # grid[255] = 0x3e341c04 -> bytes 4,28,52,62
    sw = np.full(8, 0xF0000000, np.uint32)
    b = _iq3_block(d, qs, sw)
    exact = quants.dequant_iq3xxs_blocks(b[None])
    packed = quants.dequant_iq3xxs_packed(layouts.pack_iq3_w1c(b[None], 256), 256)[0]
    assert np.array_equal(packed, exact.astype(np.float16).astype(np.float32))
    assert not np.array_equal(packed, exact)
    assert exact[3] == np.float32(0.99951171875) * np.float32(15.5) * np.float32(0.5) * 62


@pytest.mark.parametrize("rows,kdim", [(6, 512), (2, 5120)])
def test_iq3_three_restatements_agree(rows, kdim):
    raw = synth.iq3xxs_raw(np.random.default_rng(11 + rows), rows, kdim)
    packed = formats.iq3_pack_rows(raw, kdim)
    blocks = quants.dequant_iq3xxs_blocks(raw.reshape(-1, 98)).reshape(rows, kdim)   # a3a / tinygrad
    lanes = quants.dequant_iq3xxs_lanes(packed, kdim)                               # aq3k8 IQ3ROWP
    engine = quants.dequant_iq3xxs_packed(packed, kdim)                             # pack_w4
    assert np.array_equal(blocks, lanes)
    assert np.array_equal(engine, blocks.astype(np.float16).astype(np.float32))


def test_iq3_all_sign_fields():
    # every 7-bit sign index once: the 8th sign is the parity of the 7
    sidx = np.arange(128, dtype=np.uint32)
    sw = np.zeros((32, 8), np.uint32)
    for i in range(128):
        blk, word, field = i // 32, (i % 32) // 4, i % 4
        sw[blk, word] |= sidx[i] << (7 * field)
    blocks = np.stack([_iq3_block(F16_ONE, np.zeros(64, np.uint8), sw[j]) for j in range(4)])
    w = quants.dequant_iq3xxs_blocks(blocks).reshape(128, 8)
    for i in range(128):
        neg = [(i >> j) & 1 for j in range(7)] + [bin(i).count("1") & 1]
        assert np.array_equal(w[i], np.where(np.array(neg) == 1, -1.0, 1.0).astype(np.float32))


# ----------------------------------------------------------------------------- Q6_K
def _q6_block(d=1.0):
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    b[192:208] = 1
    return b


def test_q6k_known_answer():
    b = _q6_block()
    b[0] = 0x21                                # ql[0]: low nibble 1, high nibble 2
    b[128] = 0b11100100                        # qh[0]: 2-bit fields 0, 1, 2, 3
    b[192 + 15] = np.uint8(np.int8(-2).view(np.uint8))   # sc[15]: h=1, l>=16, g=3
    w = quants.dequant_q6k(b[None], 256)[0]
    exp = np.full(256, -32.0, np.float32)
    exp[0] = 1 - 32                            # q = 1 | 0<<4
    exp[32] = 16 - 32                          # ql[32] low = 0, qh field 1 -> 16
    exp[64] = (2 | 2 << 4) - 32                # high nibble 2, field 2 -> 34
    exp[96] = 48 - 32                          # field 3 -> 48
    exp[240:256] = -2.0 * -32                  # elements 128 + 96 + 16..31
    assert np.array_equal(w, exp)


@pytest.mark.parametrize("rows,kdim", [(4, 512), (1, 5120)])
def test_q6k_three_restatements_agree(rows, kdim):
    raw = synth.q6k_raw(np.random.default_rng(5 + rows), rows, kdim)
    a = quants.dequant_q6k(raw, kdim)                                     # MM_P2_ports dq_q6_k
    b = quants.dequant_q6k_h6k_lanes(raw, kdim)                           # h6k2048 lanes
    c = quants.dequant_q6k_padded_lanes(layouts.pack_q6_pad(raw, kdim), kdim)   # aq6k8 lanes
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_q6k_extremes():
    b = _q6_block(d=2.0)
    b[0:128] = 0xFF
    b[128:192] = 0xFF                          # q = 63 everywhere
    b[192:208] = np.int8(-128).view(np.uint8)
    w = quants.dequant_q6k(b[None], 256)[0]
    assert np.all(w == np.float32(2.0 * -128 * 31))


# ----------------------------------------------------------------------------- IQ4_XS
def _iq4_block():
    b = np.zeros(136, np.uint8)
    b[0:2] = F16_ONE
    return b


def test_iq4_known_answer():
    b = _iq4_block()
    b[2:4] = np.array([2], "<u2").view(np.uint8)   # scales_h: group 0 high bits = 2
    b[4] = 0x02                                    # scales_l[0]: group 0 low nibble 2, group 1 low 0
    b[8] = 0xF8                                    # qs[0]: low nibble 8, high nibble 15
    w = quants.dequant_iq4xs(b[None], 256)[0]
    kv = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    assert w[0] == 2 * kv[8]                       # ls = 2 | 2<<4 = 34 -> dl = 2
    assert w[16] == 2 * kv[15]                     # high nibble -> element 16
    assert np.all(w[1:16] == 2 * kv[0]) and np.all(w[17:32] == 2 * kv[0])
    assert np.all(w[32:] == -32 * kv[0])           # groups 1..7: ls = 0 -> dl = -32


def test_iq4_zero_scale_group():
    b = _iq4_block()
    b[2:4] = np.array([0xAAAA], "<u2").view(np.uint8)   # every group's high bits = 2
    w = quants.dequant_iq4xs(b[None], 256)[0]            # ls = 32 -> dl = 0
    assert np.all(w == 0)


@pytest.mark.parametrize("rows,kdim", [(3, 512), (1, 2048)])
def test_iq4_two_restatements_agree(rows, kdim):
    raw = synth.iq4xs_raw(np.random.default_rng(9 + rows), rows, kdim)
    assert np.array_equal(quants.dequant_iq4xs(raw, kdim), quants.dequant_iq4xs_lanes(raw, kdim))
