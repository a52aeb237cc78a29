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


# --------------------------------------------------------------------------- Q4_K / Q5_K
def _k4_pack_scales(sc, mn):
    """12-byte encoding of eight 6-bit (scale, min) pairs, written from the bit layout: bytes
    0-3 hold scales 0-3 in bits 0-5 and bits 4-5 of scales 4-7 in bits 6-7; bytes 4-7 the same
    for the mins; bytes 8-11 hold the low nibbles of scale 4+j (bits 0-3) and min 4+j (4-7)."""
    q = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return q


def _k4_block(five, d, dmin, sc, mn, qs_byte, qh_byte=0):
    blk = np.zeros(176 if five else 144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    blk[4:16] = _k4_pack_scales(sc, mn)
    if five:
        blk[16:48] = qh_byte
        blk[48:176] = qs_byte
    else:
        blk[16:144] = qs_byte
    return blk[None, :]


def test_k4_scale_min_round_trip():
    rng = np.random.default_rng(4)
    for _ in range(50):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        got_sc, got_mn = quants.k4_scale_min(_k4_pack_scales(sc, mn))
        assert np.array_equal(got_sc, sc) and np.array_equal(got_mn, mn)


@pytest.mark.parametrize("five", [False, True])
def test_k4_known_answers(five):
    sc = np.arange(8) * 7 + 1          # distinct 6-bit scales 1..50
    mn = 63 - np.arange(8) * 5         # distinct mins 63..28
    deq = quants.dequant_q5k if five else quants.dequant_q4k
    # all quants zero: every weight is -dmin*m of its sub-block
    y = deq(_k4_block(five, 0.5, 0.25, sc, mn, 0x00), 256)[0]
    np.testing.assert_array_equal(y, np.repeat(-0.25 * mn.astype(np.float32), 32))
    # all quants at their maximum: (d*sc)*qmax - dmin*m
    qmax = 31 if five else 15
    y = deq(_k4_block(five, 0.5, 0.25, sc, mn, 0xFF, 0xFF), 256)[0]
    np.testing.assert_array_equal(y, np.repeat((0.5 * sc * qmax - 0.25 * mn).astype(np.float32), 32))
    # low nibble 3, high nibble 9 (and for Q5_K only the bits of sub-blocks 1 and 6 set):
    # element k reads nibble (k >> 5) & 1 of byte 32(k >> 6) + (k & 31), qh bit k >> 5
    y = deq(_k4_block(five, 1.0, 0.0, np.ones(8, int), np.zeros(8, int), 0x93, 0b01000010), 256)[0]
    k = np.arange(256)
    want = np.where((k >> 5) & 1, 9, 3) + (16 * np.isin(k >> 5, [1, 6]) if five else 0)
    np.testing.assert_array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("five", [False, True])
@pytest.mark.parametrize("rows,kdim", [(3, 512), (1, 2048)])
def test_k4_two_restatements_agree(five, rows, kdim):
    raw = synth.k4_raw(np.random.default_rng(rows + kdim + five), rows, kdim, five)
    a = (quants.dequant_q5k if five else quants.dequant_q4k)(raw, kdim)
    b = (quants.dequant_q5k_lanes if five else quants.dequant_q4k_lanes)(raw, kdim)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ----------------------------------------------------------------------------- IQ3_S
def _grid_ramp():
    """grid[i] = (i, i+0.25, i+0.5, i+0.75) / 4: every entry and lane distinct, so a wrong index,
    lane or high bit shows up as a wrong value."""
    i = np.arange(512, dtype=np.float32)[:, None]
    return (i + np.array([0, 0.25, 0.5, 0.75], np.float32)) / 4


def _iq3s_block():
    b = np.zeros(110, np.uint8)
    b[0:2] = F16_ONE
    return b


def test_iq3s_known_answer_index_high_bit_sign_scale():
    g = _grid_ramp()
    b = _iq3s_block()
    b[2] = 5            # sub-block 0, index byte 0 -> weights 0..3: grid[5]
    b[3] = 7            # index byte 1 -> weights 4..7: grid[7 | 256] (qh bit 1 below)
    b[66] = 0b10        # qh[0]: bit 1 -> index byte 1 gains 256
    b[74] = 0b0110_0001  # signs[0]: weights 0, 5, 6 negative
    b[106] = 0x3 | (0x7 << 4)   # scales[0]: sub-block 0 nibble 3 -> db = 7; sub-block 1 nibble 7 -> 15
    b[2 + 8] = 9        # sub-block 1 index byte 0 -> weights 32..35: grid[9] * 15
    w = quants.dequant_iq3s(b[None], 256, g)[0]
    assert np.array_equal(w[0:4], 7 * g[5] * np.array([-1, 1, 1, 1], np.float32))
    assert np.array_equal(w[4:8], 7 * g[7 + 256] * np.array([1, -1, -1, 1], np.float32))
    assert np.array_equal(w[8:32], np.tile(7 * g[0], 6))   # index bytes 2..7 are 0
    assert np.array_equal(w[32:36], 15 * g[9])
    assert np.array_equal(w[64:96], np.tile(g[0], 8))   # pair 1: scales[1] = 0 -> db = 1


def test_iq3s_all_signs_and_high_bits():
    """Each of the 256 sign bits flips exactly its own weight; each of the 64 high bits moves exactly
    its own index byte's 4 weights to the upper half of the grid."""
    g = _grid_ramp()
    base = quants.dequant_iq3s(_iq3s_block()[None], 256, g)[0]
    for bit in range(256):
        b = _iq3s_block()
        b[74 + bit // 8] = 1 << (bit % 8)
        w = quants.dequant_iq3s(b[None], 256, g)[0]
        want = base.copy()
        want[bit] = -want[bit]
        assert np.array_equal(w, want), bit
    for q in range(64):
        b = _iq3s_block()
        b[66 + q // 8] = 1 << (q % 8)
        w = quants.dequant_iq3s(b[None], 256, g)[0]
        want = base.copy()
        want[4 * q:4 * q + 4] = g[256]
        assert np.array_equal(w, want), q


@pytest.mark.parametrize("rows,kdim", [(3, 512), (1, 2048)])
def test_iq3s_two_restatements_agree(rows, kdim):
    rng = np.random.default_rng(31 + rows)
    raw = synth.iq3s_raw(rng, rows, kdim)
    g = synth.iq3s_grid(rng)
    a, b = quants.dequant_iq3s(raw, kdim, g), quants.dequant_iq3s_lanes(raw, kdim, g)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ----------------------------------------------------------------------------- Q8_0
def test_q80_known_answer_every_int8():
    """Block k holds d = 2^-k (k = 0..7) and q = all 256 int8 values in order: y = d * q exactly."""
    q = np.arange(-128, 128, dtype=np.int8)
    raw = np.zeros((1, 8 * 34), np.uint8)
    for k in range(8):
        blk = raw[0, 34 * k:34 * (k + 1)]
        blk[0:2] = np.array([2.0 ** -k], np.float16).view(np.uint8)
        blk[2:34] = q[32 * k:32 * (k + 1)].view(np.uint8)
    w = quants.dequant_q8_0(raw, 256)[0]
    want = np.concatenate([q[32 * k:32 * (k + 1)].astype(np.float64) * 2.0 ** -k for k in range(8)])
    assert np.array_equal(w.astype(np.float64), want)
