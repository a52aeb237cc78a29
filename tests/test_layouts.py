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


@pytest.mark.parametrize("rows,kdim", [(16, 256), (21, 512), (32, 5120)])
def test_tiled_records_invert_and_place_fields(rows, kdim):
    raw = synth.iq3xxs_raw(np.random.default_rng(rows), rows, kdim)
    p = formats.iq3_pack_rows(raw, kdim)
    rec = layouts.pack_tiled(p, kdim)
    assert rec.shape == (-(-rows // 16), kdim // 256, 1632)
    assert np.array_equal(layouts.unpack_tiled(rec, kdim, rows), p)
    # rows past N (the tail tile) are zero
    assert np.all(layouts.unpack_tiled(rec, kdim, 16 * len(rec))[rows:] == 0)


def test_tiled_record_decodes_by_hand():
    """One slot decoded with the GGUF rules written out: grid bytes, the 7-bit sign field of the
    chunk, the 8th sign = parity, the sub-block scale nibble and d."""
    kdim, rows = 256, 16
    raw = synth.iq3xxs_raw(np.random.default_rng(5), rows, kdim)
    rec = layouts.pack_tiled(formats.iq3_pack_rows(raw, kdim), kdim)[0, 0]
    r, kq = 9, 2
    blk = raw[r]
    sw = blk[66:98].view("<u4")
    stream = np.concatenate([rec[16 * (16 * kq + r):16 * (16 * kq + r) + 16],
                             rec[1024 + 8 * (16 * kq + r):1024 + 8 * (16 * kq + r) + 8]])
    for c in range(8):
        lc = 8 * kq + c
        sfield = int(sw[lc // 4] >> (7 * (lc % 4))) & 0x7F
        signs = [(sfield >> k) & 1 for k in range(7)]
        signs.append(sum(signs) % 2)
        v = int(stream[3 * c]) | int(stream[3 * c + 1]) << 8 | int(stream[3 * c + 2]) << 16
        i0, i1 = v & 0xFFF, v >> 12
        assert i0 & 0xFF == blk[2 + 2 * lc] and i1 & 0xFF == blk[3 + 2 * lc]
        assert [(i0 >> 8 >> k) & 1 for k in range(4)] == signs[:4]
        assert [(i1 >> 8 >> k) & 1 for k in range(4)] == signs[4:]
    scw = int(rec[1536 + 4 * r:1540 + 4 * r].view("<u4")[0])
    assert [(scw >> (4 * j)) & 15 for j in range(8)] == [int(w >> 28) for w in sw]
    assert bytes(rec[1600 + 2 * r:1602 + 2 * r]) == bytes(blk[0:2])


def test_tiled_unpack_rejects_a_wrong_parity_bit():
    kdim = 256
    rec = layouts.pack_tiled(formats.iq3_pack_rows(synth.iq3xxs_raw(np.random.default_rng(1), 16, kdim), kdim), kdim)
    rec[0, 0, 2] ^= 0x80            # slot 0, chunk 0: bit 23 of the stream = i1's parity bit
    with pytest.raises(ValueError):
        layouts.unpack_tiled(rec, kdim, 16)


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


@pytest.mark.parametrize("rows,kdim", [(16, 256), (32, 512), (48, 2048)])
def test_iq4_tiled_slab_inverts(rows, kdim):
    raw = synth.iq4xs_raw(np.random.default_rng(rows + kdim), rows, kdim)
    rec = layouts.pack_iq4_tiled(raw, kdim)
    assert rec.shape == (rows // 16, kdim // 256, 2176)
    assert np.array_equal(layouts.unpack_iq4_tiled(rec, kdim), raw)


def test_iq4_tiled_slab_places_bytes_by_hand():
    """Bytes placed by the record rules written out: header of row r at 8r, quant byte j of
    sub-block ib of row r at 128 + 1024 (ib // 4) + 16 (16 (ib % 4) + r) + j."""
    kdim = 512
    raw = synth.iq4xs_raw(np.random.default_rng(3), 32, kdim)
    rec = layouts.pack_iq4_tiled(raw, kdim)
    for t, b, r in [(0, 0, 0), (0, 1, 5), (1, 0, 15), (1, 1, 9)]:
        row = raw[16 * t + r, 136 * b:136 * (b + 1)]
        assert np.array_equal(rec[t, b, 8 * r:8 * r + 8], row[:8])
        for ib in range(8):
            o = 128 + 1024 * (ib // 4) + 16 * (16 * (ib % 4) + r)
            assert np.array_equal(rec[t, b, o:o + 16], row[8 + 16 * ib:8 + 16 * ib + 16])


@pytest.mark.parametrize("rows,kdim", [(16, 256), (32, 2048), (48, 512)])
def test_ckpt_tiled_slabs_invert(rows, kdim):
    rng = np.random.default_rng(rows + 7 * kdim)
    a = rng.integers(0, 256, (rows, 110 * (kdim // 256)), dtype=np.uint8)
    rec = layouts.pack_iq3s_tiled(a, kdim)
    assert rec.shape == (rows // 16, kdim // 256, 1760)
    assert np.array_equal(layouts.unpack_iq3s_tiled(rec, kdim), a)
    b = rng.integers(0, 256, (rows, 210 * (kdim // 256)), dtype=np.uint8)
    rec = layouts.pack_q6k_tiled(b, kdim)
    assert rec.shape == (rows // 16, kdim // 256, 3360)
    assert np.array_equal(layouts.unpack_q6k_tiled(rec, kdim), b)


def test_ckpt_tiled_slabs_place_bytes_by_hand():
    """Bytes placed by the record rules written out, lane l = 16 kq + col.  IQ3_S: index byte j of
    lane l at 16 l + j (block byte 2 + 16 kq + j), sign byte j at 1024 + 8 l + j (74 + 8 kq + j),
    high-bit byte j at 1536 + 2 l + j (66 + 2 kq + j), scale byte at 1664 + l (106 + kq), d byte j at
    1728 + 2 col + j.  Q6_K: low byte j at 32 l + j (32 kq + j), high byte j of half h at
    2048 + 32 (16 h + col) + j (128 + 32 h + j), scale slot s at 3072 + 4 l + s (192 + 8 (kq / 2) +
    2 (kq % 2) + (0, 1, 4, 5)[s]), d byte j at 3328 + 2 col + j (208 + j)."""
    rng = np.random.default_rng(9)
    kdim = 512
    a = rng.integers(0, 256, (32, 220), dtype=np.uint8)
    b = rng.integers(0, 256, (32, 420), dtype=np.uint8)
    ra, rb = layouts.pack_iq3s_tiled(a, kdim), layouts.pack_q6k_tiled(b, kdim)
    for t, blk, col, kq in [(0, 0, 0, 0), (0, 1, 5, 3), (1, 0, 15, 1), (1, 1, 9, 2)]:
        l, ra_, rb_ = 16 * kq + col, a[16 * t + col, 110 * blk:], b[16 * t + col, 210 * blk:]
        rec, req = ra[t, blk], rb[t, blk]
        for j in range(16):
            assert rec[16 * l + j] == ra_[2 + 16 * kq + j]
        for j in range(8):
            assert rec[1024 + 8 * l + j] == ra_[74 + 8 * kq + j]
        for j in range(2):
            assert rec[1536 + 2 * l + j] == ra_[66 + 2 * kq + j]
            assert rec[1728 + 2 * col + j] == ra_[j]
            assert req[3328 + 2 * col + j] == rb_[208 + j]
        assert rec[1664 + l] == ra_[106 + kq]
        for j in range(32):
            assert req[32 * l + j] == rb_[32 * kq + j]
            for h in range(2):
                assert req[2048 + 32 * (16 * h + col) + j] == rb_[128 + 32 * h + j]
        for s_, off in enumerate((0, 1, 4, 5)):
            assert req[3072 + 4 * l + s_] == rb_[192 + 8 * (kq // 2) + 2 * (kq % 2) + off]
