"""Lookup tables of the GGUF "i-quant" formats, vendored as data.

The reference never ships these tables: it reads them at run time from
``tinygrad.runtime.autogen.ggml_common`` (/root/reference/engine/engine0.py:108-112,
/root/reference/engine/pack_w4.py:30-37, /root/reference/engine/mm/MM_P0_d2_repack.py:65-73),
which mirrors llama.cpp's ``ggml-common.h`` (MIT licence).  Neither package is present in
this build environment, so the two tables below are transcribed from llama.cpp's published
``ggml-common.h`` (``iq3xxs_grid`` and ``kvalues_iq4nl``).  They are format constants: a
different table would make every IQ3_XXS / IQ4_XS checkpoint decode to different numbers.

Invariants that pin the transcription (checked by ``tests/test_tables.py``):

* ``IQ3XXS_GRID``: 256 distinct uint32 words in strictly ascending order; every byte is one
  of the eight IQ3_XXS magnitude levels {4, 12, 20, 28, 36, 44, 52, 62}
  (/root/reference/engine/p8_w4ffn7.cu:6-7, /root/reference/lineage/a3a/a3a_bench.py:25).
  The ascending order follows from the word being the little-endian packing of four 3-bit
  level codes taken in lexicographic order.
* ``KVALUES_IQ4NL``: 16 strictly increasing int8 values.
* SHA-256 of the little-endian byte image of each table equals the committed digests below.
"""
import hashlib

import numpy as np

IQ3XXS_LEVELS = (4, 12, 20, 28, 36, 44, 52, 62)

IQ3XXS_GRID = np.array([
    0x04040404, 0x04040414, 0x04040424, 0x04040c0c, 0x04040c1c, 0x04040c3e, 0x04041404, 0x04041414,
    0x04041c0c, 0x04042414, 0x04043e1c, 0x04043e2c, 0x040c040c, 0x040c041c, 0x040c0c04, 0x040c0c14,
    0x040c140c, 0x040c142c, 0x040c1c04, 0x040c1c14, 0x040c240c, 0x040c2c24, 0x040c3e04, 0x04140404,
    0x04140414, 0x04140424, 0x04140c0c, 0x04141404, 0x04141414, 0x04141c0c, 0x04141c1c, 0x04141c3e,
    0x04142c0c, 0x04142c3e, 0x04143e2c, 0x041c040c, 0x041c043e, 0x041c0c04, 0x041c0c14, 0x041c142c,
    0x041c3e04, 0x04240c1c, 0x04241c3e, 0x04242424, 0x04242c3e, 0x04243e1c, 0x04243e2c, 0x042c040c,
    0x042c043e, 0x042c1c14, 0x042c2c14, 0x04341c2c, 0x04343424, 0x043e0c04, 0x043e0c24, 0x043e0c34,
    0x043e241c, 0x043e340c, 0x0c04040c, 0x0c04041c, 0x0c040c04, 0x0c040c14, 0x0c04140c, 0x0c04141c,
    0x0c041c04, 0x0c041c14, 0x0c041c24, 0x0c04243e, 0x0c042c04, 0x0c0c0404, 0x0c0c0414, 0x0c0c0c0c,
    0x0c0c1404, 0x0c0c1414, 0x0c14040c, 0x0c14041c, 0x0c140c04, 0x0c140c14, 0x0c14140c, 0x0c141c04,
    0x0c143e14, 0x0c1c0404, 0x0c1c0414, 0x0c1c1404, 0x0c1c1c0c, 0x0c1c2434, 0x0c1c3434, 0x0c24040c,
    0x0c24042c, 0x0c242c04, 0x0c2c1404, 0x0c2c1424, 0x0c2c2434, 0x0c2c3e0c, 0x0c34042c, 0x0c3e1414,
    0x0c3e2404, 0x14040404, 0x14040414, 0x14040c0c, 0x14040c1c, 0x14041404, 0x14041414, 0x14041434,
    0x14041c0c, 0x14042414, 0x140c040c, 0x140c041c, 0x140c042c, 0x140c0c04, 0x140c0c14, 0x140c140c,
    0x140c1c04, 0x140c341c, 0x140c343e, 0x140c3e04, 0x14140404, 0x14140414, 0x14140c0c, 0x14140c3e,
    0x14141404, 0x14141414, 0x14141c3e, 0x14142404, 0x14142c2c, 0x141c040c, 0x141c0c04, 0x141c0c24,
    0x141c3e04, 0x141c3e24, 0x14241c2c, 0x14242c1c, 0x142c041c, 0x142c143e, 0x142c240c, 0x142c3e24,
    0x143e040c, 0x143e041c, 0x143e0c34, 0x143e242c, 0x1c04040c, 0x1c040c04, 0x1c040c14, 0x1c04140c,
    0x1c04141c, 0x1c042c04, 0x1c04342c, 0x1c043e14, 0x1c0c0404, 0x1c0c0414, 0x1c0c1404, 0x1c0c1c0c,
    0x1c0c2424, 0x1c0c2434, 0x1c14040c, 0x1c14041c, 0x1c140c04, 0x1c14142c, 0x1c142c14, 0x1c143e14,
    0x1c1c0c0c, 0x1c1c1c1c, 0x1c241c04, 0x1c24243e, 0x1c243e14, 0x1c2c0404, 0x1c2c0434, 0x1c2c1414,
    0x1c2c2c2c, 0x1c340c24, 0x1c341c34, 0x1c34341c, 0x1c3e1c1c, 0x1c3e3404, 0x24040424, 0x24040c3e,
    0x24041c2c, 0x24041c3e, 0x24042c1c, 0x24042c3e, 0x240c3e24, 0x24141404, 0x24141c3e, 0x24142404,
    0x24143404, 0x24143434, 0x241c043e, 0x241c242c, 0x24240424, 0x24242c0c, 0x24243424, 0x242c142c,
    0x242c241c, 0x242c3e04, 0x243e042c, 0x243e0c04, 0x243e0c14, 0x243e1c04, 0x2c040c14, 0x2c04240c,
    0x2c043e04, 0x2c0c0404, 0x2c0c0434, 0x2c0c1434, 0x2c0c2c2c, 0x2c140c24, 0x2c141c14, 0x2c143e14,
    0x2c1c0414, 0x2c1c2c1c, 0x2c240c04, 0x2c24141c, 0x2c24143e, 0x2c243e14, 0x2c2c0414, 0x2c2c1c0c,
    0x2c342c04, 0x2c3e1424, 0x2c3e2414, 0x34041424, 0x34042424, 0x34042434, 0x34043424, 0x340c140c,
    0x340c340c, 0x34140c3e, 0x34143424, 0x341c1c04, 0x341c1c34, 0x34242424, 0x342c042c, 0x342c2c14,
    0x34341c1c, 0x343e041c, 0x343e140c, 0x3e04041c, 0x3e04042c, 0x3e04043e, 0x3e040c04, 0x3e041c14,
    0x3e042c14, 0x3e0c1434, 0x3e0c2404, 0x3e140c14, 0x3e14242c, 0x3e142c14, 0x3e1c0404, 0x3e1c0c2c,
    0x3e1c1c1c, 0x3e1c3404, 0x3e24140c, 0x3e24240c, 0x3e2c0404, 0x3e2c0414, 0x3e2c1424, 0x3e341c04,
], dtype=np.uint32)

KVALUES_IQ4NL = np.array(
    [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int8)


def table_sha256(arr: np.ndarray) -> str:
    """SHA-256 of the little-endian byte image of a table."""
    return hashlib.sha256(np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes()).hexdigest()


def iq3xxs_gridf() -> np.ndarray:
    """float32[1024]: grid word w expanded to its 4 little-endian bytes, in order.

    This is the ``gridf`` device buffer every IQ3_XXS kernel of the reference takes as an
    argument (/root/reference/engine/engine0.py:108-112).
    """
    b = IQ3XXS_GRID.astype("<u4").view(np.uint8)
    return b.astype(np.float32).copy()


def iq3xxs_lut8() -> np.ndarray:
    """int8[1024]: the linearized IQ3_XXS codebook of the W4A8 branch, level of grid byte j of
    grid word g at 4g + j: clip(rint(byte / 4.0507), 0, 15)
    (/root/reference/engine/p8_w4ffn7_test.py:44-46; the 8 magnitudes 4..62 map to 1, 3, ..., 15).
    """
    b = IQ3XXS_GRID.astype("<u4").view(np.uint8).astype(np.float32)
    return np.clip(np.rint(b / np.float32(4.0507)), 0, 15).astype(np.int8)


def iq4nl_f32() -> np.ndarray:
    """float32[16]: the IQ4_NL non-linear levels (/root/reference/engine/mm/MM_P2_ports.py:112-114)."""
    return KVALUES_IQ4NL.astype(np.float32)
