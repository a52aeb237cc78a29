"""Invariants of the vendored GGUF tables (their content is third-party data absent from
the reference; these checks pin the transcription)."""
import numpy as np

from thunderllamax_amd import tables

IQ3_SHA = "46e35f5a997efdee6c99ce57854c8a0d4f0ff8ca57e5e8a60c0793ea580acf5d"
IQ4_SHA = "61aa47540aa024b5d6ddaa839b84ffe59f3d5a349af5c6c7ffcb5e0474b46163"


def test_iq3xxs_grid_shape_order_levels():
    g = tables.IQ3XXS_GRID
    assert g.shape == (256,) and g.dtype == np.uint32
    assert np.all(g[1:] > g[:-1])                      # distinct, ascending
    levels = set(g.astype("<u4").view(np.uint8).tolist())
    assert levels == set(tables.IQ3XXS_LEVELS)         # /root/reference/engine/p8_w4ffn7.cu:6-7
    gf = tables.iq3xxs_gridf()
    assert gf.shape == (1024,) and gf.min() == 4 and gf.max() == 62   # a3a_bench.py:25


def test_iq3xxs_grid_first_entries_follow_level_codes():
    # word = little-endian bytes (level of code c is 4+8c for c<7, 62 for c=7); the first
    # entries are the smallest 4-code tuples in lexicographic order
    lv = np.array(tables.IQ3XXS_LEVELS)
    assert tables.IQ3XXS_GRID[0] == 0x04040404
    b = tables.IQ3XXS_GRID.astype("<u4").view(np.uint8).reshape(256, 4)
    codes = np.searchsorted(lv, b)
    assert np.all(lv[codes] == b)
    key = codes[:, 3] * 512 + codes[:, 2] * 64 + codes[:, 1] * 8 + codes[:, 0]
    assert np.all(key[1:] > key[:-1])


def test_kvalues_iq4nl():
    kv = tables.KVALUES_IQ4NL
    assert kv.shape == (16,) and kv.dtype == np.int8
    assert np.all(kv[1:] > kv[:-1])
    assert kv[0] == -127


def test_table_digests():
    assert tables.table_sha256(tables.IQ3XXS_GRID) == IQ3_SHA
    assert tables.table_sha256(tables.KVALUES_IQ4NL) == IQ4_SHA
