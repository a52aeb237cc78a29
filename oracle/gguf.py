"""GGUF v3 reader restatement and a writer for fixtures (test infrastructure only).

``parse_gguf_ref`` restates the reference's reader (/root/reference/engine/engine0.py:25-51):
magic ``GGUF``, int32 version, int64 tensor and key/value counts, the key/value section
skipped value by value (strings = u64 length + bytes, arrays = int32 element type + u64 count
+ elements, scalars by the size table of engine0.py:23), the tensor table (name, u32 n_dims,
u64 dims, int32 type, u64 offset), ``data_start`` = end of the table rounded up to 32.
``tnbytes_ref`` restates engine0.py:20-22,53-55.

``write_gguf`` writes a GGUF v3 file from the published format (header, key/values, tensor
infos with 32-aligned offsets, padding, data); it is written independently of the reader so
that the two check each other (tests/test_gguf.py), and it makes the synthetic checkpoints
the GPU tests load.
"""
import struct

import numpy as np

QUANT = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 18: (256, 98), 21: (256, 110), 22: (256, 82), 23: (256, 136), 39: (32, 17), 41: (128, 18)}
NATIVE = {0: 4, 1: 2, 24: 1, 25: 2, 26: 4, 27: 8, 28: 8, 30: 2}
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}


def tnbytes_ref(ne, t):
    if t in NATIVE:
        return NATIVE[t] * ne
    if t in QUANT:
        a, b = QUANT[t]
        return (ne // a) * b
    return 0


def parse_gguf_ref(buf):
    """bytes of the file (or its head) -> (data_start, {name: (type, dims, offset)})."""
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, buf, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0]

    def rs():
        nonlocal pos
        n = take("Q")
        s = bytes(buf[pos:pos + n]).decode()
        pos += n
        return s

    def rv(t):
        if t == 8:
            return rs()
        if t == 9:
            et = take("i")
            n = take("Q")
            return [rv(et) for _ in range(n)]
        return take(_SCALAR[t])

    assert bytes(buf[0:4]) == b"GGUF"
    pos = 4
    take("i")
    n_tensors = take("q")
    n_kv = take("q")
    for _ in range(n_kv):
        rs()
        rv(take("i"))
    infos = {}
    for _ in range(n_tensors):
        name = rs()
        nd = take("I")
        dims = [take("Q") for _ in range(nd)]
        t = take("i")
        off = take("Q")
        infos[name] = (t, dims, off)
    return (pos + 31) // 32 * 32, infos


def _w_str(out, s):
    b = s.encode()
    out += struct.pack("<Q", len(b)) + b


def _w_val(out, t, v):
    if t == 8:
        _w_str(out, v)
    elif t == 9:
        et, items = v
        out += struct.pack("<iQ", et, len(items))
        for it in items:
            _w_val(out, et, it)
    else:
        out += struct.pack("<" + _SCALAR[t], v)


def write_gguf(path, kvs, tensors, version=3):
    """kvs: [(key, type, value)] (arrays: type 9, value (elem_type, items)); tensors:
    [(name, ggml_type, dims, data bytes)].  -> (data_start, {name: (type, dims, offset)})."""
    out = bytearray(b"GGUF")
    out += struct.pack("<iqq", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        _w_str(out, key)
        out += struct.pack("<i", t)
        _w_val(out, t, v)
    infos, off = {}, 0
    for name, t, dims, data in tensors:
        _w_str(out, name)
        out += struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<Q", d)
        out += struct.pack("<iQ", t, off)
        infos[name] = (t, list(dims), off)
        off = (off + len(data) + 31) // 32 * 32
    data_start = (len(out) + 31) // 32 * 32
    out += b"\0" * (data_start - len(out))
    for name, t, dims, data in tensors:
        start = data_start + infos[name][2]
        out += b"\0" * (start - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return data_start, infos
