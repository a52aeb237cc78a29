"""GGUF v3 checkpoints into the kernels' layouts.

``parse_gguf`` returns what the reference's reader does (/root/reference/engine/engine0.py:25-51):
``(data_start, {name: (ggml_type, dims, offset)})`` with dims in GGUF order (dims[0] is the
row length), parsed by libtlx's ``tlx_gguf_parse`` from the head of the file (read in growing
pieces until the tensor table fits).  ``tensor_bytes`` memory-maps one tensor's bytes
(``read_raw``, engine0.py:57-61) and ``to_device`` copies them to the GPU, where the device
repackers (``ops.pack_iq3_rows``, ``ops.pack_q6_pad``, ``ops.pack_w7``) turn them into the
layouts the kernels read.
"""
import ctypes
import os

import numpy as np

from . import _lib


class GGUFTensor(ctypes.Structure):
    """``tlx_gguf_tensor`` of include/tlx.h."""
    _fields_ = [("name", ctypes.c_char * 128), ("type", ctypes.c_int32), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


def _parse_head(head):
    L = _lib.lib()
    ds, nt = ctypes.c_uint64(), ctypes.c_int64()
    rc = L.tlx_gguf_parse(head, len(head), ctypes.byref(ds), ctypes.byref(nt), None, 0)
    if rc != _lib.TLX_OK:
        return rc, None, None
    table = (GGUFTensor * max(nt.value, 1))()
    _lib.call("tlx_gguf_parse", head, len(head), ctypes.byref(ds), ctypes.byref(nt), table, nt.value)
    return rc, ds.value, list(table)[:nt.value]


def parse_gguf(path, head_bytes=1 << 20):
    """-> (data_start, {name: (type, dims, offset)}, {name: nbytes})."""
    size = os.path.getsize(path)
    n = min(head_bytes, size)
    while True:
        with open(path, "rb") as f:
            head = f.read(n)
        rc, ds, table = _parse_head(head)
        if rc == _lib.TLX_E_TRUNC and n < size:
            n = min(size, 4 * n)
            continue
        if rc != _lib.TLX_OK:
            raise _lib.TlxError("tlx_gguf_parse", rc, _lib.lib().tlx_strerror(rc).decode())
        break
    infos = {t.name.decode(): (int(t.type), [int(d) for d in t.dims[:t.n_dims]], int(t.offset)) for t in table}
    sizes = {t.name.decode(): int(t.nbytes) for t in table}
    return ds, infos, sizes


def tensor_bytes(path, data_start, info, nbytes):
    """The tensor's bytes as a read-only uint8 memory map."""
    return np.memmap(path, dtype=np.uint8, mode="r", offset=data_start + info[2], shape=(nbytes,))


def to_device(path, data_start, info, nbytes, device="cuda"):
    """Copy one tensor's bytes to a uint8 device tensor."""
    import torch
    return torch.from_numpy(np.array(tensor_bytes(path, data_start, info, nbytes))).to(device)
