"""GGUF v3 tensor table through libtlx (tlx_gguf_parse, host only) against the reader
restatement and the independently written fixture writer of oracle/gguf.py."""
import numpy as np
import pytest

from oracle import gguf as og
from thunderllamax_amd import gguf, synth
from thunderllamax_amd._lib import TlxError


def _file(tmp_path, name="m.gguf"):
    rng = synth.config_rng(2)
    kvs = [("general.architecture", 8, "qwen35"), ("general.alignment", 4, 32), ("x.u8", 0, 7), ("x.i8", 1, -3),
           ("x.u16", 2, 65535), ("x.i16", 3, -2), ("x.u32", 4, 123456), ("x.i32", 5, -7), ("x.f32", 6, 1.5),
           ("x.bool", 7, True), ("x.u64", 10, 2 ** 40), ("x.i64", 11, -2 ** 40), ("x.f64", 12, 0.25),
           ("tokenizer.ggml.tokens", 9, (8, ["tok%d" % i for i in range(3000)])),
           ("tokenizer.ggml.scores", 9, (6, [0.5] * 3000)),
           ("x.nested", 9, (9, [(4, [1, 2, 3]), (8, ["a", "bc"])]))]
    tensors = [
        ("blk.0.ffn_gate.weight", 18, [512, 24], synth.iq3xxs_raw(rng, 24, 512).tobytes()),
        ("output_norm.weight", 0, [512], rng.standard_normal(512).astype("<f4").tobytes()),
        ("blk.3.attn_q.weight", 14, [256, 8], synth.q6k_raw(rng, 8, 256).tobytes()),
        ("token_embd.weight", 1, [16, 5], rng.standard_normal(80).astype("<f2").tobytes()),
        ("blk.1.ffn_down.weight", 13, [256, 3], synth.k4_raw(rng, 3, 256, True).tobytes()),
        ("blk.0.ssm_a", 0, [4, 2, 2], np.arange(16, dtype="<f4").tobytes()),
    ]
    path = tmp_path / name
    ds, infos = og.write_gguf(str(path), kvs, tensors)
    return path, ds, infos, tensors


def test_parse_matches_writer_and_reference_reader(tmp_path):
    path, ds, infos, tensors = _file(tmp_path)
    got_ds, got, sizes = gguf.parse_gguf(str(path))
    ref_ds, ref = og.parse_gguf_ref(path.read_bytes())
    assert got_ds == ds == ref_ds
    assert got == infos == ref
    for name, t, dims, data in tensors:
        assert sizes[name] == og.tnbytes_ref(int(np.prod(dims)), t) == len(data)
        assert bytes(gguf.tensor_bytes(str(path), got_ds, got[name], sizes[name])) == data


def test_parse_grows_the_head_read(tmp_path):
    path, ds, infos, _ = _file(tmp_path)
    got_ds, got, _ = gguf.parse_gguf(str(path), head_bytes=64)   # the tokenizer array alone is ~30 KB
    assert got_ds == ds and got == infos


def test_parse_rejects_bad_files(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 64)
    with pytest.raises(TlxError):
        gguf.parse_gguf(str(bad))
    trunc = tmp_path / "trunc.gguf"
    path, _, _, _ = _file(tmp_path)
    trunc.write_bytes(path.read_bytes()[:40000])   # ends inside the key/value section
    with pytest.raises(TlxError):
        gguf.parse_gguf(str(trunc))
    unknown = tmp_path / "unknown.gguf"
    unknown.write_bytes(b"GGUF" + np.array([3], "<i4").tobytes() + np.array([0, 1], "<i8").tobytes()
                        + np.array([1], "<u8").tobytes() + b"k" + np.array([99], "<i4").tobytes() + b"\0" * 16)
    with pytest.raises(TlxError):
        gguf.parse_gguf(str(unknown))


def test_type_sizes():
    for t, (a, b) in og.QUANT.items():
        assert og.tnbytes_ref(4 * a, t) == 4 * b
    assert og.tnbytes_ref(10, 0) == 40 and og.tnbytes_ref(10, 30) == 20 and og.tnbytes_ref(10, 99) == 0
