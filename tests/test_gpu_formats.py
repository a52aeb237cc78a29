"""Device repackers against the layout restatements of oracle/layouts.py (byte-identical), and a
synthetic GGUF checkpoint run end to end: parse, copy to the GPU, repack there, multiply."""
import numpy as np
import pytest
import torch

from oracle import gemv, gguf as og, layouts, quants
from thunderllamax_amd import formats, gguf, ops, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K", [(24, 512), (40, 5120), (1, 256)])
def test_pack_iq3_rows(gpu, N, K):
    print(f"[case] pack_iq3_rows N={N} K={K}", flush=True)
    raw = synth.iq3xxs_raw(synth.config_rng(2), N, K)
    d = torch.from_numpy(raw.reshape(-1)).to(gpu)
    out = torch.empty_like(d)
    ops.pack_iq3_rows(d, out, N, K)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(N, -1)
    assert np.array_equal(got, layouts.pack_iq3_w1c(raw.reshape(N, -1), K))
    assert np.array_equal(layouts.unpack_iq3_w1c(got, K), raw.reshape(N, -1))


@pytest.mark.parametrize("N,K", [(8, 256), (33, 5120)])
def test_pack_q6_pad(gpu, N, K):
    print(f"[case] pack_q6_pad N={N} K={K}", flush=True)
    raw = synth.q6k_raw(synth.config_rng(1), N, K)
    d = torch.from_numpy(raw.reshape(-1)).to(gpu)
    out = torch.empty(N * 212 * (K // 256), dtype=torch.uint8, device=gpu)
    ops.pack_q6_pad(d, out, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().reshape(N, -1), layouts.pack_q6_pad(raw.reshape(N, -1), K))


@pytest.mark.parametrize("N,K", [(8, 256), (64, 5120), (24, 17408)])
def test_pack_w7(gpu, N, K):
    print(f"[case] pack_w7 N={N} K={K}", flush=True)
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(synth.config_rng(4), N, K), K)
    d = torch.from_numpy(packed.reshape(-1)).to(gpu)
    out = torch.empty(N * K // 2, dtype=torch.uint8, device=gpu)
    ops.pack_w7(d, out, N, K)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got, layouts.pack_w7(packed, K).reshape(-1))
    assert np.array_equal(layouts.unpack_w7(got.reshape(N // 8, K // 128, 32, 16), K, N), packed)


def test_gguf_checkpoint_end_to_end(gpu, tmp_path):
    """IQ3_XXS gate/up tensors in a GGUF file -> device -> packed rows (ffn8) and packed7
    (pfg3_ffn); both products against the oracle on the file's raw bytes."""
    print("[case] gguf end to end", flush=True)
    rng = synth.config_rng(2)
    K, N = 512, 256
    rg, ru = synth.iq3xxs_raw(rng, N, K), synth.iq3xxs_raw(rng, N, K)
    path = str(tmp_path / "ffn.gguf")
    og.write_gguf(path, [("general.architecture", 8, "test")],
                  [("blk.0.ffn_gate.weight", 18, [K, N], rg.tobytes()), ("blk.0.ffn_up.weight", 18, [K, N], ru.tobytes())])
    ds, infos, sizes = gguf.parse_gguf(path)
    dev = {}
    for name in ("blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"):
        t, dims, _ = infos[name]
        assert t == 18 and dims == [K, N]
        raw = gguf.to_device(path, ds, infos[name], sizes[name], gpu)
        packed = torch.empty_like(raw)
        ops.pack_iq3_rows(raw, packed, N, K)
        p7 = torch.empty(N * K // 2, dtype=torch.uint8, device=gpu)
        ops.pack_w7(packed, p7, N, K)
        dev[name] = (packed, p7)
    wg = quants.dequant_iq3xxs_packed(layouts.pack_iq3_w1c(rg.reshape(N, -1), K), K)
    wu = quants.dequant_iq3xxs_packed(layouts.pack_iq3_w1c(ru.reshape(N, -1), K), K)
    gridf = formats.gridf_tensor(gpu)
    x = synth.activations_f16(rng, 256, K)
    xd = torch.from_numpy(x).to(gpu)
    out = torch.empty(256, N, dtype=torch.float16, device=gpu)
    ops.pfg3_ffn(dev["blk.0.ffn_gate.weight"][1], dev["blk.0.ffn_up.weight"][1], gridf, xd, out)
    g8 = torch.empty(4, N, dtype=torch.float16, device=gpu)
    ops.ffn8(dev["blk.0.ffn_gate.weight"][0], dev["blk.0.ffn_up.weight"][0], gridf, xd[:4].contiguous(), g8)
    torch.cuda.synchronize()
    _, _, ref = gemv.pf_ffn_ref(wg, wu, x)
    got = out.cpu().numpy()
    assert max(gemv.rel_err(got[m], ref[m]) for m in range(256)) <= 1e-3
    got8 = g8.cpu().numpy()
    assert max(gemv.rel_err(got8[m], ref[m]) for m in range(4)) <= 1e-3
