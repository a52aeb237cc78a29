"""GPU prefill dequant-GEMMs (pf_gemm3 family) against the oracle.

Tolerance: norm-wise relative error <= 1e-3 per output row against the exact float64 product
of the fp16-dequantized weights and the fp16 activations, followed by the kernel's epilogue
(the RES epilogue is checked on out32 - res as well, so a large residual cannot hide an error
in the product).  Full-size launches (config 4, M = 2048) are checked on seeded weight-row
samples over every activation row.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _iq3(rng, rows, kdim, dev):
    """Packed rows (what the oracle dequantizes) and their packed7 units on the GPU."""
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, rows, kdim), kdim)
    return packed, torch.from_numpy(formats.iq3_pack7(packed, kdim)).to(dev)


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


@pytest.mark.parametrize("M,N,K", [(256, 128, 512), (512, 256, 1024), (256, 384, 5120)])
def test_pfg3_ffn_parity(gpu, M, N, K):
    print(f"[case] pfg3_ffn M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(4)
    pg, wg = _iq3(rng, N, K, gpu)
    pu, wu = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.pfg3_ffn(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    _, _, ref = gemv.pf_ffn_ref(quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K), x)
    err = _rows_err(out.cpu().numpy(), ref)
    print(f"[pfg3_ffn M={M} N={N} K={K}] max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (512, 512, 2048), (256, 256, 6144), (256, 256, 768)])
def test_pfg3_iq3o_parity(gpu, M, N, K):
    print(f"[case] pfg3_iq3o M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(4)
    pw, w = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.pfg3_iq3o(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    _, ref = gemv.pf_o_ref(quants.dequant_iq3xxs_packed(pw, K), x)
    err = _rows_err(out.cpu().numpy(), ref)
    print(f"[pfg3_iq3o M={M} N={N} K={K}] max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (512, 512, 3072)])
def test_pfg3_iq3d_parity(gpu, M, N, K):
    print(f"[case] pfg3_iq3d M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(4)
    pw, w = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    res = rng.standard_normal((M, N)).astype(np.float32)
    out = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.pfg3_iq3d(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), torch.from_numpy(res).to(gpu), out)
    torch.cuda.synchronize()
    acc, ref = gemv.pf_res_ref(quants.dequant_iq3xxs_packed(pw, K), x, res)
    y = out.cpu().numpy()
    err = _rows_err(y, ref)
    err_acc = _rows_err(y.astype(np.float64) - res, acc)
    print(f"[pfg3_iq3d M={M} N={N} K={K}] rel-err out {err:.3e}, product {err_acc:.3e}")
    assert err <= TOL and err_acc <= TOL


def test_pfg3_ffn_full_size_sampled_rows(gpu):
    """Config 4 gate+up: M=2048, K=5120, N=17408; 256 seeded weight rows over all 2048 rows."""
    print("[case] pfg3_ffn full-size M=2048", flush=True)
    rng = synth.config_rng(4)
    M, N, K = 2048, 17408, 5120
    pg, wg = _iq3(rng, N, K, gpu)
    pu, wu = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.pfg3_ffn(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(3).choice(N, 256, replace=False))
    _, _, ref = gemv.pf_ffn_ref(quants.dequant_iq3xxs_packed(pg[cols], K),
                                quants.dequant_iq3xxs_packed(pu[cols], K), x)
    y = out.cpu().numpy()[:, cols]
    err = _rows_err(y, ref)
    print(f"[pfg3_ffn full] max row rel-err {err:.3e}")
    assert err <= TOL
    assert np.isfinite(out.float().cpu().numpy()).all()


def test_pfg3_iq3d_full_size_sampled_rows(gpu):
    """Config 4 down: M=2048, K=17408, N=5120; 128 seeded weight rows over all 2048 rows."""
    print("[case] pfg3_iq3d full-size M=2048", flush=True)
    rng = synth.config_rng(4)
    M, N, K = 2048, 5120, 17408
    pw, w = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    res = rng.standard_normal((M, N)).astype(np.float32)
    out = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.pfg3_iq3d(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), torch.from_numpy(res).to(gpu), out)
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(5).choice(N, 128, replace=False))
    acc, ref = gemv.pf_res_ref(quants.dequant_iq3xxs_packed(pw[cols], K), x, res[:, cols])
    y = out.cpu().numpy()[:, cols]
    err = _rows_err(y.astype(np.float64) - res[:, cols], acc)
    print(f"[pfg3_iq3d full] max row rel-err (product) {err:.3e}")
    assert err <= TOL


def test_pfg3_deterministic(gpu):
    """Two launches on the same inputs give identical bits (fixed k order, no atomics)."""
    print("[case] pfg3_iq3o determinism", flush=True)
    rng = synth.config_rng(4)
    M, N, K = 512, 512, 2048
    _, w = _iq3(rng, N, K, gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    g = formats.gridf_tensor(gpu)
    a = torch.empty(M, N, dtype=torch.float16, device=gpu)
    b = torch.empty_like(a)
    ops.pfg3_iq3o(w, g, x, a)
    ops.pfg3_iq3o(w, g, x, b)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_pfg3_bad_arguments_raise(gpu):
    print("[case] pfg3 argument checks", flush=True)
    rng = synth.config_rng(4)
    g = formats.gridf_tensor(gpu)
    _, w = _iq3(rng, 256, 512, gpu)
    x = torch.zeros(256, 512, dtype=torch.float16, device=gpu)
    out = torch.empty(256, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(TlxError):   # M not a multiple of 256
        ops.pfg3_iq3o(w, g, x[:128], out[:128])
    with pytest.raises(TlxError):   # only the packed7 layout is accepted
        ops.pfg3_iq3o(w, g, x, out, layout=LAYOUT_PACKED)
    with pytest.raises(TlxError):   # K not a multiple of 128
        ops.pfg3_iq3o(w, g, torch.zeros(256, 320, dtype=torch.float16, device=gpu), out)
    with pytest.raises(TlxError):   # N not a multiple of the 256-row tile
        ops.pfg3_iq3o(w, g, x, torch.empty(256, 128, dtype=torch.float16, device=gpu))
