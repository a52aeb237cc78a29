"""GPU RMSNorm producers against oracle/norm.py (hh bit-exact; fp16 outputs equal to the
rounded float64 ideal or one ulp away, with at most 1% of elements off it), and the fused
hh{M} + ffn8 entry point bit-identical to the two calls it replaces."""
import numpy as np
import pytest
import torch

from oracle import norm
from thunderllamax_amd import formats, ops, synth

pytestmark = pytest.mark.gpu


def _x(rng, M, D, scale=1.0):
    return (rng.standard_normal((M, D)) * scale).astype(np.float32)


@pytest.mark.parametrize("M,D", [(1, 5120), (11, 5120), (300, 2048), (4, 64)])
def test_rms_f16(gpu, M, D):
    print(f"[case] rms_f16 M={M} D={D}", flush=True)
    rng = np.random.default_rng(M + D)
    x, nw = _x(rng, M, D, 3.0), (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    x[0, :8] = 0.0
    xh = torch.empty(M, D, dtype=torch.float16, device=gpu)
    ops.rms_f16(torch.from_numpy(x).to(gpu), torch.from_numpy(nw).to(gpu), xh)
    torch.cuda.synchronize()
    ideal, r16 = norm.rms_ref(x, nw)
    got = xh.cpu().numpy()
    assert norm.within_one_ulp(got, ideal).all()
    assert (got != r16).mean() <= 0.01


@pytest.mark.parametrize("M,D", [(1, 5120), (11, 5120), (2048, 5120)])
def test_add_rms_f16(gpu, M, D):
    print(f"[case] add_rms_f16 M={M} D={D}", flush=True)
    rng = np.random.default_rng(7 + M)
    x, nw = _x(rng, M, D), (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    a = rng.standard_normal((M, D)).astype(np.float16)
    hh = torch.empty(M, D, dtype=torch.float32, device=gpu)
    hhx = torch.empty(M, D, dtype=torch.float16, device=gpu)
    ops.add_rms_f16(torch.from_numpy(x).to(gpu), torch.from_numpy(a).to(gpu), torch.from_numpy(nw).to(gpu), hh, hhx)
    torch.cuda.synchronize()
    rhh, ideal, r16 = norm.add_rms_ref(x, a, nw)
    assert np.array_equal(hh.cpu().numpy().view(np.uint32), rhh.view(np.uint32))
    got = hhx.cpu().numpy()
    assert norm.within_one_ulp(got, ideal).all()
    assert (got != r16).mean() <= 0.01


@pytest.mark.parametrize("M", [1, 4, 6, 11, 16])
def test_ffn8_hh_equals_separate_calls(gpu, M):
    print(f"[case] ffn8_hh M={M}", flush=True)
    K, N = 5120, 256
    rng = synth.config_rng(2)
    wg = torch.from_numpy(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)).to(gpu)
    wu = torch.from_numpy(formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)).to(gpu)
    gridf = formats.gridf_tensor(gpu)
    x = torch.from_numpy(_x(rng, M, K)).to(gpu)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(gpu)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(gpu)
    hh1, hhx1 = torch.empty(M, K, device=gpu), torch.empty(M, K, dtype=torch.float16, device=gpu)
    g1 = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.add_rms_f16(x, a, nw, hh1, hhx1)
    ops.ffn8(wg, wu, gridf, hhx1, g1)
    hh2, hhx2 = torch.empty_like(hh1), torch.empty_like(hhx1)
    g2 = torch.empty_like(g1)
    ops.ffn8_hh(wg, wu, gridf, x, a, nw, hh2, hhx2, g2)
    torch.cuda.synchronize()
    assert torch.equal(hh1, hh2) and torch.equal(hhx1, hhx2)
    assert torch.equal(g1.view(torch.int16), g2.view(torch.int16))
