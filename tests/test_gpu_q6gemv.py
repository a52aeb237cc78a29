"""Q6_K decode GEMV with fp16 activations (the q-branch of aq6k8 / a_qkv_q6 and the Q6_K head)
against the oracle.

Tolerance: norm-wise relative error <= 1e-3 per output row against the exact (float64) product
of the dequantized Q6_K weights and the fp16 activations, rounded to fp16 as the kernel's
output is.  Shapes are chosen so tiles split between waves, waves with no work, tail tiles and
the row-group path (activations larger than the LDS budget) all run.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _q6(rng, rows, kdim, layout, dev):
    raw = synth.q6k_raw(rng, rows, kdim)
    w = raw if layout == LAYOUT_RAW else formats.q6_pad_rows(raw, kdim)
    return raw, torch.from_numpy(np.ascontiguousarray(w)).to(dev)


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


def _run(gpu, M, N, K, layout, seed):
    rng = np.random.default_rng(seed)
    raw, w = _q6(rng, N, K, layout, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.full((M, N), -3.0, dtype=torch.float16, device=gpu)
    ops.q6k_gemv16(w, torch.from_numpy(x).to(gpu), out, layout)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(quants.dequant_q6k(raw, K), x)
    return out, ref, w, x


@pytest.mark.parametrize("layout", [LAYOUT_RAW, LAYOUT_PACKED])
@pytest.mark.parametrize("M", [1, 4, 11, 16])
def test_q6k_gemv16_parity(gpu, M, layout):
    print(f"[case] q6k_gemv16 M={M} N=300 K=5120 layout={layout}", flush=True)
    out, ref, _, _ = _run(gpu, M, 300, 5120, layout, 100 + M)
    err = _rows_err(out.cpu().numpy(), ref)
    print(f"[q6k_gemv16 M={M} layout={layout}] max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("N,K", [(48, 5120), (640, 512), (9600, 1024), (37, 768), (16, 256)])
def test_q6k_gemv16_work_splits(gpu, N, K):
    """Tiles split across waves (48x5120), waves without items (640x512, 16x256), several tiles
    per workgroup (9600x1024) and an odd block count with a tail tile (37x768)."""
    print(f"[case] q6k_gemv16 split N={N} K={K}", flush=True)
    out, ref, _, _ = _run(gpu, 5, N, K, LAYOUT_PACKED, N + K)
    assert _rows_err(out.cpu().numpy(), ref) <= TOL


def test_q6k_gemv16_rows_invariant_and_deterministic(gpu):
    """Row r of an M=11 call equals an M=1 call on activation row r bit for bit; repeated calls
    agree bit for bit."""
    print("[case] q6k_gemv16 invariance", flush=True)
    out, _, w, x = _run(gpu, 11, 200, 5120, LAYOUT_RAW, 7)
    xt = torch.from_numpy(x).to(gpu)
    again = torch.empty_like(out)
    ops.q6k_gemv16(w, xt, again, LAYOUT_RAW)
    one = torch.empty(1, 200, dtype=torch.float16, device=gpu)
    for r in range(11):
        ops.q6k_gemv16(w, xt[r:r + 1].contiguous(), one, LAYOUT_RAW)
        assert torch.equal(one[0].view(torch.int16), out[r].view(torch.int16)), r
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_q6k_gemv16_q_projection_size_sampled_rows(gpu):
    """The attention q shape of config 3 (12288 x 5120, padded blocks) at M=11; 256 seeded rows
    checked against the oracle."""
    print("[case] q6k_gemv16 12288x5120 M=11", flush=True)
    rng = synth.config_rng(3)
    N, K, M = 12288, 5120, 11
    raw, w = _q6(rng, N, K, LAYOUT_PACKED, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.q6k_gemv16(w, torch.from_numpy(x).to(gpu), out, LAYOUT_PACKED)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(3).choice(N, 256, replace=False))
    _, ref = gemv.gemv16_ref(quants.dequant_q6k(raw[rows], K), x)
    err = _rows_err(out.cpu().numpy()[:, rows], ref)
    print(f"[q6k_gemv16 12288] sampled max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M", [1, 11])
def test_aq6k8_parity(gpu, M):
    print(f"[case] aq6k8 M={M}", flush=True)
    rng = np.random.default_rng(300 + M)
    K, Nq, Nk, Nv = 5120, 768, 128, 112
    rawq, wq = _q6(rng, Nq, K, LAYOUT_PACKED, gpu)
    pk = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, Nk, K), K)
    pv = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, Nv, K), K)
    x = synth.activations_f16(rng, M, K)
    outs = [torch.empty(M, n, dtype=torch.float16, device=gpu) for n in (Nq, Nk, Nv)]
    ops.aq6k8(wq, torch.from_numpy(pk).to(gpu), torch.from_numpy(pv).to(gpu),
              formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), *outs)
    torch.cuda.synchronize()
    refs = [gemv.gemv16_ref(quants.dequant_q6k(rawq, K), x)[1],
            gemv.gemv16_ref(quants.dequant_iq3xxs_packed(pk, K), x)[1],
            gemv.gemv16_ref(quants.dequant_iq3xxs_packed(pv, K), x)[1]]
    for o, ref in zip(outs, refs):
        assert _rows_err(o.cpu().numpy(), ref) <= TOL


def test_q6k_gemv16_rejects_bad_arguments(gpu):
    print("[case] q6k_gemv16 bad args", flush=True)
    rng = np.random.default_rng(1)
    _, w = _q6(rng, 32, 512, LAYOUT_RAW, gpu)
    x = torch.zeros(17, 512, dtype=torch.float16, device=gpu)
    out = torch.empty(17, 32, dtype=torch.float16, device=gpu)
    with pytest.raises(TlxError):          # M = 17 > TLX_MAX_M
        ops.q6k_gemv16(w, x, out, LAYOUT_RAW)
    wide = torch.zeros(32, 212 * 2, dtype=torch.uint8, device=gpu)
    with pytest.raises(TlxError):          # unknown layout
        ops.q6k_gemv16(wide, x[:2], out[:2], 5)
