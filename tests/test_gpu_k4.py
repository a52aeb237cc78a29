"""Q4_K / Q5_K on the GPU against the oracle: dequantization bit for bit (fp32 and fp16
outputs), decode GEMVs (the Q4_K v rows of the fused attention projections and the Q5_K head)
within norm-wise relative error 1e-3 per output row of the exact float64 product of the
dequantized weights and the fp16 activations, rounded to fp16 as the kernel's output is."""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import ops, synth
from thunderllamax_amd._lib import TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


@pytest.mark.parametrize("five", [False, True])
@pytest.mark.parametrize("rows,kdim", [(7, 256), (33, 5120)])
def test_k4_dequant_bit_exact(gpu, five, rows, kdim):
    print(f"[case] k4 dequant five={five} rows={rows} k={kdim}", flush=True)
    raw = synth.k4_raw(np.random.default_rng(rows + kdim + five), rows, kdim, five)
    ref = (quants.dequant_q5k if five else quants.dequant_q4k)(raw, kdim)
    w = torch.from_numpy(raw).to(gpu)
    out32 = torch.empty(rows, kdim, dtype=torch.float32, device=gpu)
    out16 = torch.empty(rows, kdim, dtype=torch.float16, device=gpu)
    deq = ops.q5k_dequant if five else ops.q4k_dequant
    deq(w, out32, kdim)
    deq(w, out16, kdim)
    torch.cuda.synchronize()
    assert np.array_equal(out32.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))


def _gemv(gpu, five, M, N, K, seed):
    rng = np.random.default_rng(seed)
    raw = synth.k4_raw(rng, N, K, five)
    x = synth.activations_f16(rng, M, K)
    out = torch.full((M, N), -3.0, dtype=torch.float16, device=gpu)
    (ops.q5k_gemv16 if five else ops.q4k_gemv16)(torch.from_numpy(raw).to(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref((quants.dequant_q5k if five else quants.dequant_q4k)(raw, K), x)
    return _rows_err(out.cpu().numpy(), ref)


@pytest.mark.parametrize("five", [False, True])
@pytest.mark.parametrize("M", [1, 4, 11, 16])
def test_k4_gemv16_parity(gpu, five, M):
    print(f"[case] k4 gemv five={five} M={M} N=300 K=5120", flush=True)
    err = _gemv(gpu, five, M, 300, 5120, 200 + M + 20 * five)
    print(f"[k4 gemv five={five} M={M}] max row rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("five", [False, True])
@pytest.mark.parametrize("N,K", [(48, 5120), (640, 512), (37, 768), (16, 256)])
def test_k4_gemv16_work_splits(gpu, five, N, K):
    print(f"[case] k4 gemv split five={five} N={N} K={K}", flush=True)
    assert _gemv(gpu, five, 5, N, K, N + K + five) <= TOL


def test_head8_q5k_sampled_rows(gpu):
    """The head8 contract on a 24576-row Q5_K slice of the reference's 248320 x 5120 head at
    M=11; 256 seeded rows checked against the oracle."""
    print("[case] head8 24576x5120 M=11", flush=True)
    rng = np.random.default_rng(8)
    V, K, M = 24576, 5120, 11
    raw = synth.k4_raw(rng, V, K, True)
    x = synth.activations_f16(rng, M, K)
    logits = torch.empty(M, V, dtype=torch.float16, device=gpu)
    ops.head8(torch.from_numpy(raw).to(gpu), torch.from_numpy(x).to(gpu), logits)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(9).choice(V, 256, replace=False))
    _, ref = gemv.gemv16_ref(quants.dequant_q5k(raw[rows], K), x)
    err = _rows_err(logits.cpu().numpy()[:, rows], ref)
    print(f"[head8] sampled max row rel-err {err:.3e}")
    assert err <= TOL


def test_k4_gemv16_rejects_bad_arguments(gpu):
    print("[case] k4 gemv bad args", flush=True)
    w = torch.zeros(64, 144 * 2 + 16, dtype=torch.uint8, device=gpu)
    x = torch.zeros(17, 512, dtype=torch.float16, device=gpu)
    out = torch.empty(17, 32, dtype=torch.float16, device=gpu)
    with pytest.raises(TlxError):          # M = 17 > TLX_MAX_M
        ops.q4k_gemv16(w, x, out)
    with pytest.raises(TlxError):          # weights not 16-B aligned
        ops.q4k_gemv16(w.view(-1)[8:8 + 32 * 288], x[:2], out[:2])
