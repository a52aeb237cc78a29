"""GPU int8-activation (W4A8) prefill branch against oracle/p8.py.

The quantizer is bit-exact (int8 values, scales, row sums).  The GEMM output is checked
per activation row, norm-wise, within 1e-3 of the float64 product of the dequantized int8
activations and the linearized weights followed by the fp16 SwiGLU epilogue (the kernel's
fp32 sums and its one-step regrouping of the scale differ from float64 only by rounding).
"""
import numpy as np
import pytest
import torch

from oracle import gemv, p8
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _x(rng, M, K):
    return (rng.standard_normal((M, K)) * 0.7).astype(np.float16)


def _quant(gpu, x):
    M, K = x.shape
    xq = torch.empty(M, K, dtype=torch.int8, device=gpu)
    sx = torch.empty(M, K // 128, dtype=torch.float32, device=gpu)
    rs = torch.empty(M, K // 128, dtype=torch.int32, device=gpu)
    ops.p8_quant(torch.from_numpy(x).to(gpu), xq, sx, rs)
    torch.cuda.synchronize()
    return xq, sx, rs


@pytest.mark.parametrize("M,K", [(37, 640), (256, 5120)])
def test_p8_quant_bit_exact(gpu, M, K):
    print(f"[case] p8_quant M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K)
    x = _x(rng, M, K)
    x[1, 128:256] = 0                        # all-zero chunk
    x[2, 0:128] = np.float16(2.5)            # ties after scaling
    x[2, 5] = np.float16(127.0)
    x[3, 300] = np.float16(-60000.0)         # dominant element near the fp16 limit
    xq, sx, rs = _quant(gpu, x)
    rq, rsx, rrs = p8.quant_rows_ref(x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), rsx.view(np.uint32))
    assert np.array_equal(rs.cpu().numpy(), rrs)


def _w(rng, N, K, gpu):
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
    return packed, torch.from_numpy(formats.iq3_pack7(packed, K)).to(gpu)


@pytest.mark.parametrize("M,N,K", [(128, 64, 256), (256, 128, 1024), (128, 192, 5120), (384, 64, 768)])
def test_p8w4_ffn_parity(gpu, M, N, K):
    print(f"[case] p8w4_ffn M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(4)
    pg, wg = _w(rng, N, K, gpu)
    pu, wu = _w(rng, N, K, gpu)
    xq, sx, _ = _quant(gpu, _x(rng, M, K))
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.p8w4_ffn(wg, wu, formats.lut8_tensor(gpu), xq, sx, out)
    torch.cuda.synchronize()
    _, _, ref = p8.w4a8_ffn_ref(p8.dequant_lin_packed(pg, K), p8.dequant_lin_packed(pu, K),
                                xq.cpu().numpy(), sx.cpu().numpy())
    got = out.cpu().numpy()
    err = max(gemv.rel_err(got[m], ref[m]) for m in range(M))
    print(f"[p8w4_ffn M={M} N={N} K={K}] max row rel-err {err:.3e}")
    assert err <= TOL


def test_p8w4_ffn_config4_sampled(gpu):
    """Config 4 shape (M=2048, K=5120, N=17408): every activation row against 96 sampled
    output columns; and a second call is bit-identical."""
    print("[case] p8w4_ffn config 4 M=2048 sampled", flush=True)
    M, N, K = 2048, 17408, 5120
    rng = synth.config_rng(4)
    pg, wg = _w(rng, N, K, gpu)
    pu, wu = _w(rng, N, K, gpu)
    xq, sx, _ = _quant(gpu, _x(rng, M, K))
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    lut = formats.lut8_tensor(gpu)
    ops.p8w4_ffn(wg, wu, lut, xq, sx, out)
    torch.cuda.synchronize()
    first = out.clone()
    ops.p8w4_ffn(wg, wu, lut, xq, sx, out)
    torch.cuda.synchronize()
    assert torch.equal(first, out)
    cols = np.sort(np.random.default_rng(9).choice(N, 96, replace=False))
    _, _, ref = p8.w4a8_ffn_ref(p8.dequant_lin_packed(pg[cols], K), p8.dequant_lin_packed(pu[cols], K),
                                xq.cpu().numpy(), sx.cpu().numpy())
    got = out.cpu().numpy()[:, cols]
    err = max(gemv.rel_err(got[m], ref[m]) for m in range(M))
    print(f"[p8w4_ffn config 4] max row rel-err over sampled columns {err:.3e}")
    assert err <= TOL


def test_p8_bad_arguments(gpu):
    print("[case] p8 argument checks", flush=True)
    rng = synth.config_rng(4)
    _, wg = _w(rng, 64, 256, gpu)
    xq = torch.zeros(128, 256, dtype=torch.int8, device=gpu)
    sx = torch.ones(128, 2, dtype=torch.float32, device=gpu)
    out = torch.empty(128, 64, dtype=torch.float16, device=gpu)
    lut = formats.lut8_tensor(gpu)
    with pytest.raises(TlxError):   # only the packed7 layout is accepted
        ops.p8w4_ffn(wg, wg, lut, xq, sx, out, layout=LAYOUT_PACKED)
    with pytest.raises(TlxError):   # M must be a multiple of 128
        ops.p8w4_ffn(wg, wg, lut, xq[:64], sx[:64], out[:64])
    with pytest.raises(ValueError):
        ops.p8_quant(torch.zeros(4, 100, dtype=torch.float16, device=gpu), xq, sx, sx)
