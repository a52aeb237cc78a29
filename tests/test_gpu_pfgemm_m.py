"""The merged multi-class prefill GEMM (tlx_pfg3m, the reference's pf_gemm3m) against the oracle.

* Operands: with unit-vector activation rows x = e_m, out[m][n] = half(W16[n][m]) exactly (a -0
  weight gives +0: the fp32 sum starts at +0), so the
  fp16 operand of every weight class is checked bit for bit against fp16 of the oracle's fp32
  dequantization (quants.dequant_q4k / dequant_q5k / dequant_q6k / dequant_iq3xxs_packed, the
  formulas of /root/reference/engine/pf_gemm3m.cu:61-136).
* Products: random activations, relative error <= 1e-3 per output row against the float64 product
  of the dequantized weights followed by the half rounding (the path's accuracy contract).
* The reference's three merged configurations (/root/reference/engine/build_p7b.py:58-77) at
  config 4's M = 2048, K = 5120: attention q/k/v with an IQ3_XXS q, the same with a Q6_K q, and
  the GDN qkv (Q5_K) with the IQ3_XXS gate.  Sampled rows against the oracle, every segment bit
  for bit equal to a one-segment call on the same matrix, two calls bit for bit equal.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import (LAYOUT_PACK7, LAYOUT_PACKED, LAYOUT_RAW, TYPE_IQ3_XXS, TYPE_Q4_K, TYPE_Q5_K,
                                    TYPE_Q6_K, TlxError)

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _mat(rng, cls, n, k):
    """(device bytes, oracle fp32 dequant callable over row indices) of one weight class."""
    if cls == "iq3":
        packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, n, k), k)
        dev = formats.iq3_pack7(packed, k)
        return dev, (lambda rows: quants.dequant_iq3xxs_packed(packed[rows], k)), TYPE_IQ3_XXS, LAYOUT_PACK7
    if cls in ("q4k", "q5k"):
        raw = synth.k4_raw(rng, n, k, cls == "q5k")
        deq = quants.dequant_q5k if cls == "q5k" else quants.dequant_q4k
        return raw, (lambda rows: deq(raw[rows], k)), (TYPE_Q5_K if cls == "q5k" else TYPE_Q4_K), LAYOUT_RAW
    raw = synth.q6k_raw(rng, n, k)
    return formats.q6_pad_rows(raw, k), (lambda rows: quants.dequant_q6k(raw[rows], k)), TYPE_Q6_K, LAYOUT_PACKED


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(gpu)


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("cls", ["iq3", "q4k", "q5k", "q6k"])
def test_pfg3m_operands_bit_exact(gpu, cls):
    print(f"[case] pfg3m operands {cls}", flush=True)
    rng = np.random.default_rng(800 + len(cls))
    N, K = 256, 512
    w, deq, t, lay = _mat(rng, cls, N, K)
    x = torch.eye(K, dtype=torch.float16, device=gpu)          # M = K = 512 unit rows
    out = torch.empty(K, N, dtype=torch.float16, device=gpu)
    ops.pfg3m([_dev(w, gpu)], [out], [t], [lay], formats.gridf_tensor(gpu), x)
    torch.cuda.synchronize()
    want = deq(np.arange(N)).astype(np.float16).T                # [k][n] = fp16(W[n][k])
    want[want == 0] = 0      # a -0 weight sums to +0 in the fp32 accumulation (0 + -0 = +0)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), np.argwhere(got.view(np.uint16) != want.view(np.uint16))[:5]


@pytest.mark.parametrize("cls", ["iq3", "q4k", "q5k", "q6k"])
def test_pfg3m_single_segment_parity(gpu, cls):
    print(f"[case] pfg3m single {cls}", flush=True)
    rng = np.random.default_rng(810 + len(cls))
    M, N, K = 256, 512, 1024
    w, deq, t, lay = _mat(rng, cls, N, K)
    xn = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.pfg3m([_dev(w, gpu)], [out], [t], [lay], formats.gridf_tensor(gpu), torch.from_numpy(xn).to(gpu))
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(deq(np.arange(N)), xn)
    y = out.cpu().numpy()
    err = max(gemv.rel_err(y[m], ref[m]) for m in range(M))
    print(f"[pfg3m {cls}] max row rel-err {err:.3e}")
    assert err <= TOL


CONFIGS = {   # /root/reference/engine/build_p7b.py:58-77 (segment class, rows)
    "attnqkv_i3": [("iq3", 12288), ("iq3", 1024), ("q4k", 1024)],
    "attnqkv_q6": [("q6k", 12288), ("iq3", 1024), ("q4k", 1024)],
    "gdnqg": [("q5k", 10240), ("iq3", 6144)],
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_pfg3m_reference_configs(gpu, name):
    print(f"[case] pfg3m {name} M=2048 K=5120", flush=True)
    rng = np.random.default_rng(820 + len(name))
    M, K = 2048, 5120
    segs = [_mat(rng, cls, n, K) + (n,) for cls, n in CONFIGS[name]]
    xn = synth.activations_f16(rng, M, K)
    x = torch.from_numpy(xn).to(gpu)
    g = formats.gridf_tensor(gpu)
    ws = [_dev(s[0], gpu) for s in segs]
    outs = [torch.empty(M, s[4], dtype=torch.float16, device=gpu) for s in segs]
    again = [torch.empty_like(o) for o in outs]
    ops.pfg3m(ws, outs, [s[2] for s in segs], [s[3] for s in segs], g, x)
    ops.pfg3m(ws, again, [s[2] for s in segs], [s[3] for s in segs], g, x)
    alone = []
    for w, s in zip(ws, segs):
        o = torch.empty(M, s[4], dtype=torch.float16, device=gpu)
        ops.pfg3m([w], [o], [s[2]], [s[3]], g, x)
        alone.append(o)
    torch.cuda.synchronize()
    mrows = np.sort(np.random.default_rng(1).choice(M, 24, replace=False))
    for i, (s, o) in enumerate(zip(segs, outs)):
        assert torch.equal(_bits(o), _bits(again[i])), f"segment {i} not deterministic"
        assert torch.equal(_bits(o), _bits(alone[i])), f"segment {i} differs from its one-segment call"
        rows = np.sort(np.random.default_rng(2 + i).choice(s[4], 128, replace=False))
        _, ref = gemv.gemv16_ref(s[1](rows), xn[mrows])
        y = o.cpu().numpy()[mrows][:, rows]
        err = max(gemv.rel_err(y[m], ref[m]) for m in range(len(mrows)))
        print(f"[pfg3m {name} seg {i}] sampled max row rel-err {err:.3e}")
        assert err <= TOL


def test_pfg3m_rejects_bad_segments(gpu):
    g = formats.gridf_tensor(gpu)
    x = torch.zeros(256, 512, dtype=torch.float16, device=gpu)
    w = torch.zeros(256 * 212 * 2, dtype=torch.uint8, device=gpu)
    o = torch.empty(256, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError):          # Q6_K raw blocks are not a segment class
        ops.pfg3m([w], [o], [TYPE_Q6_K], [LAYOUT_RAW], g, x)
    with pytest.raises(ValueError):          # weight buffer too small for the shape
        ops.pfg3m([w[:1000]], [o], [TYPE_Q6_K], [LAYOUT_PACKED], g, x)
    with pytest.raises(TlxError):            # n % 256
        ops.pfg3m([w], [torch.empty(256, 128, dtype=torch.float16, device=gpu)], [TYPE_Q6_K], [LAYOUT_PACKED], g, x)
