"""GPU decode GEMVs against the oracle.

Tolerance (the accuracy contract of the path): norm-wise relative error <= 1e-3 per output
row against the exact product of the dequantized weights and the fp16 activations, followed
by the kernel's epilogue.  Full-size launches are checked on a seeded sample of rows.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_PACKED, LAYOUT_RAW, TlxError

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _iq3(rng, rows, kdim, dev):
    raw = synth.iq3xxs_raw(rng, rows, kdim)
    packed = formats.iq3_pack_rows(raw, kdim)
    return packed, torch.from_numpy(packed).to(dev)


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


@pytest.mark.parametrize("M", [1, 4, 8, 11, 16])
def test_ffn8_parity(gpu, M):
    print(f"[case] ffn8 M={M} N=512 K=5120", flush=True)
    rng = synth.config_rng(2)
    N, K = 512, 5120
    pg, wg = _iq3(rng, N, K, gpu)
    pu, wu = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    gact = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.ffn8(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), gact)
    torch.cuda.synchronize()
    Wg, Wu = quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K)
    _, _, ref = gemv.ffn8_ref(Wg, Wu, x)
    err = _rows_err(gact.cpu().numpy(), ref)
    print(f"[ffn8 M={M}] max row rel-err {err:.3e}")
    assert err <= TOL


def test_ffn8_full_size_sampled_rows(gpu):
    """Config 2 shape (N=17408, K=5120) at M=11; 384 seeded rows checked against the oracle."""
    print("[case] ffn8 full-size M=11", flush=True)
    rng = synth.config_rng(2)
    N, K, M = 17408, 5120, 11
    pg, wg = _iq3(rng, N, K, gpu)
    pu, wu = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    gact = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.ffn8(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), gact)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(N, 384, replace=False))
    Wg = quants.dequant_iq3xxs_packed(pg[rows], K)
    Wu = quants.dequant_iq3xxs_packed(pu[rows], K)
    _, _, ref = gemv.ffn8_ref(Wg, Wu, x)
    err = _rows_err(gact.cpu().numpy()[:, rows], ref)
    print(f"[ffn8 full] sampled max row rel-err {err:.3e}")
    assert err <= TOL


def test_ffn8_rows_invariant_and_deterministic(gpu):
    """Row r of an M=11 call equals an M=1 call on activation row r, bit for bit, and two
    runs agree bit for bit."""
    print("[case] ffn8 row invariance", flush=True)
    rng = np.random.default_rng(21)
    N, K, M = 256, 5120, 11
    _, wg = _iq3(rng, N, K, gpu)
    _, wu = _iq3(rng, N, K, gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    g = formats.gridf_tensor(gpu)
    full = torch.empty(M, N, dtype=torch.float16, device=gpu)
    again = torch.empty_like(full)
    ops.ffn8(wg, wu, g, x, full)
    ops.ffn8(wg, wu, g, x, again)
    one = torch.empty(1, N, dtype=torch.float16, device=gpu)
    for r in range(M):
        ops.ffn8(wg, wu, g, x[r:r + 1].contiguous(), one)
        assert torch.equal(one[0].view(torch.int16), full[r].view(torch.int16)), r
    assert torch.equal(full.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("M", [1, 11, 16])
def test_down8_parity(gpu, M):
    print(f"[case] down8 M={M} N=256 K=17408", flush=True)
    rng = np.random.default_rng(40 + M)
    N, K = 256, 17408
    pd, wd = _iq3(rng, N, K, gpu)
    gact = synth.activations_f16(rng, M, K)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    y = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.down8(wd, formats.gridf_tensor(gpu), torch.from_numpy(gact).to(gpu), torch.from_numpy(hh).to(gpu), y)
    torch.cuda.synchronize()
    acc, ref = gemv.down8_ref(quants.dequant_iq3xxs_packed(pd, K), gact, hh)
    yy = y.cpu().numpy()
    err = _rows_err(yy - hh, ref - hh)
    print(f"[down8 M={M}] max row rel-err {err:.3e}")
    assert err <= TOL


def test_down8_full_size_sampled_rows(gpu):
    print("[case] down8 full-size M=11", flush=True)
    rng = np.random.default_rng(77)
    N, K, M = 5120, 17408, 11
    pd, wd = _iq3(rng, N, K, gpu)
    gact = synth.activations_f16(rng, M, K)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    y = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.down8(wd, formats.gridf_tensor(gpu), torch.from_numpy(gact).to(gpu), torch.from_numpy(hh).to(gpu), y)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(2).choice(N, 192, replace=False))
    _, ref = gemv.down8_ref(quants.dequant_iq3xxs_packed(pd[rows], K), gact, hh[:, rows])
    err = _rows_err(y.cpu().numpy()[:, rows] - hh[:, rows], ref - hh[:, rows])
    assert err <= TOL


def test_iq3_gemv_ragged_rows(gpu):
    """N not a multiple of the 16-row tile: the tail rows are computed, nothing past N is written."""
    print("[case] iq3_gemv ragged N=1000", flush=True)
    rng = np.random.default_rng(5)
    N, K, M = 1000, 6144, 3
    p, w = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.full((M, N + 8), -7.0, dtype=torch.float16, device=gpu)
    view = out[:, :N]
    tmp = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), tmp)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
    assert _rows_err(tmp.cpu().numpy(), ref) <= TOL
    assert view.numel() > 0 and torch.all(out[:, N:] == -7.0)


@pytest.mark.parametrize("M", [3, 9])
@pytest.mark.parametrize("N,K", [(48, 5120), (640, 512), (40, 1024), (9600, 1024)])
def test_iq3_gemv_work_splits(gpu, N, K, M):
    """Tiles split across waves (48x5120), waves without items (640x512, 40x1024) and several
    tiles per workgroup (9600x1024)."""
    print(f"[case] iq3_gemv split N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(N + K)
    p, w = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(w, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), out)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
    assert _rows_err(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("N,K", [(5120, 17408), (16, 17408), (1000, 6144), (17408, 5120)])
def test_rows_invariant_across_activation_paths(gpu, N, K):
    """From M=6 on the activations are read from a tile-ordered copy in the library workspace,
    below that straight from x: row r of an M=11 call equals an M=1 call bit for bit, and the
    same call after a call of another shape (which rewrites the workspace) reproduces the first
    bit for bit.  Sampled rows are checked against the oracle."""
    print(f"[case] iq3_gemv activation-path invariance N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + 3 * K)
    p, w = _iq3(rng, N, K, gpu)
    x = torch.from_numpy(synth.activations_f16(rng, 11, K)).to(gpu)
    g = formats.gridf_tensor(gpu)
    full = torch.empty(11, N, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(w, g, x, full)
    small = torch.empty(11, 48, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(w[:48] if N >= 48 else torch.cat([w] * 3), g, x, small)
    again = torch.empty_like(full)
    ops.iq3_gemv(w, g, x, again)
    one = torch.empty(1, N, dtype=torch.float16, device=gpu)
    for r in (0, 5, 10):
        ops.iq3_gemv(w, g, x[r:r + 1].contiguous(), one)
        assert torch.equal(one[0].view(torch.int16), full[r].view(torch.int16)), r
    assert torch.equal(full.view(torch.int16), again.view(torch.int16))
    rows = np.sort(np.random.default_rng(N).choice(N, min(N, 64), replace=False))
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p[rows], K), x.cpu().numpy())
    assert _rows_err(full.cpu().numpy()[:, rows], ref) <= TOL


@pytest.mark.parametrize("M", [3, 9])
@pytest.mark.parametrize("N,K", [(40, 5120), (24, 1024), (200, 512)])
def test_ffn8_work_splits(gpu, N, K, M):
    """Gate/up pairs over several block ranges and a ragged row count (200)."""
    print(f"[case] ffn8 split N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(7 * N + K)
    pg, wg = _iq3(rng, N, K, gpu)
    pu, wu = _iq3(rng, N, K, gpu)
    x = synth.activations_f16(rng, M, K)
    gact = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.ffn8(wg, wu, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), gact)
    torch.cuda.synchronize()
    Wg, Wu = quants.dequant_iq3xxs_packed(pg, K), quants.dequant_iq3xxs_packed(pu, K)
    _, _, ref = gemv.ffn8_ref(Wg, Wu, x)
    assert _rows_err(gact.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M", [1, 11])
def test_aq3k8_parity(gpu, M):
    print(f"[case] aq3k8 M={M}", flush=True)
    rng = np.random.default_rng(90 + M)
    K, Nq, Nk, Nv = 5120, 768, 128, 112
    pq, wq = _iq3(rng, Nq, K, gpu)
    pk, wk = _iq3(rng, Nk, K, gpu)
    pv, wv = _iq3(rng, Nv, K, gpu)
    x = synth.activations_f16(rng, M, K)
    outs = [torch.empty(M, n, dtype=torch.float16, device=gpu) for n in (Nq, Nk, Nv)]
    ops.aq3k8(wq, wk, wv, formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu), *outs)
    torch.cuda.synchronize()
    for p, o in zip((pq, pk, pv), outs):
        _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_packed(p, K), x)
        assert _rows_err(o.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("layout", [LAYOUT_RAW, LAYOUT_PACKED])
def test_q6k_gemv_config1(gpu, layout):
    """Config 1: Q6_K 5120x5120, fp32 x, fp32 y (seed 20261202), full size."""
    print(f"[case] q6k_gemv config1 layout={layout}", flush=True)
    rng = synth.config_rng(1)
    rows = K = 5120
    raw = synth.q6k_raw(rng, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    host = raw if layout == LAYOUT_RAW else formats.q6_pad_rows(raw, K)
    y = torch.empty(rows, dtype=torch.float32, device=gpu)
    ops.h6k_gemv(torch.from_numpy(host).to(gpu), torch.from_numpy(x).to(gpu), y, layout)
    torch.cuda.synchronize()
    ref = gemv.q6k_gemv_ref(quants.dequant_q6k(raw, K), x)
    err = gemv.rel_err(y.cpu().numpy(), ref)
    print(f"[q6k config1] rel-err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("rows,K,layout", [(1000, 2304, LAYOUT_RAW), (37, 12288, LAYOUT_PACKED),
                                            (333, 15360, LAYOUT_RAW), (5, 256, LAYOUT_PACKED), (4099, 5120, LAYOUT_RAW)])
def test_q6k_gemv_shapes(gpu, rows, K, layout):
    """The fp32 GEMV's other paths: a block count that is not a multiple of 4 (blocks past the end
    weighted 0), several rounds of steps (K > 6144), the largest K (15360: x and its group sums
    fill 75 KB of LDS, past the 64 KB default limit), odd row counts (a workgroup's last rows masked) and tiny matrices."""
    print(f"[case] q6k_gemv rows={rows} K={K} layout={layout}", flush=True)
    rng = np.random.default_rng(rows + K)
    raw = synth.q6k_raw(rng, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    host = raw if layout == LAYOUT_RAW else formats.q6_pad_rows(raw, K)
    y = torch.full((rows + 3,), 7.0, dtype=torch.float32, device=gpu)
    ops.h6k_gemv(torch.from_numpy(host).to(gpu), torch.from_numpy(x).to(gpu), y[:rows], layout)
    torch.cuda.synchronize()
    ref = gemv.q6k_gemv_ref(quants.dequant_q6k(raw, K), x)
    yy = y.cpu().numpy()
    assert np.all(yy[rows:] == 7.0)   # nothing past the output
    err = gemv.rel_err(yy[:rows], ref)
    print(f"[q6k rows={rows} K={K}] rel-err {err:.3e}")
    assert err <= TOL


def test_q6k_gemv_rejects_k_beyond_lds(gpu):
    """K = 15616 is past the largest K the staged activations are sized for: rejected before any launch."""
    K = 15616
    with pytest.raises(TlxError):
        ops.h6k_gemv(torch.zeros(210 * (K // 256), dtype=torch.uint8, device=gpu), torch.zeros(K, device=gpu),
                     torch.zeros(1, device=gpu), LAYOUT_RAW)


def test_bad_arguments_raise(gpu):
    g = formats.gridf_tensor(gpu)
    w = torch.zeros(16 * 1960, dtype=torch.uint8, device=gpu)
    x = torch.zeros(17, 5120, dtype=torch.float16, device=gpu)
    out = torch.zeros(17, 16, dtype=torch.float16, device=gpu)
    with pytest.raises(TlxError):
        ops.ffn8(w, w, g, x, out)


# ---------------------------------------------------------------- GGUF-block (raw) IQ3_XXS rows
@pytest.mark.parametrize("M,K", [(1, 5120), (11, 5120), (4, 768)])
def test_iq3_gemv_raw_blocks(gpu, M, K):
    """The GEMV on GGUF-ordered blocks (2-B aligned fields; an odd block count is allowed)."""
    print(f"[case] iq3_gemv raw M={M} K={K}", flush=True)
    rng = np.random.default_rng(400 + M + K)
    N = 300
    raw = synth.iq3xxs_raw(rng, N, K)
    x = synth.activations_f16(rng, M, K)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(torch.from_numpy(raw).to(gpu), formats.gridf_tensor(gpu), torch.from_numpy(x).to(gpu),
                 out, LAYOUT_RAW)
    torch.cuda.synchronize()
    _, ref = gemv.gemv16_ref(quants.dequant_iq3xxs_blocks(raw.reshape(-1, 98)).reshape(N, K), x)
    assert _rows_err(out.cpu().numpy(), ref) <= TOL


def test_ffn8_and_down8_raw_blocks(gpu):
    print("[case] ffn8/down8 raw", flush=True)
    rng = np.random.default_rng(501)
    N, K, M = 256, 5120, 5
    rg, ru = synth.iq3xxs_raw(rng, N, K), synth.iq3xxs_raw(rng, N, K)
    x = synth.activations_f16(rng, M, K)
    g = formats.gridf_tensor(gpu)
    gact = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.ffn8(torch.from_numpy(rg).to(gpu), torch.from_numpy(ru).to(gpu), g, torch.from_numpy(x).to(gpu),
             gact, LAYOUT_RAW)
    deq = lambda r, k: quants.dequant_iq3xxs_blocks(r.reshape(-1, 98)).reshape(len(r), k)
    _, _, ref = gemv.ffn8_ref(deq(rg, K), deq(ru, K), x)
    assert _rows_err(gact.cpu().numpy(), ref) <= TOL
    Kd = 1024
    rd = synth.iq3xxs_raw(rng, N, Kd)
    xd = synth.activations_f16(rng, M, Kd)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    y = torch.empty(M, N, dtype=torch.float32, device=gpu)
    ops.down8(torch.from_numpy(rd).to(gpu), g, torch.from_numpy(xd).to(gpu), torch.from_numpy(hh).to(gpu),
              y, LAYOUT_RAW)
    torch.cuda.synchronize()
    _, refd = gemv.down8_ref(deq(rd, Kd), xd, hh)
    assert _rows_err(y.cpu().numpy() - hh, refd - hh) <= TOL


# ---------------------------------------------------------------- fused attention variants
def _attn_case(gpu, name, M, seed):
    from thunderllamax_amd._lib import V_Q4K
    rng = np.random.default_rng(seed)
    K, Nq, Nk, Nv = 5120, 384, 64, 48
    deq3 = lambda r: quants.dequant_iq3xxs_blocks(r.reshape(-1, 98)).reshape(len(r), K)
    rq3, rk3, rv3 = synth.iq3xxs_raw(rng, Nq, K), synth.iq3xxs_raw(rng, Nk, K), synth.iq3xxs_raw(rng, Nv, K)
    rq6 = synth.q6k_raw(rng, Nq, K)
    rv4 = synth.k4_raw(rng, Nv, K, False)
    x = synth.activations_f16(rng, M, K)
    pk = lambda r: formats.iq3_pack_rows(r, K)
    if name == "aq3k8_v4":
        w = (pk(rq3), pk(rk3), rv4); fn = lambda *a: ops.aq3k8(*a, layout=LAYOUT_PACKED | V_Q4K)
        W = (deq3(rq3), deq3(rk3), quants.dequant_q4k(rv4, K))
    elif name == "aq6k8_raw_v4":
        w = (rq6, pk(rk3), rv4); fn = lambda *a: ops.aq6k8(*a, layout=LAYOUT_RAW | V_Q4K)
        W = (quants.dequant_q6k(rq6, K), deq3(rk3), quants.dequant_q4k(rv4, K))
    elif name == "a_qkv_iq3":
        w = (rq3, rk3, rv4); fn = ops.a_qkv_iq3
        W = (deq3(rq3), deq3(rk3), quants.dequant_q4k(rv4, K))
    else:
        w = (rq6, rk3, rv4); fn = ops.a_qkv_q6
        W = (quants.dequant_q6k(rq6, K), deq3(rk3), quants.dequant_q4k(rv4, K))
    outs = [torch.empty(M, n, dtype=torch.float16, device=gpu) for n in (Nq, Nk, Nv)]
    fn(*[torch.from_numpy(np.ascontiguousarray(t)).to(gpu) for t in w], formats.gridf_tensor(gpu),
       torch.from_numpy(x).to(gpu), *outs)
    torch.cuda.synchronize()
    return [_rows_err(o.cpu().numpy(), gemv.gemv16_ref(Wm, x)[1]) for o, Wm in zip(outs, W)]


@pytest.mark.parametrize("name", ["aq3k8_v4", "aq6k8_raw_v4", "a_qkv_iq3", "a_qkv_q6"])
@pytest.mark.parametrize("M", [1, 11])
def test_attention_variants(gpu, name, M):
    print(f"[case] attention {name} M={M}", flush=True)
    errs = _attn_case(gpu, name, M, 600 + M)
    print(f"[{name} M={M}] q/k/v rel-err {errs}")
    assert max(errs) <= TOL
