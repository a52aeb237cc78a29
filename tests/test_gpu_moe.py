"""GPU MoE path (config 5: 256 IQ4_XS experts + 1 shared, hidden 2048, FF 512, top-8) against
the oracle.

Router ids and the sort are bit-exact; gates / sg within float32 exp rounding; the expert
GEMMs (fp16 operands, fp32 accumulation) within norm-wise rel-err 1e-3 per output row of the
exact float64 products of the dequantized weights.  The layer tests scale the N(0,1) hidden
states by 0.05: with config 5's weight statistics an unscaled input drives the down
projection past the fp16 range of its output (the reference stores it as fp16 too).
"""
import numpy as np
import pytest
import torch

from oracle import gemv, layouts, moe
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_RAW, LAYOUT_TILED, TlxError, call

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def experts(gpu):
    rng = synth.config_rng(5)
    gu, dn = synth.moe_expert_slabs(rng, moe.E + 1)
    dgu = [torch.from_numpy(s).to(gpu) for s in gu]
    ddn = [torch.from_numpy(s).to(gpu) for s in dn]
    return {
        "gu": gu, "dn": dn, "dgu": dgu, "ddn": ddn,
        "ptbl": formats.pointer_table(dgu[:moe.E], gpu),
        "ptbl_dn": formats.pointer_table(ddn[:moe.E], gpu),
        "ptbl_sh": formats.pointer_table([dgu[moe.E], ddn[moe.E]], gpu),
        "iq4nl": formats.iq4nl_tensor(gpu),
    }


@pytest.fixture(scope="module")
def experts_tiled(gpu, experts):
    """The same experts as tiled slabs (tlx_pack_iq4_tiled on the GPU); two slabs of each kind
    checked byte for byte against the oracle's restatement."""
    def tile(slabs, n, k):
        return [ops.pack_iq4_tiled(s, torch.empty_like(s), n, k) for s in slabs]
    tgu = tile(experts["dgu"], 2 * moe.FF, moe.HID)
    tdn = tile(experts["ddn"], moe.HID, moe.FF)
    torch.cuda.synchronize()
    for e in (0, moe.E):
        assert np.array_equal(tgu[e].cpu().numpy(),
                              layouts.pack_iq4_tiled(experts["gu"][e].reshape(2 * moe.FF, -1), moe.HID).ravel())
        assert np.array_equal(tdn[e].cpu().numpy(),
                              layouts.pack_iq4_tiled(experts["dn"][e].reshape(moe.HID, -1), moe.FF).ravel())
    return {
        "dgu": tgu, "ddn": tdn,
        "ptbl": formats.pointer_table(tgu[:moe.E], gpu),
        "ptbl_dn": formats.pointer_table(tdn[:moe.E], gpu),
        "ptbl_sh": formats.pointer_table([tgu[moe.E], tdn[moe.E]], gpu),
        "iq4nl": experts["iq4nl"],
    }


def _rows_err(y, ref):
    return max(gemv.rel_err(y[i], ref[i]) for i in range(ref.shape[0]))


def _run_layer(gpu, ex, x, logits, sg, hres, layout=LAYOUT_RAW):
    P = x.shape[0]
    np_ = 8 * P
    dx = torch.from_numpy(x).to(gpu)
    eids = torch.empty(P, 8, dtype=torch.int16, device=gpu)
    gates = torch.empty(P, 8, dtype=torch.float32, device=gpu)
    ops.moe_topk(torch.from_numpy(logits).to(gpu), eids, gates)
    eoff = torch.empty(257, dtype=torch.int32, device=gpu)
    plist = torch.empty(np_, dtype=torch.int16, device=gpu)
    items = torch.empty(ops.moe_max_items(np_), dtype=torch.int32, device=gpu)
    nitp = torch.empty(1, dtype=torch.int32, device=gpu)
    ops.moe_sort(eids, eoff, plist, items, nitp)
    act = torch.empty(np_, moe.FF, dtype=torch.float32, device=gpu)
    ops.moe_up4(ex["ptbl"], items, nitp, eoff, plist, dx, ex["iq4nl"], act, layout=layout)
    parts = torch.empty(np_, moe.HID, dtype=torch.float16, device=gpu)
    ops.moe_dn4(ex["ptbl_dn"], items, nitp, eoff, plist, act, ex["iq4nl"], parts, layout=layout)
    sact = torch.empty(P, moe.FF, dtype=torch.float32, device=gpu)
    shared = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
    ops.moe_shared(ex["ptbl_sh"], dx, ex["iq4nl"], sact, shared, layout=layout)
    y = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
    ops.moe_combine(parts, gates, torch.from_numpy(sg).to(gpu), shared, torch.from_numpy(hres).to(gpu), y)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in dict(eids=eids, gates=gates, eoff=eoff, plist=plist, items=items,
                                                   nitp=nitp, act=act, parts=parts, sact=sact, shared=shared,
                                                   y=y).items()}


def _inputs(rng, P):
    x = synth.bf16_round(0.05 * rng.standard_normal((P, moe.HID)).astype(np.float32))
    logits = rng.standard_normal((P, moe.E)).astype(np.float32)
    sg = (1.0 / (1.0 + np.exp(-rng.standard_normal(P)))).astype(np.float32)
    hres = rng.standard_normal((P, moe.HID)).astype(np.float32)
    return x, logits, sg, hres


def test_moe_topk_ties_and_gates(gpu):
    print("[case] moe topk P=300 with planted ties", flush=True)
    rng = np.random.default_rng(11)
    P = 300
    lg = rng.standard_normal((P, moe.E)).astype(np.float32)
    for p in range(0, P, 2):
        top = np.argsort(-lg[p])[:10]
        lg[p, top[6]] = lg[p, top[3]]
        lg[p, rng.integers(0, moe.E)] = lg[p, top[0]]
    eids = torch.empty(P, 8, dtype=torch.int16, device=gpu)
    gates = torch.empty(P, 8, dtype=torch.float32, device=gpu)
    ops.moe_topk(torch.from_numpy(lg).to(gpu), eids, gates)
    torch.cuda.synchronize()
    ref_e, ref_g = moe.topk_ref(lg)
    assert np.array_equal(eids.cpu().numpy().view(np.uint16), ref_e)
    np.testing.assert_allclose(gates.cpu().numpy(), ref_g, rtol=2e-6, atol=1e-7)


def test_moe_route(gpu):
    print("[case] moe route P=16", flush=True)
    rng = np.random.default_rng(12)
    P = 16
    wrt = (rng.standard_normal((moe.E, moe.HID)) * 0.02).astype(np.float32)
    wsh = (rng.standard_normal(moe.HID) * 0.02).astype(np.float32)
    h = rng.standard_normal((P, moe.HID)).astype(np.float32)
    eids = torch.empty(P, 8, dtype=torch.int16, device=gpu)
    gates = torch.empty(P, 8, dtype=torch.float32, device=gpu)
    sg = torch.empty(P, dtype=torch.float32, device=gpu)
    ops.moe_route(torch.from_numpy(wrt).to(gpu), torch.from_numpy(wsh).to(gpu), torch.from_numpy(h).to(gpu),
                  eids, gates, sg)
    torch.cuda.synchronize()
    lg64, ref_e, ref_g, ref_sg = moe.route_ref(wrt, wsh, h)
    got = eids.cpu().numpy().view(np.uint16)
    checked = 0
    for p in range(P):
        srt = np.sort(lg64[p])[::-1]
        if np.min(np.abs(np.diff(srt[:9]))) < 1e-4:   # fp32 summation order could flip a near-tie
            continue
        assert np.array_equal(got[p], ref_e[p]), p
        np.testing.assert_allclose(gates.cpu().numpy()[p], ref_g[p], rtol=1e-4)
        checked += 1
    assert checked >= P // 2
    np.testing.assert_allclose(sg.cpu().numpy(), ref_sg, rtol=1e-5)


@pytest.mark.parametrize("P", [11, 2048])
def test_moe_sort(gpu, P):
    print(f"[case] moe sort P={P}", flush=True)
    rng = np.random.default_rng(13 + P)
    ref_e, _ = moe.topk_ref(rng.standard_normal((P, moe.E)).astype(np.float32))
    np_ = 8 * P
    eids = torch.from_numpy(ref_e.view(np.int16)).to(gpu)
    eoff = torch.empty(257, dtype=torch.int32, device=gpu)
    plist = torch.empty(np_, dtype=torch.int16, device=gpu)
    items = torch.empty(ops.moe_max_items(np_), dtype=torch.int32, device=gpu)
    nitp = torch.empty(1, dtype=torch.int32, device=gpu)
    ops.moe_sort(eids, eoff, plist, items, nitp)
    torch.cuda.synchronize()
    ref_off, ref_pl = moe.sort_ref(ref_e)
    assert np.array_equal(eoff.cpu().numpy(), ref_off)
    assert np.array_equal(plist.cpu().numpy().view(np.uint16), ref_pl)
    cnt = np.diff(ref_off)
    tok = 64 if np_ <= 512 else 96   # pairs per item: 64 up to 512 pairs, 96 above
    want = [(e << 16) | k for e in range(moe.E) for k in range(0, int(cnt[e]), tok)]
    n = int(nitp.cpu().numpy()[0])
    assert n == len(want)
    assert np.array_equal(items.cpu().numpy().view(np.uint32)[:n], np.array(want, dtype=np.uint32))


def _check_layer(ex, x, logits, sg, hres, out, pairs, positions):
    """Compares the sampled pairs' act/parts and the sampled positions' y with the oracle."""
    eids, gates = moe.topk_ref(logits)
    assert np.array_equal(out["eids"].view(np.uint16), eids)
    by_e = {}
    for pair in pairs:
        by_e.setdefault(int(eids[pair // 8, pair % 8]), []).append(pair)
    for e, prs in by_e.items():
        xa = x[[p // 8 for p in prs]]
        act = moe.up_ref(ex["gu"][e], xa)
        assert _rows_err(out["act"][prs], act) <= TOL, e
        part = moe.down_ref(ex["dn"][e], act)
        assert _rows_err(out["parts"][prs].astype(np.float64), part) <= TOL, e
    sh = moe.down_ref(ex["dn"][moe.E], moe.up_ref(ex["gu"][moe.E], x[positions]))
    assert _rows_err(out["shared"][positions], sh) <= TOL
    # y from the GPU's own parts/shared (the combine alone): float32 rounding of ~10 operations,
    # bounded relative to the magnitude of the summands (the sum itself can cancel)
    pp = out["parts"][[8 * p + r for p in positions for r in range(8)]].reshape(len(positions), 8, moe.HID)
    g, s_, h = out["gates"][positions], sg[positions], hres[positions]
    yref = moe.combine_ref(pp, g, s_, out["shared"][positions], h)
    scale = np.abs(h) + np.einsum("pr,prk->pk", np.abs(g), np.abs(pp.astype(np.float64))) \
        + np.abs(s_)[:, None] * np.abs(out["shared"][positions])
    assert np.all(np.abs(out["y"][positions] - yref) <= 4e-6 * scale + 1e-30)


@pytest.mark.parametrize("P", [100, 300, 2048])
def test_moe_grouped_shared_fused(gpu, experts, experts_tiled, P):
    """moe_up4_sh / moe_dn4_sh -- the grouped forms and the shared expert in one launch each where
    both sides run their MFMA forms (P = 300, 2048), two launches otherwise (P = 100: the shared
    expert's GEMV form) -- against moe_up4 / moe_dn4 / moe_shared, bit for bit, GGUF rows and
    tiled slabs; and the oracle on sampled pairs and positions."""
    print(f"[case] grouped forms + shared expert in one launch, P={P}", flush=True)
    rng = np.random.default_rng(80 + P)
    x, logits, sg, hres = _inputs(rng, P)
    np_ = 8 * P
    dx = torch.from_numpy(x).to(gpu)
    eids = torch.empty(P, 8, dtype=torch.int16, device=gpu)
    gates = torch.empty(P, 8, dtype=torch.float32, device=gpu)
    ops.moe_topk(torch.from_numpy(logits).to(gpu), eids, gates)
    eoff = torch.empty(257, dtype=torch.int32, device=gpu)
    plist = torch.empty(np_, dtype=torch.int16, device=gpu)
    items = torch.empty(ops.moe_max_items(np_), dtype=torch.int32, device=gpu)
    nitp = torch.empty(1, dtype=torch.int32, device=gpu)
    ops.moe_sort(eids, eoff, plist, items, nitp)
    for ex, lay in ((experts, LAYOUT_RAW), (experts_tiled, LAYOUT_TILED)):
        bufs = {k: torch.full(shape, -3.0, dtype=dt, device=gpu) for k, (shape, dt) in dict(
            act=((np_, moe.FF), torch.float32), parts=((np_, moe.HID), torch.float16),
            sact=((P, moe.FF), torch.float32), shared=((P, moe.HID), torch.float32)).items()}
        fused = {k: torch.full_like(v, -5.0) for k, v in bufs.items()}
        ops.moe_up4(ex["ptbl"], items, nitp, eoff, plist, dx, ex["iq4nl"], bufs["act"], layout=lay)
        ops.moe_dn4(ex["ptbl_dn"], items, nitp, eoff, plist, bufs["act"], ex["iq4nl"], bufs["parts"], layout=lay)
        ops.moe_shared(ex["ptbl_sh"], dx, ex["iq4nl"], bufs["sact"], bufs["shared"], layout=lay)
        ops.moe_up4_sh(ex["ptbl"], items, nitp, eoff, plist, dx, ex["iq4nl"], fused["act"], ex["ptbl_sh"][0:1],
                       fused["sact"], layout=lay)
        ops.moe_dn4_sh(ex["ptbl_dn"], items, nitp, eoff, plist, fused["act"], ex["iq4nl"], fused["parts"],
                       ex["ptbl_sh"][1:2], fused["sact"], fused["shared"], layout=lay)
        torch.cuda.synchronize()
        for k in bufs:
            a, b = bufs[k].cpu().numpy(), fused[k].cpu().numpy()
            assert np.array_equal(a.view(np.uint16 if a.dtype == np.float16 else np.uint32),
                                  b.view(np.uint16 if b.dtype == np.float16 else np.uint32)), (lay, k)
    out = {k: v.cpu().numpy() for k, v in fused.items()}
    out.update(eids=eids.cpu().numpy(), gates=gates.cpu().numpy())
    ev, _ = moe.topk_ref(logits)
    pairs = [int(p) for p in np.random.default_rng(9).choice(np_, 24, replace=False)]
    by_e = {}
    for pair in pairs:
        by_e.setdefault(int(ev[pair // 8, pair % 8]), []).append(pair)
    for e, prs in by_e.items():
        act = moe.up_ref(experts["gu"][e], x[[p // 8 for p in prs]])
        assert _rows_err(out["act"][prs], act) <= TOL, e
        assert _rows_err(out["parts"][prs].astype(np.float64), moe.down_ref(experts["dn"][e], act)) <= TOL, e
    pos = sorted(int(p) for p in np.random.default_rng(10).choice(P, 8, replace=False))
    sh = moe.down_ref(experts["dn"][moe.E], moe.up_ref(experts["gu"][moe.E], x[pos]))
    assert _rows_err(out["shared"][pos], sh) <= TOL


def test_moe_layer_unscaled_overflow(gpu, experts):
    """Config 5's hidden states as the benchmark states them, N(0,1) unscaled (the other tests
    scale them by 0.05): about a fifth of the fp16 parts overflow, as the reference's fp16 parts
    would.  Where the oracle's part is clearly past fp16's range (|v| >= 66,200, 1% beyond the
    rounding edge 65,520) the GPU's is inf of the same sign; clearly inside (|v| <= 65,000) it is
    finite and, over those elements, within TOL.  y is the combine of the GPU's own parts in inf
    arithmetic: its nan and inf positions (and inf signs) are the oracle combine's exactly, the
    finite rest within the combine bound."""
    print("[case] moe layer P=11, N(0,1) hidden states (fp16 parts overflow)", flush=True)
    rng = np.random.default_rng(91)
    P = 11
    x = synth.bf16_round(rng.standard_normal((P, moe.HID)).astype(np.float32))
    logits = rng.standard_normal((P, moe.E)).astype(np.float32)
    sg = (1.0 / (1.0 + np.exp(-rng.standard_normal(P)))).astype(np.float32)
    hres = rng.standard_normal((P, moe.HID)).astype(np.float32)
    out = _run_layer(gpu, experts, x, logits, sg, hres)
    eids, _ = moe.topk_ref(logits)
    assert np.array_equal(out["eids"].view(np.uint16), eids)
    n_over = 0
    for pair in range(8 * P):
        e = int(eids[pair // 8, pair % 8])
        act = moe.up_ref(experts["gu"][e], x[pair // 8: pair // 8 + 1])
        assert _rows_err(out["act"][[pair]], act) <= TOL, pair
        ref = moe.down_ref(experts["dn"][e], out["act"][[pair]].astype(np.float64))[0]
        got = out["parts"][pair].astype(np.float64)
        big, small = np.abs(ref) >= 66200.0, np.abs(ref) <= 65000.0
        assert np.all(np.isinf(got[big]) & (np.sign(got[big]) == np.sign(ref[big]))), pair
        assert np.all(np.isfinite(got[small])), pair
        assert gemv.rel_err(got[small], ref[small]) <= TOL, pair
        n_over += int(big.sum())
    assert n_over > 1000   # the edge is exercised
    sh = moe.down_ref(experts["dn"][moe.E], moe.up_ref(experts["gu"][moe.E], x))
    assert _rows_err(out["shared"], sh) <= TOL
    pp = out["parts"].reshape(P, 8, moe.HID)
    with np.errstate(invalid="ignore"):
        yref = moe.combine_ref(pp, out["gates"], sg, out["shared"], hres)
    y = out["y"].astype(np.float64)
    assert np.array_equal(np.isnan(y), np.isnan(yref))
    inf = np.isinf(yref)
    assert inf.any() and np.array_equal(y[inf], yref[inf])
    fin = np.isfinite(yref)
    scale = np.abs(hres) + np.einsum("pr,prk->pk", np.abs(out["gates"]), np.abs(pp.astype(np.float64))) \
        + np.abs(sg)[:, None] * np.abs(out["shared"])
    assert np.all(np.abs(y[fin] - yref[fin]) <= 4e-6 * scale[fin] + 1e-30)


def test_moe_layer_decode_m11(gpu, experts):
    print("[case] moe layer P=11", flush=True)
    rng = np.random.default_rng(21)
    P = 11
    x, logits, sg, hres = _inputs(rng, P)
    out = _run_layer(gpu, experts, x, logits, sg, hres)
    _check_layer(experts, x, logits, sg, hres, out, list(range(8 * P)), list(range(P)))


@pytest.mark.parametrize("P", [16, 20])
def test_moe_layer_gemv_forms_swapped_grid(gpu, experts, P):
    """128 and 160 pairs: both GEMV forms on grids of 128+ columns, which run swapped (an
    item's row-tile groups dispatched one after another), every pair and position checked."""
    print(f"[case] moe layer P={P} (swapped GEMV grids)", flush=True)
    rng = np.random.default_rng(70 + P)
    x, logits, sg, hres = _inputs(rng, P)
    out = _run_layer(gpu, experts, x, logits, sg, hres)
    _check_layer(experts, x, logits, sg, hres, out, list(range(8 * P)), list(range(P)))


def test_moe_layer_prefill_m2048_sampled(gpu, experts):
    print("[case] moe layer P=2048", flush=True)
    rng = np.random.default_rng(22)
    P = 2048
    x, logits, sg, hres = _inputs(rng, P)
    out = _run_layer(gpu, experts, x, logits, sg, hres)
    srng = np.random.default_rng(5)
    pairs = sorted(srng.choice(8 * P, 96, replace=False).tolist())
    positions = sorted(srng.choice(P, 24, replace=False).tolist())
    _check_layer(experts, x, logits, sg, hres, out, pairs, positions)
    assert np.isfinite(out["y"]).all()


@pytest.mark.parametrize("P", [64, 256, 300])
def test_moe_layer_skewed(gpu, experts, P):
    """A router biased towards 12 experts gives them 2..4 groups of 16 tokens, and from 96 pairs
    on several items each (ragged last ones).  P = 64 (512 pairs): the gate+up GEMV form on 64-pair
    items and the down projection's MFMA form on the same items; P = 256 and 300: the MFMA forms on
    96-pair items, the shared expert in the GEMV form (P = 256) and in 32-position MFMA chunks
    ending on a 12-position one (P = 300)."""
    print(f"[case] moe layer skewed P={P}", flush=True)
    rng = np.random.default_rng(24 + P)
    x, logits, sg, hres = _inputs(rng, P)
    logits[:, :12] += 3.0
    out = _run_layer(gpu, experts, x, logits, sg, hres)
    eids, _ = moe.topk_ref(logits)
    cnt = np.bincount(eids.ravel(), minlength=moe.E)
    assert cnt[:12].min() > 16   # every hot expert has more than one group
    hot = [int(np.argmax(cnt[:12])), int(np.argmin(cnt[:12]))]
    pairs = [8 * p + r for p in range(P) for r in range(8) if eids[p, r] in hot]
    srng = np.random.default_rng(6)
    pairs = sorted(set(pairs) | set(srng.choice(8 * P, 48, replace=False).tolist()))
    positions = sorted(srng.choice(P, 12, replace=False).tolist())
    _check_layer(experts, x, logits, sg, hres, out, pairs, positions)


def test_moe_layer_deterministic(gpu, experts):
    print("[case] moe determinism P=256", flush=True)
    rng = np.random.default_rng(23)
    x, logits, sg, hres = _inputs(rng, 256)
    a = _run_layer(gpu, experts, x, logits, sg, hres)
    b = _run_layer(gpu, experts, x, logits, sg, hres)
    for k in ("plist", "act", "parts", "shared", "y"):
        assert np.array_equal(a[k], b[k]), k


def test_moe_bad_arguments(gpu, experts):
    print("[case] moe argument checks", flush=True)
    n = 16385   # one pair more than the sort supports: the library rejects it
    with pytest.raises(TlxError):
        ops.moe_sort(torch.zeros(n, dtype=torch.int16, device=gpu), torch.zeros(257, dtype=torch.int32, device=gpu),
                     torch.zeros(n, dtype=torch.int16, device=gpu),
                     torch.zeros(ops.moe_max_items(n), dtype=torch.int32, device=gpu),
                     torch.zeros(1, dtype=torch.int32, device=gpu))
    z = torch.zeros(16, dtype=torch.int32, device=gpu)
    with pytest.raises(TlxError):
        ops.moe_topk(torch.zeros(0, 256, dtype=torch.float32, device=gpu), z, z)
    # the fused decode launches: no positions, and a shared-activation buffer off 16-B alignment
    x1 = torch.zeros(1, 2048, device=gpu)
    e8 = torch.zeros(8, dtype=torch.int16, device=gpu)
    a8 = torch.zeros(8, 512, device=gpu)
    sa = torch.zeros(2 * 512 + 4, device=gpu)
    with pytest.raises(TlxError):
        call("tlx_moe_up4_pairs_sh", experts["ptbl"].data_ptr(), e8.data_ptr(), x1.data_ptr(), experts["iq4nl"].data_ptr(),
             a8.data_ptr(), experts["ptbl_sh"].data_ptr(), sa.data_ptr(), 0, LAYOUT_RAW, 0)
    with pytest.raises(TlxError):
        call("tlx_moe_up4_pairs_sh", experts["ptbl"].data_ptr(), e8.data_ptr(), x1.data_ptr(), experts["iq4nl"].data_ptr(),
             a8.data_ptr(), experts["ptbl_sh"].data_ptr(), sa[1:].data_ptr(), 1, LAYOUT_RAW, 0)
    with pytest.raises(ValueError):   # a pointer table shorter than 256 entries never reaches the library
        ops.moe_up4(experts["ptbl"][:8], torch.zeros(ops.moe_max_items(8), dtype=torch.int32, device=gpu),
                    torch.zeros(1, dtype=torch.int32, device=gpu), torch.zeros(257, dtype=torch.int32, device=gpu),
                    torch.zeros(8, dtype=torch.int16, device=gpu), torch.zeros(1, 2048, device=gpu),
                    experts["iq4nl"], torch.zeros(8, 512, device=gpu))


@pytest.mark.parametrize("P", [1, 11])
def test_moe_pair_walk_equals_grouped(gpu, experts, P):
    """The pair-walk decode forms (gx8e256up4 / gx8e256dn: expert eids[p], no sort) give the
    grouped forms' act and parts bit for bit, and the oracle's within tolerance."""
    print(f"[case] moe pair walk P={P}", flush=True)
    rng = np.random.default_rng(40 + P)
    x, logits, sg, hres = _inputs(rng, P)
    a = _run_layer(gpu, experts, x, logits, sg, hres)
    np_ = 8 * P
    eids = torch.from_numpy(a["eids"].reshape(-1)).to(gpu)
    act = torch.empty(np_, moe.FF, dtype=torch.float32, device=gpu)
    ops.moe_up4_pairs(experts["ptbl"], eids, torch.from_numpy(x).to(gpu), experts["iq4nl"], act)
    parts = torch.empty(np_, moe.HID, dtype=torch.float16, device=gpu)
    ops.moe_dn4_pairs(experts["ptbl_dn"], eids, act, experts["iq4nl"], parts)
    torch.cuda.synchronize()
    assert np.array_equal(act.cpu().numpy(), a["act"])
    assert np.array_equal(parts.cpu().numpy(), a["parts"])


@pytest.mark.parametrize("P", [1, 11, 70])
@pytest.mark.parametrize("lay", ["raw", "tiled"])
def test_moe_pair_walk_with_shared_expert(gpu, experts, experts_tiled, P, lay):
    """The fused decode launches (pair walk + the shared expert's 16-position chunks in one grid)
    give the separate calls' act, parts (the pair-walk calls), shared activations and shared
    output (tlx_moe_shared: 64-position chunks) bit for bit (P = 70: five shared chunks, the last
    of 6 positions)."""
    print(f"[case] moe pair walk + shared P={P} {lay}", flush=True)
    ex, layout = (experts, LAYOUT_RAW) if lay == "raw" else (experts_tiled, LAYOUT_TILED)
    rng = np.random.default_rng(60 + P)
    x, logits, sg, hres = _inputs(rng, P)
    a = _run_layer(gpu, ex, x, logits, sg, hres, layout=layout)
    np_ = 8 * P
    eids = torch.from_numpy(a["eids"].reshape(-1)).to(gpu)
    dx = torch.from_numpy(x).to(gpu)
    ract = torch.empty(np_, moe.FF, dtype=torch.float32, device=gpu)
    ops.moe_up4_pairs(ex["ptbl"], eids, dx, ex["iq4nl"], ract, layout=layout)
    rparts = torch.empty(np_, moe.HID, dtype=torch.float16, device=gpu)
    ops.moe_dn4_pairs(ex["ptbl_dn"], eids, ract, ex["iq4nl"], rparts, layout=layout)
    act = torch.full((np_, moe.FF), float("nan"), dtype=torch.float32, device=gpu)
    sact = torch.full((P, moe.FF), float("nan"), dtype=torch.float32, device=gpu)
    ops.moe_up4_pairs_sh(ex["ptbl"], eids, torch.from_numpy(x).to(gpu), ex["iq4nl"], act, ex["ptbl_sh"][0:1], sact,
                         layout=layout)
    parts = torch.full((np_, moe.HID), float("nan"), dtype=torch.float16, device=gpu)
    shared = torch.full((P, moe.HID), float("nan"), dtype=torch.float32, device=gpu)
    ops.moe_dn4_pairs_sh(ex["ptbl_dn"], eids, act, ex["iq4nl"], parts, ex["ptbl_sh"][1:2], sact, shared,
                         layout=layout)
    torch.cuda.synchronize()
    assert np.array_equal(act.cpu().numpy(), ract.cpu().numpy())
    assert np.array_equal(sact.cpu().numpy(), a["sact"])
    assert np.array_equal(parts.cpu().numpy(), rparts.cpu().numpy())
    assert np.array_equal(shared.cpu().numpy(), a["shared"])


def test_moe_layer_overlapped_equals_sequential(gpu, experts):
    """ops.moe_layer gives the separate sequential calls' results bit for bit, eagerly and in every
    replay of a captured graph (eager work and synchronizations between the replays): at P = 11
    with its defaults (the pair walk with the shared expert inside its launches) and with the
    shared expert on a second stream beside the pair walk and beside the sorted, grouped forms;
    at P = 300 with its defaults (the grouped forms with the shared expert inside) and with the
    shared expert on a second stream."""
    print("[case] moe_layer routes vs sequential P=11 / 300", flush=True)
    for P, pw, ov in ((11, None, None), (11, True, True), (11, False, True), (300, None, None), (300, None, True)):
        print(f"[case] moe_layer P={P} pair_walk={pw} overlap={ov}", flush=True)
        rng = np.random.default_rng(31 + P)
        x, logits, sg, hres = _inputs(rng, P)
        ref = _run_layer(gpu, experts, x, logits, sg, hres)
        dx, dl = torch.from_numpy(x).to(gpu), torch.from_numpy(logits).to(gpu)
        dsg, dh = torch.from_numpy(sg).to(gpu), torch.from_numpy(hres).to(gpu)
        sc = ops.MoeScratch(P, gpu)
        y = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
        args = (dl, dsg, dx, dh, y, experts["ptbl"], experts["ptbl_dn"], experts["ptbl_sh"], experts["iq4nl"], sc)
        ops.moe_layer(*args, pair_walk=pw, overlap_shared=ov)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), ref["y"])
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            ops.moe_layer(*args, stream=st, pair_walk=pw, overlap_shared=ov)
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            ops.moe_layer(*args, stream=st, pair_walk=pw, overlap_shared=ov)
        for _ in range(3):
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), ref["y"])


@pytest.mark.parametrize("P", [11, 300, 2048])
def test_moe_tiled_slabs_equal_gguf_rows(gpu, experts, experts_tiled, P):
    """Tiled expert slabs give the GGUF rows' router-to-combine results bit for bit: GEMV form
    (P = 11), GEMM form with ragged items (P = 300, a biased router) and config 5's M = 2048;
    at P = 11 also the pair-walk forms.  (The GGUF-row results are checked against the oracle by
    the tests above.)"""
    print(f"[case] moe tiled slabs P={P}", flush=True)
    rng = np.random.default_rng(50 + P)
    x, logits, sg, hres = _inputs(rng, P)
    if P == 300:
        logits[:, :12] += 3.0
    a = _run_layer(gpu, experts, x, logits, sg, hres)
    b = _run_layer(gpu, experts_tiled, x, logits, sg, hres, layout=LAYOUT_TILED)
    for k in ("act", "parts", "shared", "y"):
        assert np.array_equal(a[k], b[k]), k
    if P == 11:
        np_ = 8 * P
        eids = torch.from_numpy(a["eids"].reshape(-1)).to(gpu)
        act = torch.empty(np_, moe.FF, dtype=torch.float32, device=gpu)
        ops.moe_up4_pairs(experts_tiled["ptbl"], eids, torch.from_numpy(x).to(gpu), experts["iq4nl"], act,
                          layout=LAYOUT_TILED)
        parts = torch.empty(np_, moe.HID, dtype=torch.float16, device=gpu)
        ops.moe_dn4_pairs(experts_tiled["ptbl_dn"], eids, act, experts["iq4nl"], parts, layout=LAYOUT_TILED)
        torch.cuda.synchronize()
        assert np.array_equal(act.cpu().numpy(), a["act"])
        assert np.array_equal(parts.cpu().numpy(), a["parts"])
