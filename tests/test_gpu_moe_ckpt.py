"""The MoE weight classes of the reference's real checkpoint on the GPU against the oracle: IQ3_S
routed gate/up (gxu_gm / gx8e256up), Q6_K routed down (gxm_dn6 / gx8e256dn6), the Q8_0 shared
expert (shexp8), and the IQ3_S / Q8_0 dequantizers.

* Dequantizers: bit for bit against quants.dequant_iq3s / dequant_q8_0 (f32), and the f16 outputs
  against the same values rounded by numpy (round to nearest even).
* Expert GEMMs: norm-wise rel-err <= 1e-3 per output row against the float64 products of the
  dequantized weights (moe.up3s_ref / down6_ref / shared8_ref), for the sorted form and the pair
  walk each; the two forms within 1e-5 of each other (f32 act; the pair walk's k-steps take the
  same products in another order) and within half an fp16 ulp norm-wise (parts); two calls bit for
  bit equal.
* The IQ3_S grid is synthetic (synth.iq3s_grid: ggml's level set, random entries): the real table
  is a third-party constant absent here, and the kernels take it at run time as the reference's do.
"""
import numpy as np
import pytest
import torch

from oracle import gemv, layouts, moe, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_RAW, LAYOUT_TILED, TlxError, call

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _rows_err(y, ref):
    return max(gemv.rel_err(y[i], ref[i]) for i in range(ref.shape[0]))


@pytest.fixture(scope="module")
def ckpt(gpu):
    rng = np.random.default_rng(20261205)
    gu, dn, shared = synth.moe_ckpt_slabs(rng, moe.E)
    grid = synth.iq3s_grid(rng)
    dgu = [torch.from_numpy(s).to(gpu) for s in gu]
    ddn = [torch.from_numpy(s).to(gpu) for s in dn]
    return {
        "gu": gu, "dn": dn, "shared": shared, "grid": grid, "dgu": dgu, "ddn": ddn,
        "ptbl": formats.pointer_table(dgu, gpu), "ptbl_dn": formats.pointer_table(ddn, gpu),
        "gridf": torch.from_numpy(grid.reshape(-1)).to(gpu),
        "dsh": [torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(gpu) for a in shared],
    }


def test_iq3s_dequant_bit_exact(gpu):
    print("[case] iq3s dequant 37 x 2048", flush=True)
    rng = np.random.default_rng(41)
    raw = synth.iq3s_raw(rng, 37, 2048)
    grid = synth.iq3s_grid(rng)
    want = quants.dequant_iq3s(raw, 2048, grid)
    w = torch.from_numpy(raw.reshape(-1)).to(gpu)
    g = torch.from_numpy(grid.reshape(-1)).to(gpu)
    o32 = ops.iq3s_dequant(w, g, torch.empty(37, 2048, dtype=torch.float32, device=gpu), 2048)
    o16 = ops.iq3s_dequant(w, g, torch.empty(37, 2048, dtype=torch.float16, device=gpu), 2048)
    torch.cuda.synchronize()
    assert np.array_equal(o32.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(o16.cpu().numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_q80_dequant_bit_exact(gpu):
    print("[case] q8_0 dequant 29 x 512", flush=True)
    raw = synth.q80_raw(np.random.default_rng(42), 29, 512)
    want = quants.dequant_q8_0(raw, 512)
    w = torch.from_numpy(raw.reshape(-1)).to(gpu)
    o32 = ops.q8_0_dequant(w, torch.empty(29, 512, dtype=torch.float32, device=gpu), 512)
    o16 = ops.q8_0_dequant(w, torch.empty(29, 512, dtype=torch.float16, device=gpu), 512)
    torch.cuda.synchronize()
    assert np.array_equal(o32.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(o16.cpu().numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))


def _route(gpu, rng, P):
    x = synth.bf16_round(0.05 * rng.standard_normal((P, moe.HID)).astype(np.float32))
    eids_ref, _ = moe.topk_ref(rng.standard_normal((P, moe.E)).astype(np.float32))
    np_ = 8 * P
    eids = torch.from_numpy(eids_ref.reshape(-1).view(np.int16)).to(gpu)
    eoff = torch.empty(257, dtype=torch.int32, device=gpu)
    plist = torch.empty(np_, dtype=torch.int16, device=gpu)
    items = torch.empty(ops.moe_max_items(np_), dtype=torch.int32, device=gpu)
    nitp = torch.empty(1, dtype=torch.int32, device=gpu)
    ops.moe_sort(eids, eoff, plist, items, nitp)
    return x, eids_ref.reshape(-1), eids, eoff, plist, items, nitp


def _run(gpu, ck, x, eids, eoff, plist, items, nitp, np_):
    dx = torch.from_numpy(x).to(gpu)
    act = torch.empty(np_, moe.FF, dtype=torch.float32, device=gpu)
    act_w = torch.empty_like(act)
    ops.moe_up3s(ck["ptbl"], eoff, plist, dx, ck["gridf"], act)
    ops.moe_up3s_pairs(ck["ptbl"], eids, dx, ck["gridf"], act_w)
    parts = torch.empty(np_, moe.HID, dtype=torch.float16, device=gpu)
    parts_w = torch.empty_like(parts)
    ops.moe_dn6(ck["ptbl_dn"], items, nitp, eoff, plist, act, parts)
    ops.moe_dn6_pairs(ck["ptbl_dn"], eids, act, parts_w)
    torch.cuda.synchronize()
    return act.cpu().numpy(), act_w.cpu().numpy(), parts.cpu().numpy(), parts_w.cpu().numpy()


def _check_pairs(ck, x, eids, act, parts, pairs, act_in=None):
    """act against the oracle's gate+up of x, parts against its down projection of act_in (the
    activations the down kernel read; act by default)."""
    act_in = act if act_in is None else act_in
    by_e = {}
    for p in pairs:
        by_e.setdefault(int(eids[p]), []).append(p)
    for e, prs in by_e.items():
        ref = moe.up3s_ref(ck["gu"][e], ck["grid"], x[[p // 8 for p in prs]])
        assert _rows_err(act[prs], ref) <= TOL, e
        part = moe.down6_ref(ck["dn"][e], act_in[prs])
        assert _rows_err(parts[prs].astype(np.float64), part) <= TOL, e


def _forms_agree(act, act_w, parts, parts_w):
    assert _rows_err(act_w, act.astype(np.float64)) <= 1e-5
    # fp16 outputs: a reordered f32 sum can round to a neighbouring fp16 value, several ulps of an
    # output that cancels towards zero -- a norm-wise bound, half an fp16 ulp of the row
    assert _rows_err(parts_w.astype(np.float64), parts.astype(np.float64)) <= 2.0 ** -11


def test_ckpt_experts_decode_m11(gpu, ckpt):
    print("[case] IQ3_S up + Q6_K down, P=11, every pair", flush=True)
    rng = np.random.default_rng(43)
    P = 11
    x, eids, deids, eoff, plist, items, nitp = _route(gpu, rng, P)
    act, act_w, parts, parts_w = _run(gpu, ckpt, x, deids, eoff, plist, items, nitp, 8 * P)
    _forms_agree(act, act_w, parts, parts_w)
    _check_pairs(ckpt, x, eids, act, parts, list(range(8 * P)))
    _check_pairs(ckpt, x, eids, act_w, parts_w, list(range(8 * P)), act_in=act)


def test_ckpt_pairs_ragged(gpu, ckpt):
    """The pair walk at pair counts that are not a multiple of 8 (the grid's padding): 1 and 13."""
    rng = np.random.default_rng(48)
    x, eids, deids, *_ = _route(gpu, rng, 2)
    dx = torch.from_numpy(x).to(gpu)
    for np_ in (1, 13):
        print(f"[case] IQ3_S up + Q6_K down pair walk, {np_} pairs", flush=True)
        act = torch.full((np_ + 3, moe.FF), -7.0, dtype=torch.float32, device=gpu)
        parts = torch.full((np_ + 3, moe.HID), -7.0, dtype=torch.float16, device=gpu)
        ops.moe_up3s_pairs(ckpt["ptbl"], deids[:np_], dx, ckpt["gridf"], act[:np_])
        ops.moe_dn6_pairs(ckpt["ptbl_dn"], deids[:np_], act[:np_], parts[:np_])
        torch.cuda.synchronize()
        a, pt = act.cpu().numpy(), parts.cpu().numpy()
        assert np.all(a[np_:] == -7.0) and np.all(pt[np_:] == -7.0)   # nothing past the pairs
        _check_pairs(ckpt, x, eids, a, pt, list(range(np_)))


def test_ckpt_experts_prefill_m2048(gpu, ckpt):
    print("[case] IQ3_S up + Q6_K down, P=2048, sampled pairs", flush=True)
    rng = np.random.default_rng(44)
    P = 2048
    x, eids, deids, eoff, plist, items, nitp = _route(gpu, rng, P)
    act, act_w, parts, parts_w = _run(gpu, ckpt, x, deids, eoff, plist, items, nitp, 8 * P)
    _forms_agree(act, act_w, parts, parts_w)
    again = _run(gpu, ckpt, x, deids, eoff, plist, items, nitp, 8 * P)
    assert np.array_equal(again[0].view(np.uint32), act.view(np.uint32))
    assert np.array_equal(again[1].view(np.uint32), act_w.view(np.uint32))
    assert np.array_equal(again[2].view(np.uint16), parts.view(np.uint16))
    assert np.array_equal(again[3].view(np.uint16), parts_w.view(np.uint16))
    # the largest bins (several 64-token passes) and a spread of others
    cnt = np.bincount(eids, minlength=moe.E)
    big = np.argsort(-cnt)[:2]
    pairs = [int(p) for e in big for p in np.nonzero(eids == e)[0][::7]]
    pairs += [int(p) for p in np.random.default_rng(5).choice(8 * P, 48, replace=False)]
    _check_pairs(ckpt, x, eids, act, parts, sorted(set(pairs)))
    _check_pairs(ckpt, x, eids, act_w, parts_w, sorted(set(pairs)), act_in=act)


@pytest.mark.parametrize("P", [1, 11, 16, 17, 300])
def test_ckpt_shared_q80(gpu, ckpt, P):
    """P <= 16 runs the decode (GEMV-shaped) form, larger P the LDS-staged one."""
    print(f"[case] Q8_0 shared expert P={P}", flush=True)
    rng = np.random.default_rng(45 + P)
    x = synth.bf16_round(0.05 * rng.standard_normal((P, moe.HID)).astype(np.float32))
    dx = torch.from_numpy(x).to(gpu)
    act = torch.empty(P, moe.FF, dtype=torch.float32, device=gpu)
    y = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
    ops.moe_shared8(*ckpt["dsh"], dx, y, act)
    torch.cuda.synchronize()
    wg, wu, wd = ckpt["shared"]
    ref = moe.shared8_ref(wg, wu, wd, x)
    assert _rows_err(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("P", [11, 300])
def test_ckpt_grouped_shared_fused(gpu, ckpt, P):
    """moe_up3s_sh / moe_dn6_sh (the sorted forms and the Q8_0 shared expert in one launch each
    above P = 16, two launches at P = 11) against moe_up3s / moe_dn6 / moe_shared8, bit for bit."""
    print(f"[case] sorted forms + Q8_0 shared expert in one launch, P={P}", flush=True)
    rng = np.random.default_rng(60 + P)
    x, eids, deids, eoff, plist, items, nitp = _route(gpu, rng, P)
    dx = torch.from_numpy(x).to(gpu)
    np_ = 8 * P
    mk = lambda shape, dt, v: torch.full(shape, v, dtype=dt, device=gpu)
    sep = dict(act=mk((np_, moe.FF), torch.float32, -3.0), parts=mk((np_, moe.HID), torch.float16, -3.0),
               sact=mk((P, moe.FF), torch.float32, -3.0), shared=mk((P, moe.HID), torch.float32, -3.0))
    fus = {k: torch.full_like(v, -5.0) for k, v in sep.items()}
    wg8, wu8, wd8 = ckpt["dsh"]
    ops.moe_up3s(ckpt["ptbl"], eoff, plist, dx, ckpt["gridf"], sep["act"])
    ops.moe_dn6(ckpt["ptbl_dn"], items, nitp, eoff, plist, sep["act"], sep["parts"])
    ops.moe_shared8(wg8, wu8, wd8, dx, sep["shared"], sep["sact"])
    ops.moe_up3s_sh(ckpt["ptbl"], eoff, plist, dx, ckpt["gridf"], fus["act"], wg8, wu8, fus["sact"])
    ops.moe_dn6_sh(ckpt["ptbl_dn"], items, nitp, eoff, plist, fus["act"], fus["parts"], wd8, fus["sact"],
                   fus["shared"])
    torch.cuda.synchronize()
    for k in sep:
        a, b = sep[k].cpu().numpy(), fus[k].cpu().numpy()
        v = np.uint16 if a.dtype == np.float16 else np.uint32
        assert np.array_equal(a.view(v), b.view(v)), k
    ref = moe.shared8_ref(*ckpt["shared"], x)
    assert _rows_err(fus["shared"].cpu().numpy(), ref) <= TOL


def test_ckpt_tiled_repack_matches_oracle(gpu, ckpt):
    """tlx_pack_iq3s_tiled / tlx_pack_q6k_tiled on an expert's slabs: byte for byte the oracle's
    records (which the CPU tests invert back to the GGUF rows)."""
    print("[case] IQ3_S / Q6_K tiled repack, expert 5's slabs", flush=True)
    gu, dn = ckpt["gu"][5], ckpt["dn"][5]
    tgu = ops.pack_iq3s_tiled(ckpt["dgu"][5], torch.empty_like(ckpt["dgu"][5]), 2 * moe.FF, moe.HID)
    tdn = ops.pack_q6k_tiled(ckpt["ddn"][5], torch.empty_like(ckpt["ddn"][5]), moe.HID, moe.FF)
    torch.cuda.synchronize()
    assert np.array_equal(tgu.cpu().numpy(), layouts.pack_iq3s_tiled(gu.reshape(2 * moe.FF, -1), moe.HID).reshape(-1))
    assert np.array_equal(tdn.cpu().numpy(), layouts.pack_q6k_tiled(dn.reshape(moe.HID, -1), moe.FF).reshape(-1))


@pytest.fixture(scope="module")
def ckpt_tiled(gpu, ckpt):
    tgu = [ops.pack_iq3s_tiled(s, torch.empty_like(s), 2 * moe.FF, moe.HID) for s in ckpt["dgu"]]
    tdn = [ops.pack_q6k_tiled(s, torch.empty_like(s), moe.HID, moe.FF) for s in ckpt["ddn"]]
    torch.cuda.synchronize()
    return {"tgu": tgu, "tdn": tdn, "ptbl": formats.pointer_table(tgu, gpu), "ptbl_dn": formats.pointer_table(tdn, gpu)}


@pytest.mark.parametrize("P", [11, 300, 2048])
def test_ckpt_tiled_forms_bit_identical(gpu, ckpt, ckpt_tiled, P):
    """Every checkpoint-class routed form over the tiled slabs (layout=LAYOUT_TILED) against the same
    form over the GGUF rows, bit for bit: the pair walks, the sorted forms, the forms with the shared
    expert, and the down's staged form (parts not 8-B aligned)."""
    print(f"[case] checkpoint-class forms on tiled slabs vs GGUF rows, P={P}", flush=True)
    rng = np.random.default_rng(80 + P)
    x, eids, deids, eoff, plist, items, nitp = _route(gpu, rng, P)
    dx = torch.from_numpy(x).to(gpu)
    np_ = 8 * P
    wg8, wu8, wd8 = ckpt["dsh"]

    def run(lay):
        pt, pd = (ckpt["ptbl"], ckpt["ptbl_dn"]) if lay == LAYOUT_RAW else (ckpt_tiled["ptbl"], ckpt_tiled["ptbl_dn"])
        o = {}
        o["act"] = torch.full((np_, moe.FF), -3.0, device=gpu)
        ops.moe_up3s(pt, eoff, plist, dx, ckpt["gridf"], o["act"], layout=lay)
        o["act_w"] = torch.full_like(o["act"], -3.0)
        ops.moe_up3s_pairs(pt, deids, dx, ckpt["gridf"], o["act_w"], layout=lay)
        o["parts"] = torch.full((np_, moe.HID), -3.0, dtype=torch.float16, device=gpu)
        ops.moe_dn6(pd, items, nitp, eoff, plist, o["act"], o["parts"], layout=lay)
        o["parts_w"] = torch.full_like(o["parts"], -3.0)
        ops.moe_dn6_pairs(pd, deids, o["act"], o["parts_w"], layout=lay)
        buf = torch.full((np_ * moe.HID + 1,), -3.0, dtype=torch.float16, device=gpu)
        o["parts_u"] = buf[1:].view(np_, moe.HID)   # 2-B aligned: the staged form
        ops.moe_dn6(pd, items, nitp, eoff, plist, o["act"], o["parts_u"], layout=lay)
        o["act_sh"] = torch.full_like(o["act"], -3.0)
        o["sact"] = torch.full((P, moe.FF), -3.0, device=gpu)
        ops.moe_up3s_sh(pt, eoff, plist, dx, ckpt["gridf"], o["act_sh"], wg8, wu8, o["sact"], layout=lay)
        o["shared"] = torch.full((P, moe.HID), -3.0, device=gpu)
        o["parts_sh"] = torch.full_like(o["parts"], -3.0)
        ops.moe_dn6_sh(pd, items, nitp, eoff, plist, o["act"], o["parts_sh"], wd8, o["sact"], o["shared"], layout=lay)
        buf2 = torch.full((np_ * moe.HID + 1,), -3.0, dtype=torch.float16, device=gpu)
        o["parts_shu"] = buf2[1:].view(np_, moe.HID)
        ops.moe_dn6_sh(pd, items, nitp, eoff, plist, o["act"], o["parts_shu"], wd8, o["sact"], o["shared"],
                       layout=lay)
        torch.cuda.synchronize()
        return {k: v.cpu().numpy() for k, v in o.items()}

    raw, til = run(LAYOUT_RAW), run(LAYOUT_TILED)
    for k in raw:
        v = np.uint16 if raw[k].dtype == np.float16 else np.uint32
        assert np.array_equal(raw[k].view(v), til[k].view(v)), k
    _check_pairs(ckpt, x, eids, til["act"], til["parts"], list(range(0, np_, 7 if P <= 300 else 509)))


@pytest.mark.parametrize("P,lay", [(1, LAYOUT_RAW), (11, LAYOUT_TILED), (16, LAYOUT_RAW), (17, LAYOUT_TILED)])
def test_ckpt_pairs_shared_fused(gpu, ckpt, ckpt_tiled, P, lay):
    """moe_up3s_pairs_sh / moe_dn6_pairs_sh (the pair walks and the Q8_0 shared expert in one launch
    each at P <= 16, the two launches at P = 17) against moe_up3s_pairs / moe_dn6_pairs /
    moe_shared8, bit for bit; the shared expert against the oracle."""
    print(f"[case] pair walks + Q8_0 shared expert in one launch, P={P} layout={lay}", flush=True)
    rng = np.random.default_rng(90 + P)
    x, eids, deids, eoff, plist, items, nitp = _route(gpu, rng, P)
    dx = torch.from_numpy(x).to(gpu)
    np_ = 8 * P
    pt, pd = (ckpt["ptbl"], ckpt["ptbl_dn"]) if lay == LAYOUT_RAW else (ckpt_tiled["ptbl"], ckpt_tiled["ptbl_dn"])
    mk = lambda shape, dt, v: torch.full(shape, v, dtype=dt, device=gpu)
    sep = dict(act=mk((np_, moe.FF), torch.float32, -3.0), parts=mk((np_, moe.HID), torch.float16, -3.0),
               sact=mk((P, moe.FF), torch.float32, -3.0), shared=mk((P, moe.HID), torch.float32, -3.0))
    fus = {k: torch.full_like(v, -5.0) for k, v in sep.items()}
    wg8, wu8, wd8 = ckpt["dsh"]
    ops.moe_up3s_pairs(pt, deids, dx, ckpt["gridf"], sep["act"], layout=lay)
    ops.moe_dn6_pairs(pd, deids, sep["act"], sep["parts"], layout=lay)
    ops.moe_shared8(wg8, wu8, wd8, dx, sep["shared"], sep["sact"])
    ops.moe_up3s_pairs_sh(pt, deids, dx, ckpt["gridf"], fus["act"], wg8, wu8, fus["sact"], layout=lay)
    ops.moe_dn6_pairs_sh(pd, deids, fus["act"], fus["parts"], wd8, fus["sact"], fus["shared"], layout=lay)
    torch.cuda.synchronize()
    for k in sep:
        a, b = sep[k].cpu().numpy(), fus[k].cpu().numpy()
        v = np.uint16 if a.dtype == np.float16 else np.uint32
        assert np.array_equal(a.view(v), b.view(v)), k
    ref = moe.shared8_ref(*ckpt["shared"], x)
    assert _rows_err(fus["shared"].cpu().numpy(), ref) <= TOL


def test_ckpt_argument_validation(gpu, ckpt):
    dx = torch.zeros(2, moe.HID, device=gpu)
    act = torch.empty(16, moe.FF, dtype=torch.float32, device=gpu)
    eids = torch.zeros(16, dtype=torch.int16, device=gpu)
    with pytest.raises(ValueError):   # xs too small for 24 pairs (3 positions)
        ops.moe_up3s_pairs(ckpt["ptbl"], torch.zeros(24, dtype=torch.int16, device=gpu), dx, ckpt["gridf"],
                           torch.empty(24, moe.FF, dtype=torch.float32, device=gpu))
    with pytest.raises(TlxError):     # xs not 16-B aligned
        call("tlx_moe_up3s_pairs", ckpt["ptbl"].data_ptr(), eids.data_ptr(), dx.data_ptr() + 8,
             ckpt["gridf"].data_ptr(), act.data_ptr(), 16, LAYOUT_RAW, None)
    with pytest.raises(TlxError):     # more pairs than the sort supports
        call("tlx_moe_dn6_pairs", ckpt["ptbl_dn"].data_ptr(), eids.data_ptr(), act.data_ptr(), act.data_ptr(),
             16385, LAYOUT_TILED, None)


@pytest.mark.parametrize("P", [11, 300])
def test_ckpt_layer(gpu, ckpt, P):
    """ops.moe_layer_ckpt (top-8, pair walk at P=11 / sort + grouped forms at P=300, IQ3_S up,
    Q6_K down, Q8_0 shared, combine): every pair's act / parts and the shared expert against the
    oracle, y against the combine of the GPU's own parts and shared output."""
    print(f"[case] checkpoint-class MoE layer P={P}", flush=True)
    rng = np.random.default_rng(47 + P)
    x = synth.bf16_round(0.05 * rng.standard_normal((P, moe.HID)).astype(np.float32))
    logits = rng.standard_normal((P, moe.E)).astype(np.float32)
    sg = (1.0 / (1.0 + np.exp(-rng.standard_normal(P)))).astype(np.float32)
    hres = rng.standard_normal((P, moe.HID)).astype(np.float32)
    sc = ops.MoeScratch(P, gpu)
    y = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
    ops.moe_layer_ckpt(torch.from_numpy(logits).to(gpu), torch.from_numpy(sg).to(gpu), torch.from_numpy(x).to(gpu),
                       torch.from_numpy(hres).to(gpu), y, ckpt["ptbl"], ckpt["ptbl_dn"], ckpt["dsh"], ckpt["gridf"], sc)
    torch.cuda.synchronize()
    eids, gates = moe.topk_ref(logits)
    assert np.array_equal(sc.eids.cpu().numpy().view(np.uint16), eids)
    act, parts, shared = sc.act.cpu().numpy(), sc.parts.cpu().numpy(), sc.shared.cpu().numpy()
    pairs = list(range(8 * P)) if P <= 16 else sorted(np.random.default_rng(6).choice(8 * P, 40, replace=False))
    _check_pairs(ckpt, x, eids.reshape(-1), act, parts, pairs)
    wg, wu, wd = ckpt["shared"]
    assert _rows_err(shared, moe.shared8_ref(wg, wu, wd, x)) <= TOL
    pp = parts.reshape(P, 8, moe.HID)
    g = sc.gates.cpu().numpy()
    yref = moe.combine_ref(pp, g, sg, shared, hres)
    scale = np.abs(hres) + np.einsum("pr,prk->pk", np.abs(g), np.abs(pp.astype(np.float64))) + np.abs(sg)[:, None] * np.abs(shared)
    assert np.all(np.abs(y.cpu().numpy() - yref) <= 4e-6 * scale + 1e-30)


@pytest.mark.parametrize("P", [11, 300])
def test_ckpt_layer_graph_replays(gpu, ckpt, P):
    """ops.moe_layer_ckpt captured in a graph: every replay (eager work and synchronizations
    between them) equals the eager layer bit for bit, with the shared expert in the routed
    launches (P = 300) or its own (P = 11), and with it on a second stream."""
    rng = np.random.default_rng(70 + P)
    x = synth.bf16_round(0.05 * rng.standard_normal((P, moe.HID)).astype(np.float32))
    dl = torch.from_numpy(rng.standard_normal((P, moe.E)).astype(np.float32)).to(gpu)
    dsg = torch.from_numpy((1.0 / (1.0 + np.exp(-rng.standard_normal(P)))).astype(np.float32)).to(gpu)
    dh = torch.from_numpy(rng.standard_normal((P, moe.HID)).astype(np.float32)).to(gpu)
    dx = torch.from_numpy(x).to(gpu)
    for ov in (None, True):
        print(f"[case] checkpoint-class layer graph replays P={P} overlap={ov}", flush=True)
        sc = ops.MoeScratch(P, gpu)
        y = torch.empty(P, moe.HID, dtype=torch.float32, device=gpu)
        args = (dl, dsg, dx, dh, y, ckpt["ptbl"], ckpt["ptbl_dn"], ckpt["dsh"], ckpt["gridf"], sc)
        ops.moe_layer_ckpt(*args, overlap_shared=ov)
        torch.cuda.synchronize()
        ref = y.cpu().numpy().copy()
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            ops.moe_layer_ckpt(*args, stream=st, overlap_shared=ov)
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            ops.moe_layer_ckpt(*args, stream=st, overlap_shared=ov)
        for _ in range(3):
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
