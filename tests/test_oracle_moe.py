"""Pins the MoE oracle (router top-8, sort, expert FFN, combine) against library routines and
closed forms, independently of how the oracle restates them."""
import numpy as np
import pytest
from scipy.special import expit, softmax

from oracle import moe


def _logits_with_ties(rng, P):
    lg = rng.standard_normal((P, moe.E)).astype(np.float32)
    for p in range(0, P, 3):           # plant exact ties among the leaders
        top = np.argsort(-lg[p])[:10]
        lg[p, top[5]] = lg[p, top[2]]
        lg[p, rng.integers(0, moe.E)] = lg[p, top[0]]
    return lg


def test_topk_matches_stable_argsort_and_softmax():
    rng = np.random.default_rng(0)
    lg = _logits_with_ties(rng, 40)
    eids, gates = moe.topk_ref(lg)
    want = np.argsort(-lg, axis=1, kind="stable")[:, :moe.TOPK]   # ties: lower id first
    assert np.array_equal(eids.astype(np.int64), want)
    for p in range(lg.shape[0]):
        np.testing.assert_allclose(gates[p], softmax(lg[p, want[p]].astype(np.float64)), rtol=1e-6)


def test_route_shared_gate_is_sigmoid_of_dot():
    rng = np.random.default_rng(1)
    wrt = rng.standard_normal((moe.E, moe.HID)).astype(np.float32) * 0.02
    wsh = rng.standard_normal(moe.HID).astype(np.float32) * 0.02
    h = rng.standard_normal((3, moe.HID)).astype(np.float32)
    lg64, eids, _, sg = moe.route_ref(wrt, wsh, h)
    np.testing.assert_allclose(lg64, np.einsum("ek,pk->pe", wrt.astype(np.float64), h.astype(np.float64)), rtol=1e-12)
    np.testing.assert_allclose(sg, expit(h.astype(np.float64) @ wsh.astype(np.float64)), rtol=1e-6)
    assert eids.shape == (3, moe.TOPK)


@pytest.mark.parametrize("n", [1, 88, 1000])
def test_sort_matches_python_sorted(n):
    rng = np.random.default_rng(n)
    e = rng.integers(0, moe.E, size=n).astype(np.uint16)
    eoff, plist = moe.sort_ref(e)
    assert np.array_equal(plist.astype(np.int64), np.array(sorted(range(n), key=lambda i: (int(e[i]), i))))
    assert np.array_equal(eoff, np.searchsorted(np.sort(e.astype(np.int64)), np.arange(moe.E + 1)))


def _const_iq4_rows(rows, kdim, qbyte):
    """IQ4_XS rows whose every weight is kv[qbyte & 15] (low) / kv[qbyte >> 4] (high):
    d = 1.0, ls = 33 for every group (dl = 1)."""
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.uint16(0xAAAA).tobytes(), np.uint8)   # high 2 bits of ls = 2
    blk[4:8] = 0x11                                                    # low 4 bits of ls = 1
    blk[8:136] = qbyte
    return np.tile(blk, (rows, kdim // 256))


def test_expert_ffn_closed_form():
    # gate weights kv[8] = 1 (g = s = sum(x)), up weights kv[9] = 13 (u = 13 s): act = silu(s) * 13 s.
    # The halves differ, so reading the up rows as gate (silu(13 s) * s) or a wrong GATE_B4 offset
    # (/root/reference/engine/mm/MM_P2_gx8e256up4.cu:22) fails.  Every down weight kv[9] = 13.
    gu = np.concatenate([_const_iq4_rows(moe.FF, moe.HID, 0x88).ravel(), _const_iq4_rows(moe.FF, moe.HID, 0x99).ravel()])
    dn = _const_iq4_rows(moe.HID, moe.FF, 0x99).ravel()
    x = 0.02 * np.random.default_rng(2).standard_normal((4, moe.HID))   # s = sum(x) of order 1
    s = x.sum(axis=1)
    act = moe.up_ref(gu, x)
    np.testing.assert_allclose(act, np.repeat((s / (1 + np.exp(-s)) * 13.0 * s)[:, None], moe.FF, axis=1), rtol=1e-12)
    swapped = (13.0 * s / (1 + np.exp(-13.0 * s))) * s
    assert np.all(np.abs(act[:, 0] - swapped) > 1e-3 * np.abs(swapped))
    part = moe.down_ref(dn, act)
    np.testing.assert_allclose(part, np.repeat(13.0 * act.sum(axis=1)[:, None], moe.HID, axis=1), rtol=1e-12)


def _const_iq3s_rows(rows, kdim, nib):
    """IQ3_S rows whose weights are all d (1 + 2 nib) * grid[0][c] with d = 1/64 and no signs."""
    blk = np.zeros(110, np.uint8)
    blk[0:2] = np.array([1 / 64], np.float16).view(np.uint8)
    blk[106:110] = nib | (nib << 4)
    return np.tile(blk, (rows, kdim // 256))


def _const_q80_rows(rows, kdim, q):
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([1 / 64], np.float16).view(np.uint8)
    blk[2:34] = np.int8(q).view(np.uint8)
    return np.tile(blk, (rows, kdim // 32))


def test_checkpoint_classes_closed_form():
    """IQ3_S gate+up (grid all ones: gate nibble 0 -> d, up nibble 1 -> 3d, so act = silu(ds) * 3ds
    and a swap of the halves or a wrong 450,560-B offset fails), Q6_K down (q = 33, sc = 1,
    d = 1/16: every weight 1/16), the Q8_0 shared expert (q = 2, 3, 5 for gate, up, down)."""
    grid = np.ones((512, 4), np.float32)
    gu = np.concatenate([_const_iq3s_rows(moe.FF, moe.HID, 0).ravel(), _const_iq3s_rows(moe.FF, moe.HID, 1).ravel()])
    x = 0.5 * np.random.default_rng(4).standard_normal((3, moe.HID))
    s = x.sum(axis=1) / 64
    act = moe.up3s_ref(gu, grid, x)
    np.testing.assert_allclose(act, np.repeat((s / (1 + np.exp(-s)) * 3 * s)[:, None], moe.FF, axis=1), rtol=1e-12)
    swapped = (3 * s / (1 + np.exp(-3 * s))) * s
    assert np.all(np.abs(act[:, 0] - swapped) > 1e-3 * np.abs(swapped))
    q6 = np.zeros(210, np.uint8)
    q6[0:128] = 0x11            # ql nibbles 1
    q6[128:192] = 0xAA          # qh: 2 in every 2-bit field -> q = 1 | 32 = 33
    q6[192:208] = 1             # sc = 1
    q6[208:210] = np.array([1 / 16], np.float16).view(np.uint8)
    dn = np.tile(q6, (moe.HID, moe.FF // 256))
    part = moe.down6_ref(dn, act)
    np.testing.assert_allclose(part, np.repeat(act.sum(axis=1)[:, None] / 16, moe.HID, axis=1), rtol=1e-12)
    wg, wu, wd = _const_q80_rows(moe.FF, moe.HID, 2), _const_q80_rows(moe.FF, moe.HID, 3), _const_q80_rows(moe.HID, moe.FF, 5)
    g, u = 2 * x.sum(axis=1) / 64, 3 * x.sum(axis=1) / 64
    y = moe.shared8_ref(wg, wu, wd, x)
    np.testing.assert_allclose(y, np.repeat((5 / 64 * moe.FF * g / (1 + np.exp(-g)) * u)[:, None], moe.HID, axis=1),
                               rtol=1e-12)


def test_combine_one_hot_gates():
    rng = np.random.default_rng(3)
    P = 5
    parts = rng.standard_normal((P, moe.TOPK, moe.HID))
    gates = np.zeros((P, moe.TOPK))
    gates[np.arange(P), np.arange(P) % moe.TOPK] = 1.0
    sg = rng.random(P)
    shared = rng.standard_normal((P, moe.HID))
    hres = rng.standard_normal((P, moe.HID))
    y = moe.combine_ref(parts, gates, sg, shared, hres)
    np.testing.assert_allclose(y, hres + parts[np.arange(P), np.arange(P) % moe.TOPK] + sg[:, None] * shared)
