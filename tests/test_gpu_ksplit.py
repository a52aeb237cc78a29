"""The k-split form of the tiled-record GEMV: long-K single matrices (the down and output
projections, K >= 5632 in four whole-block ranges) with few enough tiles are computed by four
groups of workgroups, one per k-range over every tile; the last of a tile's four arrivals adds the
range partials in range order.

* iq3_gemv (fp16 out) and down8 (fp32 residual out) stay within the path's rel-err 1e-3 of the
  oracle on the shapes that take the form: the fewest tiles it allows (one tile per workgroup of a
  group), the most, a tail tile, and the config 2/3 down / output projection shapes.
* Rows of an M-row call are bit-identical to M=1 calls of the same rows (the split depends on N, K
  and the device only; M changes where the activations are read from, not the arithmetic), at M
  where the activation slice is staged in LDS and where it is not.
* Repeated calls agree bit for bit (the per-tile arrival counters return to zero by themselves).
"""
import numpy as np
import pytest
import torch

from oracle import gemv, quants
from thunderllamax_amd import formats, ops, synth
from thunderllamax_amd._lib import LAYOUT_TILED

pytestmark = pytest.mark.gpu
TOL = 1e-3

# (N, K): 5120 x 17408 down projection, 5120 x 6144 output projection, 64 tiles (one per
# workgroup of a group) at K = 8192, 512 tiles (8 per workgroup) at K = 6144, and 65 tiles with a
# half-full tail tile
SHAPES = [(5120, 17408), (5120, 6144), (1024, 8192), (8192, 6144), (1032, 6144)]


def _mat(gpu, rng, N, K):
    packed = formats.iq3_pack_rows(synth.iq3xxs_raw(rng, N, K), K)
    t = torch.empty(-(-N // 16) * 16 * 102 * (K // 256), dtype=torch.uint8, device=gpu)
    ops.pack_iq3_tiled(torch.from_numpy(packed).to(gpu), t, N, K)
    return packed, t


def _rows_err(y, ref):
    return max(gemv.rel_err(y[m], ref[m]) for m in range(ref.shape[0]))


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 11, 16])
def test_ksplit_parity(gpu, N, K, M):
    print(f"[case] k-split iq3_gemv / down8 tiled M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(21)
    p, t = _mat(gpu, rng, N, K)
    g = formats.gridf_tensor(gpu)
    x = synth.activations_f16(rng, M, K)
    hh = rng.standard_normal((M, N)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    o = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    y = torch.full((M, N), float("nan"), device=gpu)
    ops.iq3_gemv(t, g, xd, o, layout=LAYOUT_TILED)
    ops.down8(t, g, xd, torch.from_numpy(hh).to(gpu), y, layout=LAYOUT_TILED)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(4).choice(N, min(N, 192), replace=False))
    rows = np.union1d(rows, [N - 1])   # the tail tile's last row
    W = quants.dequant_iq3xxs_packed(p[rows], K)
    _, oref = gemv.gemv16_ref(W, x)
    _, yref = gemv.down8_ref(W, x, hh[:, rows])
    eo = _rows_err(o.cpu().numpy()[:, rows], oref)
    ey = _rows_err(y.cpu().numpy()[:, rows], yref)
    print(f"[k-split M={M} N={N} K={K}] iq3_gemv rel-err {eo:.3e}; down8 {ey:.3e}")
    assert eo <= TOL and ey <= TOL
    assert not torch.isnan(o).any() and not torch.isnan(y).any()


@pytest.mark.parametrize("N,K", [(5120, 17408), (5120, 6144)])
def test_ksplit_rows_independent_of_m_and_repeatable(gpu, N, K):
    print(f"[case] k-split rows across M / repeated calls N={N} K={K}", flush=True)
    rng = synth.config_rng(22)
    _, t = _mat(gpu, rng, N, K)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(synth.activations_f16(rng, 16, K)).to(gpu)
    hh = torch.randn(16, N, device=gpu)
    one = torch.empty(16, N, dtype=torch.float16, device=gpu)
    one_y = torch.empty(16, N, device=gpu)
    for m in range(16):
        ops.iq3_gemv(t, g, x[m:m + 1], one[m:m + 1], layout=LAYOUT_TILED)
        ops.down8(t, g, x[m:m + 1], hh[m:m + 1], one_y[m:m + 1], layout=LAYOUT_TILED)
    for M in (4, 11, 16):
        o = torch.empty(M, N, dtype=torch.float16, device=gpu)
        y = torch.empty(M, N, device=gpu)
        for rep in range(2):
            ops.iq3_gemv(t, g, x[:M], o, layout=LAYOUT_TILED)
            ops.down8(t, g, x[:M], hh[:M], y, layout=LAYOUT_TILED)
            torch.cuda.synchronize()
            assert torch.equal(o, one[:M]), (M, rep)
            assert torch.equal(y, one_y[:M]), (M, rep)


@pytest.mark.parametrize("N,K", [(6144, 5120), (5120, 6144), (5120, 17408)])
@pytest.mark.parametrize("M", [1, 11, 16])
def test_tileord_input_staged_equals_row_major(gpu, N, K, M):
    """Activations handed over in the tile-ordered form are staged into LDS like row-major ones
    where the (range's) rows fit, and read from memory where they do not (M = 16 at K = 17408):
    the outputs equal the row-major call's bit for bit, with and without the k-split."""
    print(f"[case] tile-ordered input iq3_gemv M={M} N={N} K={K}", flush=True)
    rng = synth.config_rng(23)
    _, t = _mat(gpu, rng, N, K)
    g = formats.gridf_tensor(gpu)
    x = torch.from_numpy(synth.activations_f16(rng, M, K)).to(gpu)
    xt = ops.tileord_empty(K, gpu)
    xt.copy_(torch.cat([x, x[-1:].expand(16 - M, K)]).reshape(16, K // 8, 8).permute(1, 0, 2))
    o = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ot = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ops.iq3_gemv(t, g, x, o, layout=LAYOUT_TILED)
    ops.iq3_gemv(t, g, xt, ot, layout=LAYOUT_TILED, in_tileord=True, m=M)
    torch.cuda.synchronize()
    assert torch.equal(o, ot)
