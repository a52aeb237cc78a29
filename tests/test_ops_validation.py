"""The Python entry points reject buffers too small for the shape and layout they are described
with, before any device call (the library itself sees only pointers)."""
import pytest
import torch

from thunderllamax_amd import ops


def _u8(n):
    return torch.zeros(n, dtype=torch.uint8)


def test_pfg3_rejects_packed_rows_given_for_packed7():
    M, N, K = 256, 256, 5120
    rows = _u8(N * 98 * (K // 256))          # packed rows: smaller than the packed7 units
    x = torch.zeros(M, K, dtype=torch.float16)
    out = torch.zeros(M, N, dtype=torch.float16)
    with pytest.raises(ValueError, match="packed7"):
        ops.pfg3_iq3o(rows, torch.zeros(1024), x, out)
    with pytest.raises(ValueError, match="packed7"):
        ops.pfg3_ffn(rows, rows, torch.zeros(1024), x, out)


def test_gemv_rejects_short_weights_and_outputs():
    M, N, K = 4, 64, 512
    x = torch.zeros(M, K, dtype=torch.float16)
    with pytest.raises(ValueError, match="wg"):
        ops.ffn8(_u8(N * 98 * 2 - 1), _u8(N * 98 * 2), torch.zeros(1024), x, torch.zeros(M, N, dtype=torch.float16))
    with pytest.raises(ValueError, match="hh"):
        ops.down8(_u8(N * 98 * 2), torch.zeros(1024), x, torch.zeros(M, N - 1), torch.zeros(M, N))


def test_moe_rejects_short_tables():
    P = 4
    with pytest.raises(ValueError, match="items"):
        ops.moe_sort(torch.zeros(P, 8, dtype=torch.int16), torch.zeros(257, dtype=torch.int32),
                     torch.zeros(8 * P, dtype=torch.int16), torch.zeros(3, dtype=torch.int32),
                     torch.zeros(1, dtype=torch.int32))
