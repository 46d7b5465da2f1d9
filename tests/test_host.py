"""CPU checks of the package's host-side logic (no GPU): the table math
the adapters hand to the kernels."""
from importlib import import_module

import pytest
import torch


@pytest.mark.parametrize("B,T", [(1, 8), (3, 200), (6, 1536), (5, 24), (2, 16)])
def test_pack_meta_is_an_identity_layout(B, T):
    """The identity tables that pack channel-major K/V through the paged
    write (compat._pack_meta): under the page rule, position start + i of
    row b is packed row b*T + i for every i < T, and no table entry read for
    those positions leaves the buffer."""
    compat = import_module("tm-opt_amd.compat")
    meta = compat._pack_meta(B, T, "cpu")
    P = (B * T + 15) // 16
    for b in range(B):
        start, lo, n = (int(x) for x in meta[b, :3])
        assert (lo, n) == (0, T)
        pos = start + torch.arange(T)
        table = meta[b, 3:]
        assert int(pos[-1]) // 16 < table.numel()
        rows = table[pos // 16].long() * 16 + pos % 16
        assert torch.equal(rows, b * T + torch.arange(T))
        assert int(table[pos // 16].max()) < P
