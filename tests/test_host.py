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
    start, lens, table = compat._pack_meta(B, T, "cpu")
    P = (B * T + 15) // 16
    assert table.is_contiguous() and table.shape[0] == B
    assert torch.equal(lens, torch.full((B,), T, dtype=torch.int32))
    for b in range(B):
        pos = int(start[b]) + torch.arange(T)
        assert int(pos[-1]) // 16 < table.shape[1]
        rows = table[b][pos // 16].long() * 16 + pos % 16
        assert torch.equal(rows, b * T + torch.arange(T))
        assert int(table[b][pos // 16].max()) < P
