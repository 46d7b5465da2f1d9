"""Shared comparison helpers for the parity tests."""
import torch

# Tolerances from BASELINE.json: attention outputs max-abs 2e-2 / rtol
# 1e-2 against the fp32 oracle, LSE within 1e-3 (absolute, natural log).
OUT_ATOL = 2e-2
OUT_RTOL = 1e-2
LSE_ATOL = 1e-3


def assert_out_close(got, ref, what=""):
    got = got.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    err = (got - ref).abs()
    bound = OUT_ATOL + OUT_RTOL * ref.abs()
    bad = err > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.numel()} outputs outside "
        f"atol {OUT_ATOL} + rtol {OUT_RTOL}; max err {float(err.max()):.4g}")
    return float(err.max())


def assert_lse_close(got, ref, what=""):
    got = got.float().cpu()
    ref = ref.float().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got)), f"{what}: LSE finiteness"
    err = (got[fin] - ref[fin]).abs()
    m = float(err.max()) if err.numel() else 0.0
    assert m <= LSE_ATOL, f"{what}: LSE max err {m:.3g} > {LSE_ATOL}"
    return m


class PagedCache:
    """Shaped like the reference's pool-backed PagedKV (kv.py:117-212):
    shared pools, a host page list filled from a free list on demand and
    mirrored into a device table row, n tokens stored."""

    def __init__(self, kp, vp, free, table_dev_row):
        self.kp, self.vp = kp, vp
        self.free = free
        self.table_dev_row = table_dev_row
        self.page_size = 16
        self.table = []
        self.n = 0

    def ensure_pages(self, last_page):
        first = len(self.table)
        while len(self.table) <= last_page:
            self.table.append(self.free.pop(0))
        if len(self.table) > first:
            self.table_dev_row[first:len(self.table)] = torch.tensor(
                self.table[first:], device=self.table_dev_row.device)


class RingCache:
    """Shaped like the reference's RingKV (kv.py:66-114): a [W, HK, D] ring
    per K and V, position p at slot p % W, n tokens seen."""

    def __init__(self, k, v):
        self.k, self.v = k, v
        self.n = 0
