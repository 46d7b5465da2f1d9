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
