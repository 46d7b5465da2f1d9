"""The allocation-free decode entry point (tmopt_attn_decode_paged_noalloc:
the workspace is the library's static per-GPU scratch array) against the
workspace entry point tmopt_attn_decode_paged on the same inputs, through
the C ABI: two calls in a row, the second on a smaller input, each output
and LSE bitwise equal to the workspace entry point's (same kernels, same
split) and within the BASELINE tolerance of the fp32 oracle. A launch shape
needing more scratch than the static buffer is refused with
TMOPT_EWORKSPACE before anything runs."""
from importlib import import_module

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _both(tm, case, dev, **kw):
    c = case.to(dev)
    ref = tm.decode_paged(c.q, c.k_pool, c.v_pool, c.block_table, c.ctx_lens,
                          c.scale, window=c.window, **kw)
    out = torch.full_like(c.q, float("nan"))
    lse = torch.full(c.q.shape[:2], float("nan"), dtype=torch.float32,
                     device=dev)
    got = tm.decode_paged_noalloc(c.q, c.k_pool, c.v_pool, c.block_table,
                                  c.ctx_lens, c.scale, out, lse,
                                  window=c.window, **kw)
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_matches_workspace_entry(tm, dev):
    wl = import_module("tm-opt_amd.workloads")
    big = wl.config2(poison=True)                      # B=64, 4 MB scratch
    small = wl.make_decode("na_small", 82, 9, 1, 900, window=256)
    for case, kw in ((big, {}), (small, dict(min_pages=1,
                                             num_workgroups=37))):
        (ro, rl), (go, gl) = _both(tm, case, dev, **kw)
        assert torch.equal(go, ro) and torch.equal(gl, rl), case.name
        ref_o, ref_l = attn_ref.decode_paged(case.q, case.k_pool,
                                             case.v_pool, case.block_table,
                                             case.ctx_lens, case.scale,
                                             window=case.window)
        assert_out_close(go, ref_o, f"noalloc {case.name}")
        assert_lse_close(gl, ref_l, f"noalloc {case.name}")


def test_noalloc_refuses_oversized_launch(tm, dev):
    """(B + G) * HQ * 512 bytes of partials above 16 MiB: refused."""
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("na_big", 83, 2048, 1, 40, 0).to(dev)
    assert tm.decode_workspace_size(2048, 32, 4) > 16 << 20
    out = torch.empty_like(case.q)
    with pytest.raises(tm.TmoptError) as e:
        tm.decode_paged_noalloc(case.q, case.k_pool, case.v_pool,
                                case.block_table, case.ctx_lens, case.scale,
                                out)
    assert e.value.status == tm._lib.TMOPT_EWORKSPACE
