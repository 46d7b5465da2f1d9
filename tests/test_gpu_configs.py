"""BASELINE configs 2 and 3 at full size, launched exactly as bench.py
launches them, checked on every sequence against the fp32 oracle.

C2: global paged decode, B=64, 32Q/4KV, ctx U[1024, 8192], block size 16,
shuffled pool of twice the needed pages. C3: window-4096 decode, B=128,
ctx U[2048, 32768]; only the window's pages are backed and every logical
page before a sequence's window points at one NaN page, so a read of any
page the window excludes poisons that row. Both run at the bench launch
(default persistent grid, min_pages 8) and at the grid config 5's step gives
the decode beside its prefill (two thirds of the default). Tolerances
outputs 2e-2 + 1e-2 |ref|, LSE 1e-3.
"""
from importlib import import_module

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _wl():
    return import_module("tm-opt_amd.workloads")


def _compact(case):
    """CPU copy of the pages the block table references (the pools are
    GBs; the oracle reads only these), with the table renumbered."""
    t = case.block_table.long()
    pages = torch.unique(t[t >= 0])
    remap = torch.full((case.k_pool.shape[0],), -1, dtype=torch.long,
                       device=t.device)
    remap[pages] = torch.arange(pages.numel(), device=t.device)
    tc = torch.where(t >= 0, remap[t.clamp(min=0)], t)
    return case.k_pool[pages].cpu(), case.v_pool[pages].cpu(), tc.cpu()


@pytest.fixture(scope="module", params=["C2", "C3"])
def config(request, dev):
    wl = _wl()
    make = wl.config2 if request.param == "C2" else wl.config3
    case = make(device="cuda", poison=True)
    kc, vc, tc = _compact(case)
    ref = attn_ref.decode_paged(case.q.cpu(), kc, vc, tc,
                                case.ctx_lens.cpu(), case.scale,
                                window=case.window)
    return request.param, case, ref


@pytest.mark.parametrize("grid", ["bench", "c5_step"])
def test_full_config_every_sequence(tm, dev, config, grid):
    name, case, (ref_o, ref_l) = config
    HKV = case.k_pool.shape[2]
    wgs = 0 if grid == "bench" else max(
        1, tm.decode_default_workgroups(HKV) * 2 // 3)
    ws = tm.decode_workspace(case.B, case.q.shape[1], HKV, dev, wgs)
    out, lse = tm.decode_paged(case.q, case.k_pool, case.v_pool,
                               case.block_table, case.ctx_lens, case.scale,
                               window=case.window, min_pages=8,
                               num_workgroups=wgs, workspace=ws)
    torch.cuda.synchronize()
    what = f"{name} grid={grid} ({wgs or 'default'} work-groups)"
    assert_out_close(out, ref_o, what)
    assert_lse_close(lse, ref_l, what)

