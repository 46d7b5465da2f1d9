"""HIP kernels against the committed golden vectors (plain-Python brute
force, tests/golden/make_golden.py): decode (global GQA 8, window 7, ring
table + fused rel bias), prefill (causal, window 3), KV write (bit-exact)."""
import numpy as np
import pytest
import torch

from golden import load as golden
from helpers import assert_lse_close, assert_out_close
from oracle import kv_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("c", golden.cases("decode"), ids=lambda c: c["name"])
@pytest.mark.parametrize("wgs", [0, 3])
def test_decode_golden(tm, dev, c, wgs):
    table = torch.tensor(c["block_table"], dtype=torch.int32, device=dev)
    rel = c["rel"].to(dev) if c["rel"] is not None else None
    out, lse = tm.decode_paged(c["q"].to(dev), c["k_pool"].to(dev),
                               c["v_pool"].to(dev), table,
                               torch.tensor(c["ctx"], dtype=torch.int32,
                                            device=dev),
                               c["scale"], window=c["window"],
                               table_wrap=c["table_wrap"], rel=rel,
                               min_pages=1, num_workgroups=wgs)
    torch.cuda.synchronize()
    assert_out_close(out, c["out"], c["name"])
    assert_lse_close(lse, c["lse"], c["name"])


@pytest.mark.parametrize("c", golden.cases("prefill"),
                         ids=lambda c: c["name"])
def test_prefill_golden(tm, dev, c):
    out, lse = tm.prefill_varlen(c["q"].to(dev), c["k"].to(dev),
                                 c["v"].to(dev),
                                 torch.tensor(c["cu"], dtype=torch.int32,
                                              device=dev),
                                 c["scale"], window=c["window"])
    torch.cuda.synchronize()
    assert_out_close(out, c["out"], c["name"])
    assert_lse_close(lse, c["lse"], c["name"])


def test_kv_write_golden(tm, dev):
    c = golden.cases("kv_write")[0]
    pool = c["pool"].to(torch.bfloat16).to(dev)
    pv = torch.zeros_like(pool)
    k = c["k"].to(torch.bfloat16)
    tm.kv_write_paged(k.to(dev), k.to(dev),
                      torch.tensor(c["block_table"], dtype=torch.int32,
                                   device=dev),
                      torch.tensor(c["start"], dtype=torch.int32, device=dev),
                      pool, pv,
                      cu_seqlens=torch.tensor(c["cu"], dtype=torch.int32,
                                              device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(pool),
                          kv_ref.as_u16(c["want"].to(torch.bfloat16)))


@pytest.mark.parametrize("c", golden.cases("prefill_paged"),
                         ids=lambda c: c["name"])
def test_prefill_paged_golden(tm, dev, c):
    """Chunked prefill against the brute force: prior keys from a shuffled
    page pool (or a ring of 2 pages under a window of 20, with a 40-token
    chunk longer than the ring), the run's own keys from the pool (paged
    source) or from packed k/v (mixed source)."""
    table = torch.tensor(c["block_table"], dtype=torch.int32, device=dev)
    prior = torch.tensor(c["prior"], dtype=torch.int32, device=dev)
    cu = torch.tensor(c["cu"], dtype=torch.int32, device=dev)
    sources = ("mixed",) if c["table_wrap"] else ("paged", "mixed")
    for source in sources:
        own = source == "mixed"
        out, lse = tm.prefill_varlen(
            c["q"].to(dev), c["k"].to(dev) if own else None,
            c["v"].to(dev) if own else None, cu, c["scale"],
            window=c["window"], prior_lens=prior,
            k_pool=c["k_pool"].to(dev), v_pool=c["v_pool"].to(dev),
            block_table=table, table_wrap=c["table_wrap"])
        torch.cuda.synchronize()
        assert_out_close(out, c["out"], f"{c['name']} {source}")
        assert_lse_close(lse, c["lse"], f"{c['name']} {source}")
