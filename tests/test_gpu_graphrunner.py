"""The reference-signature adapters captured with GraphRunner's semantics
(graph.AttnGraphRunner; engine/pyengine/graphrun.py:76-380): rows padded to
max_batch with dead rows on the scratch slot / page, one program per
512-token L_pad bucket captured on first sight under the dead-row config,
a monotone high-water mark. A schedule of decode steps in which a row
crosses the 511 -> 512 bucket edge, a sequence is admitted at position
1400 and another one finishes: every replay's live rows match the fp32
oracle over the pools as the step's own append left them, the buckets and
the number of captures follow the reference's rule, and the live rows'
appended tokens land bit-exact. Mirrors the reference's graph arms
(t_graph_ab.py, t_graphrun.py). Tolerances: 2e-2 + 1e-2 |ref| (BASELINE)."""
from importlib import import_module

import pytest
import torch

from helpers import assert_out_close
from oracle import attn_ref, geometry

pytestmark = pytest.mark.gpu

D, HQ = 128, 64


def test_graphed_adapters_across_buckets(tm, dev):
    graph = import_module("tm-opt_amd.graph")
    g = torch.Generator().manual_seed(95)
    MB, W = 6, 512
    HKg, HKs, E = 8, 16, 1024
    num_pages = 128                     # reach 2048 positions per sequence
    total = MB * num_pages
    bf = torch.bfloat16
    kp = (torch.randn((total + 1, 16, HKg, D), generator=g) * .5).to(bf)
    vp = (torch.randn((total + 1, 16, HKg, D), generator=g) * .5).to(bf)
    table_dev = torch.zeros((MB + 1, num_pages), dtype=torch.int64)
    table_dev[:MB] = torch.randperm(total, generator=g).view(MB, num_pages)
    table_dev[MB] = total                               # scratch page
    sk = (torch.randn((MB + 1, W, HKs, D), generator=g) * .5).to(bf)
    sv = (torch.randn((MB + 1, W, HKs, D), generator=g) * .5).to(bf)
    layers = [
        {"kind": "global", "kp": kp.to(dev), "vp": vp.to(dev),
         "table_dev": table_dev.to(dev), "rel_extent": E},
        {"kind": "swa", "k": sk.to(dev), "v": sv.to(dev)},
    ]
    runner = graph.AttnGraphRunner(layers, MB, HQ, device=dev)
    # (slot, position) of the live rows per step, in admission order
    A, B, C = 2, 0, 4
    schedule = [
        [(A, 10), (B, 509)],
        [(A, 11), (B, 510)],
        [(A, 12), (B, 511)],
        [(A, 13), (B, 512)],                # bucket 512 -> 1024
        [(A, 14), (B, 513), (C, 1400)],     # admission: bucket 1536
        [(A, 15), (C, 1401)],               # B finished: bucket stays 1536
    ]
    want_buckets = []
    hw = 0
    for rows in schedule:
        hw = geometry.bucket_len(max(p for _, p in rows), hw,
                                 cap=num_pages * 16)
        want_buckets.append(hw)
    assert want_buckets == [512, 512, 512, 1024, 1536, 1536]
    for step, rows in enumerate(schedule):
        slots = [s for s, _ in rows]
        pos = [p for _, p in rows]
        nb = len(rows)
        for l in range(2):
            for buf in (runner.q[l], runner.k_new[l], runner.v_new[l],
                        runner.rel[l]):
                buf[:nb].copy_((torch.randn(buf[:nb].shape, generator=g) *
                                (0.5 if buf is runner.rel[l] else 1.0))
                               .to(bf))
        L_pad = runner.step(pos, slots)
        torch.cuda.synchronize()
        assert L_pad == want_buckets[step]
        # the oracle over the pools as the replay's append left them
        ps = torch.tensor(pos)
        sl = torch.tensor(slots)
        q0 = runner.q[0][:nb].cpu()
        ref, _ = attn_ref.decode_paged(
            q0, layers[0]["kp"].cpu(), layers[0]["vp"].cpu(),
            table_dev[sl], ps + 1, 1.0 / D, rel=runner.rel[0][:nb].cpu())
        assert_out_close(runner.out[0][:nb], ref, f"global step {step}")
        ref, _ = attn_ref.decode_reference_semantics(
            runner.q[1][:nb].cpu(), layers[1]["k"].cpu(),
            layers[1]["v"].cpu(), sl, ps, runner.rel[1][:nb].cpu(), W)
        assert_out_close(runner.out[1][:nb], ref, f"swa step {step}")
        # the live rows' new tokens landed where model.py:938-948 puts them
        for i, (s, p) in enumerate(rows):
            pg = int(table_dev[s, p // 16])
            assert torch.equal(layers[0]["kp"][pg, p % 16],
                               runner.k_new[0][i])
            assert torch.equal(layers[1]["k"][s, p % W], runner.k_new[1][i])
    assert runner.captures == 3
