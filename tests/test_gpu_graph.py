"""hipGraph capture of the decode step (tm-opt_amd/graph.py): one capture,
several replays with fresh inputs copied into the static buffers between
them (plus eager work and synchronisation in between, as replays must
survive), each replay checked bitwise against an eager run of the same step
on the same pool state and against the fp32 oracle. Mirrors the reference's
graph arms (t_graph_ab.py:67-104: eager vs graph, run1 == run2 bitwise)."""
from importlib import import_module

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _layers(dev, g, MB, HKV, D, ctx_max):
    # global layer: shuffled page pool covering every row's final length
    npg = (ctx_max + 15) // 16
    P = 2 * MB * npg + 1
    perm = torch.randperm(P - 1, generator=g)[:MB * npg]
    table_g = perm.view(MB, npg).to(torch.int32)
    kg = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    vg = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    # SWA layer: ring pool of W = 256 tokens per row, viewed as 16 pages
    W, per = 256, 16
    ks = torch.randn((MB * per, 16, HKV, D), generator=g).to(torch.bfloat16)
    vs = torch.randn((MB * per, 16, HKV, D), generator=g).to(torch.bfloat16)
    table_s = (torch.arange(MB)[:, None] * per +
               torch.arange(per)[None]).to(torch.int32)
    return [
        {"k_pool": kg.to(dev), "v_pool": vg.to(dev),
         "block_table": table_g.to(dev), "window": 0, "table_wrap": 0},
        {"k_pool": ks.to(dev), "v_pool": vs.to(dev),
         "block_table": table_s.to(dev), "window": W, "table_wrap": per},
        {"k_pool": kg.clone().to(dev), "v_pool": vg.clone().to(dev),
         "block_table": table_g.to(dev), "window": 100, "table_wrap": 0},
    ]


def test_decode_step_graph_replays(tm, dev):
    graph = import_module("tm-opt_amd.graph")
    g = torch.Generator().manual_seed(77)
    MB, HQ, HKV, D, steps = 8, 32, 4, 128, 4
    ctx0 = torch.tensor([1, 15, 16, 17, 300, 511, 512, 700])
    layers = _layers(dev, g, MB, HKV, D, int(ctx0.max()) + steps)
    dg = graph.DecodeStepGraph(layers, MB, HQ, HKV, device=dev)

    def fresh_inputs(step):
        dg.q.copy_(torch.randn(dg.q.shape, generator=g).to(torch.bfloat16))
        dg.k_new.copy_(torch.randn(dg.k_new.shape, generator=g).to(
            torch.bfloat16))
        dg.v_new.copy_(torch.randn(dg.v_new.shape, generator=g).to(
            torch.bfloat16))
        dg.ctx.copy_((ctx0 + 1 + step).to(torch.int32))

    fresh_inputs(0)
    dg.capture()     # warm-up writes this step's rows; replays rewrite them
    for step in range(steps):
        if step:
            fresh_inputs(step)
        snap = [(ly["k_pool"].clone(), ly["v_pool"].clone())
                for ly in layers]
        dg.replay()
        torch.cuda.synchronize()
        out_g, lse_g = dg.out.clone(), dg.lse.clone()
        pools_g = [(ly["k_pool"].clone(), ly["v_pool"].clone())
                   for ly in layers]
        for ly, (k, v) in zip(layers, snap):
            ly["k_pool"].copy_(k)
            ly["v_pool"].copy_(v)
        dg.run_eager()
        torch.cuda.synchronize()
        assert torch.equal(out_g, dg.out), f"step {step}: graph != eager"
        assert torch.equal(lse_g, dg.lse)
        for ly, (k, v) in zip(layers, pools_g):
            assert torch.equal(ly["k_pool"], k) and torch.equal(
                ly["v_pool"], v)
        # fp32 oracle over the pools as they stand after the append
        ctx = (ctx0 + 1 + step)
        for l, ly in enumerate(layers):
            ref_o, ref_l = attn_ref.decode_paged(
                dg.q[l].cpu(), ly["k_pool"].cpu(), ly["v_pool"].cpu(),
                ly["block_table"].cpu(), ctx, dg.scale,
                window=ly["window"], table_wrap=ly["table_wrap"])
            assert_out_close(out_g[l], ref_o, f"graph step {step} layer {l}")
            assert_lse_close(lse_g[l], ref_l, f"graph step {step} layer {l}")
        # the new token's K landed at position ctx-1 of every row
        ly = layers[0]
        for b in range(MB):
            p = int(ctx[b]) - 1
            pg = int(ly["block_table"][b, p // 16])
            assert torch.equal(ly["k_pool"][pg, p % 16], dg.k_new[0, b])


def test_prefill_fused_first_call_in_capture(tm, dev):
    """attn_prefill_fused with channel-major K/V and the fused bias,
    captured in a hipGraph (its run offsets and the position check are then
    built inside the capture): every replay, with eager work and a
    synchronisation between replays, equals the eager call bitwise."""
    compat = import_module("tm-opt_amd.compat")
    g = torch.Generator().manual_seed(23)
    B, T, D, hq, hk, W = 2, 136, 128, 32, 4, 64
    q = torch.randn((B, T, hq, D), generator=g).to(torch.bfloat16).to(dev)
    kc = torch.randn((B, hk, D, T), generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn((B, hk, D, T), generator=g).to(torch.bfloat16).to(dev)
    rel = (torch.randn((B, T, hq, W), generator=g) * 0.5).to(
        torch.bfloat16).to(dev)
    args = (q.transpose(1, 2), kc.transpose(2, 3), vc.transpose(2, 3),
            rel.transpose(1, 2), torch.arange(T, device=dev),
            torch.arange(T, device=dev), W)
    eager = tm.attn_prefill_fused(*args)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = tm.attn_prefill_fused(*args)
    for _ in range(3):
        graph.replay()
        noise = torch.randn((1 << 20,), device=dev) * 2.0   # eager work
        torch.cuda.synchronize()
        del noise
        assert torch.equal(out, eager)
