"""Config 5 (mixed continuous-batching step) parity: one global and one
sliding-window layer of the full-size step, run through the same three
launches the captured step uses (KV append, chunked paged prefill, paged
decode), checked on sampled rows against the fp32 oracle reading the pool
state after the append; the appended tokens are checked bit-exact; then the
whole 66-layer step is captured as one hipGraph and replayed twice, each
replay matching the eager step bitwise."""
from importlib import import_module

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def step(dev):
    wl = import_module("tm-opt_amd.workloads")
    return wl.config5(device="cuda")


def _rows(step, l, rows):
    """Compact CPU copy of the pages the given table rows reference."""
    kp, vp = step.pool(l)
    t = step.tables[l][rows].long()
    pages = torch.unique(t)
    remap = torch.full((kp.shape[0],), -1, dtype=torch.long,
                       device=t.device)
    remap[pages] = torch.arange(pages.numel(), device=t.device)
    return kp[pages].cpu(), vp[pages].cpu(), remap[t].cpu()


@pytest.mark.parametrize("layer", [0, 3])
def test_config5_layer_sampled(tm, dev, step, layer):
    graph = import_module("tm-opt_amd.graph")
    ms = graph.MixedStepGraph(step)
    ms.layer(layer)
    torch.cuda.synchronize()
    nc = ms.n_chunks
    w = 0 if step.is_global[layer] else step.window
    # decode rows
    pick = [0, 5, 17, 40, 77, 95]
    kc, vc, tc = _rows(step, layer, [nc + b for b in pick])
    ctx = step.dec_ctx.cpu()[pick]
    ref_o, ref_l = attn_ref.decode_paged(step.q_decode.cpu()[pick], kc, vc,
                                         tc, ctx, step.scale, window=w)
    assert_out_close(ms.out_d.cpu()[pick], ref_o, f"C5 L{layer} decode")
    assert_lse_close(ms.lse_d.cpu()[pick], ref_l, f"C5 L{layer} decode")
    # chunked prefill: query rows of both chunks at sampled offsets
    kc, vc, tc = _rows(step, layer, list(range(nc)))
    prior = step.chunk_prior
    qp = step.q_prefill.cpu()
    outp = ms.out_p.cpu()
    for c in range(nc):
        for j in (0, 1, 63, 64, 1000, 2047):
            r = c * step.chunk_lens[0] + j
            pos = prior[c] + j
            lo = max(0, pos - w + 1) if w else 0
            kpos = torch.arange(lo, pos + 1)
            pages = tc[c][kpos // 16]
            K = kc[pages, kpos % 16].float()
            V = vc[pages, kpos % 16].float()
            rep = qp.shape[1] // K.shape[1]
            s = torch.einsum("hd,nhd->hn", qp[r].float(),
                             K.repeat_interleave(rep, 1)) * step.scale
            ref = torch.einsum("hn,nhd->hd", torch.softmax(s, -1),
                               V.repeat_interleave(rep, 1))
            assert_out_close(outp[r], ref, f"C5 L{layer} chunk{c} q{j}")
    # the appended tokens landed where the table says (bit-exact)
    kp, _ = step.pool(layer)
    t = step.tables[layer]
    for r, tok in ((0, 0), (1, 2047), (nc + 7, None)):
        pos = int(step.start_all[r]) + (0 if tok is None else tok)
        row = int(step.cu_all[r]) + (0 if tok is None else tok)
        pg = int(t[r, pos // 16])
        assert torch.equal(kp[pg, pos % 16], step.k_new[row])


def test_config5_step_graph(tm, dev, step):
    graph = import_module("tm-opt_amd.graph")
    ms = graph.MixedStepGraph(step).capture()
    outs = []
    for _ in range(2):
        ms.replay()
        torch.cuda.synchronize()
        outs.append((ms.out_p.clone(), ms.out_d.clone(), ms.lse_d.clone()))
        torch.cuda.synchronize()
    ms.run_eager()
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o[0], ms.out_p) and torch.equal(o[1], ms.out_d)
        assert torch.equal(o[2], ms.lse_d)
    assert torch.isfinite(ms.out_p.float()).all()
    assert torch.isfinite(ms.out_d.float()).all()
