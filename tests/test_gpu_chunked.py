"""Chunked prefill over the reference's own KV storage (compat.py): the
pooled adapters over SwaPool ring rows and GlobalPool pages
(engine/pyengine/kv.py:215-268), and the per-sequence adapter over a
PagedKV- / RingKV-shaped cache (kv.py:66-212). Checked against the fp32
oracle, the pools after the append bit-exact against the numpy oracle of
RingKV.append / PagedKV.append, and chunked == whole-prompt prefill for
the same tokens (the invariant a chunked scheduler relies on).
Tolerances: outputs 2e-2 + 1e-2 |ref|, LSE 1e-3."""
import numpy as np
import pytest
import torch

from helpers import PagedCache, RingCache, assert_out_close
from oracle import attn_ref, kv_ref

pytestmark = pytest.mark.gpu

D = 128


def _bf16(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    return cu


def test_chunk_swa_over_ring_rows(tm, dev):
    """SWA layer (64Q/16KV, W = E = 512): rings that have seen 0, 300, 512,
    2000 tokens take chunks of 700, 100, 1 and 513 tokens (longer than the
    ring, too), with the fused bias; afterwards every ring holds the last
    512 positions of its sequence."""
    g = torch.Generator().manual_seed(91)
    W, HK, H = 512, 16, 64
    prior = [0, 300, 512, 2000]
    lens = [700, 100, 1, 513]
    slots = torch.tensor([3, 0, 4, 1])
    S1 = 5 + 1
    pool_k = _bf16((S1, W, HK, D), g, 0.5)
    pool_v = _bf16((S1, W, HK, D), g, 0.5)
    cu = _cu(lens)
    T = int(cu[-1])
    q = _bf16((T, H, D), g)
    k = _bf16((T, HK, D), g)
    v = _bf16((T, HK, D), g)
    rel = _bf16((T, H, W), g, 0.5)
    per = W // 16
    table = (slots[:, None] * per + torch.arange(per)[None]).to(torch.int32)
    kp = pool_k.view(S1 * per, 16, HK, D)
    vp = pool_v.view(S1 * per, 16, HK, D)
    pr = torch.tensor(prior, dtype=torch.int32)
    ref, _ = attn_ref.prefill_varlen(q, k, v, cu, 1.0 / D, window=W,
                                     prior_lens=pr, k_pool=kp, v_pool=vp,
                                     block_table=table, table_wrap=per,
                                     rel=rel)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu.numpy(), prior, table.numpy(), 16, per)
    pk, pv = pool_k.to(dev), pool_v.to(dev)
    out = tm.attn_prefill_chunk_swa(q.to(dev), k.to(dev), v.to(dev),
                                    rel.to(dev), pk, pv, slots.to(dev),
                                    torch.tensor(prior, device=dev),
                                    cu.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref, "chunk swa")
    assert np.array_equal(kv_ref.as_u16(pk.view(S1 * per, 16, HK, D)),
                          want_k)


def test_chunk_global_over_page_table(tm, dev):
    """Global layer (64Q/8KV, E = 1024): GlobalPool pages through its int64
    device table, priors 0, 40 and 1000, the fused bias reaching back into
    the prior context; the chunks land where PagedKV.append puts them."""
    g = torch.Generator().manual_seed(92)
    HK, H, E = 8, 64, 1024
    prior = [0, 40, 1000]
    lens = [300, 77, 129]
    slots = torch.tensor([2, 0, 1])
    npg = 80
    total_pages = 4 * npg
    kp = _bf16((total_pages + 1, 16, HK, D), g, 0.5)
    vp = _bf16((total_pages + 1, 16, HK, D), g, 0.5)
    table_dev = torch.zeros((3 + 1, npg), dtype=torch.int64)
    table_dev[:3] = torch.randperm(total_pages, generator=g)[:3 * npg].view(
        3, npg)
    table_dev[3] = total_pages                      # scratch row
    cu = _cu(lens)
    T = int(cu[-1])
    q = _bf16((T, H, D), g)
    k = _bf16((T, HK, D), g)
    v = _bf16((T, HK, D), g)
    rel = _bf16((T, H, E), g, 0.5)
    table = table_dev[slots]
    pr = torch.tensor(prior, dtype=torch.int32)
    ref, _ = attn_ref.prefill_varlen(q, k, v, cu, 1.0 / D, prior_lens=pr,
                                     k_pool=kp, v_pool=vp, block_table=table,
                                     rel=rel)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu.numpy(), prior, table.numpy())
    kd, vd = kp.to(dev), vp.to(dev)
    out = tm.attn_prefill_chunk_global(q.to(dev), k.to(dev), v.to(dev),
                                       rel.to(dev), kd, vd,
                                       table_dev.to(dev), slots.to(dev),
                                       torch.tensor(prior, device=dev),
                                       cu.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref, "chunk global")
    assert np.array_equal(kv_ref.as_u16(kd), want_k)


@pytest.mark.parametrize("kind", ["paged", "ring"])
def test_chunked_equals_whole_prompt(tm, dev, kind):
    """A 1,313-token prompt fed as chunks of 300, 700, 1, 250 and 62 tokens
    through prefill_chunk_state gives the whole-prompt prefill's rows (the
    packed-source kernel over all tokens at once, window 512 on the ring,
    causal on pages), with the fused bias."""
    g = torch.Generator().manual_seed(93)
    HK, H = 8, 64
    E = 512 if kind == "ring" else 1024
    chunks = [300, 700, 1, 250, 62]
    N = sum(chunks)
    q = _bf16((N, H, D), g)
    k = _bf16((N, HK, D), g)
    v = _bf16((N, HK, D), g)
    rel = _bf16((N, H, E), g, 0.5)
    qd, kd, vd, reld = q.to(dev), k.to(dev), v.to(dev), rel.to(dev)
    whole, _ = tm.prefill_varlen(
        qd, kd, vd, torch.tensor([0, N], dtype=torch.int32, device=dev),
        1.0 / D, window=E if kind == "ring" else 0, rel=reld)
    if kind == "paged":
        P = 2 * ((N + 15) // 16)
        g2 = torch.Generator().manual_seed(94)
        free = torch.randperm(P, generator=g2).tolist()
        cache = PagedCache(
            torch.zeros((P, 16, HK, D), dtype=torch.bfloat16, device=dev),
            torch.zeros((P, 16, HK, D), dtype=torch.bfloat16, device=dev),
            free, torch.zeros(P, dtype=torch.int64, device=dev))
    else:
        cache = RingCache(
            torch.zeros((E, HK, D), dtype=torch.bfloat16, device=dev),
            torch.zeros((E, HK, D), dtype=torch.bfloat16, device=dev))
    outs = []
    t0 = 0
    for T in chunks:
        sl = slice(t0, t0 + T)
        outs.append(tm.prefill_chunk_state(qd[sl], kd[sl], vd[sl], reld[sl],
                                           cache))
        t0 += T
    torch.cuda.synchronize()
    assert cache.n == N
    got = torch.cat(outs)
    assert_out_close(got, whole.float(), f"chunked == whole ({kind})")
    # and against the oracle's whole-prompt prefill
    ref, _ = attn_ref.prefill_varlen(q, k, v, torch.tensor([0, N]), 1.0 / D,
                                     window=E if kind == "ring" else 0,
                                     rel=rel)
    assert_out_close(got, ref, f"chunked vs oracle ({kind})")
