"""Parity of the HIP split-KV paged decode kernel against the fp32 oracle.

Tolerances: outputs max-abs 2e-2 / rtol 1e-2, LSE 1e-3.
Pools are NaN-poisoned outside the pages a sequence owns, so any stray read
shows up as a non-finite output. Geometry edges follow the reference's own arm
(engine/pyengine/tests/t_fused_attn.py:119-122): positions 0, 3, 200, 511,
512, 513, 800, 1500 and a dead row at position 0.
"""
import math

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu

EDGE_POS = [0, 3, 200, 511, 512, 513, 800, 1500, 0]


def _run(tm, case, dev, **kw):
    c = case.to(dev)
    out, lse = tm.decode_paged(c.q, c.k_pool, c.v_pool, c.block_table,
                               c.ctx_lens, c.scale, window=c.window, **kw)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _oracle(case, **kw):
    return attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                                 case.block_table, case.ctx_lens, case.scale,
                                 window=case.window, **kw)


def test_config1_global_decode(tm, dev):
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.config1(poison=True)
    ref_o, ref_l = _oracle(case)
    out, lse = _run(tm, case, dev)
    assert_out_close(out, ref_o, "C1")
    assert_lse_close(lse, ref_l, "C1")


@pytest.mark.parametrize("window", [0, 512])
@pytest.mark.parametrize("min_pages,wgs", [(1, 0), (1, 7), (3, 64), (8, 0),
                                           (128, 0)])
def test_edge_positions(tm, dev, window, min_pages, wgs):
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("edges", 7, len(EDGE_POS), 0, 0, window,
                          ctx=[p + 1 for p in EDGE_POS])
    ref_o, ref_l = _oracle(case)
    out, lse = _run(tm, case, dev, min_pages=min_pages, num_workgroups=wgs)
    what = f"edges w={window} min_pages={min_pages} wgs={wgs}"
    assert_out_close(out, ref_o, what)
    assert_lse_close(lse, ref_l, what)


@pytest.mark.parametrize("hq,hkv", [(64, 8), (64, 16), (32, 4), (16, 16),
                                    (32, 2), (12, 4), (6, 1), (15, 1),
                                    (96, 4), (64, 1), (17, 1), (40, 2)])
def test_gqa_shapes(tm, dev, hq, hkv):
    """GQA 1, 2, 4, 8, 16; ratios up to 16 that are not powers of two (3,
    6, 15: one read of the pages per KV head); ratios above 16 (24, 64, 17,
    20: groups of 8, 16, 1, 10 query heads per scheduled KV head)."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("gqa", 8, 6, 1, 700, 0, hq=hq, hkv=hkv)
    ref_o, ref_l = _oracle(case)
    out, lse = _run(tm, case, dev, min_pages=2, num_workgroups=40)
    assert_out_close(out, ref_o, f"gqa {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"gqa {hq}/{hkv}")


def test_window_only_reads_window_pages(tm, dev):
    """Pages before the window point at a NaN poison page; output finite and
    equal to the oracle (which never touches them either)."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("swa", 9, 12, 700, 5000, window=1000)
    assert (case.block_table == case.meta["pool_pages"] - 1).any()
    ref_o, ref_l = _oracle(case)
    out, lse = _run(tm, case, dev, min_pages=5)
    assert_out_close(out, ref_o, "swa")
    assert_lse_close(lse, ref_l, "swa")


def test_split_invariance_and_determinism(tm, dev):
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("inv", 10, 5, 900, 3000)
    outs = []
    for mp, wgs in ((1, 512), (2, 33), (7, 0), (64, 0), (4096, 1)):
        outs.append(_run(tm, case, dev, min_pages=mp, num_workgroups=wgs))
    base_o, base_l = outs[-1]          # one work-group walks everything
    for o, l in outs[:-1]:
        assert (o.float() - base_o.float()).abs().max() <= 2 * 2 ** -8 * \
            base_o.float().abs().max()
        assert (l - base_l).abs().max() <= 1e-4
    again = _run(tm, case, dev, min_pages=7, num_workgroups=0)
    assert torch.equal(again[0], outs[2][0]) and torch.equal(again[1],
                                                            outs[2][1])


def test_zero_query_closed_form(tm, dev):
    """q = 0: uniform weights, LSE = ln(n_visible), out = mean of visible V."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("q0", 11, 7, 1, 2000, window=333)
    case.q.zero_()
    out, lse = _run(tm, case, dev, min_pages=4)
    nv = case.visible().double()
    assert torch.allclose(lse.double(), torch.log(nv)[:, None].expand_as(lse),
                          atol=1e-4, rtol=0)
    ref_o, _ = _oracle(case)
    assert_out_close(out, ref_o, "q=0")


@pytest.mark.parametrize("HQ,HK", [(64, 16), (48, 4), (96, 4)])
def test_rel_bias_and_ring_table(tm, dev, HQ, HK):
    """The reference's SWA model semantics (attn_swa.py:120-141): ring pool
    [S, W, HK, D] viewed as pages, scale 1/D, fused rel bias of extent W;
    GQA 4, 12 and 24."""
    g = torch.Generator().manual_seed(5)
    S, W, D = 6, 512, 128
    pool_k = torch.randn((S + 1, W, HK, D), generator=g).to(torch.bfloat16)
    pool_v = torch.randn((S + 1, W, HK, D), generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 3, 200, 511, 512, 513, 800, 0])
    slots = torch.tensor([4, 0, 2, 5, 1, 3, 6, 6])
    B = pos.shape[0]
    q = torch.randn((B, HQ, D), generator=g).to(torch.bfloat16)
    rel = (torch.randn((B, HQ, W), generator=g) * 0.5).to(torch.bfloat16)
    ref_o, ref_l = attn_ref.decode_reference_semantics(q, pool_k, pool_v,
                                                       slots, pos, rel, W)
    per = W // 16
    kp = pool_k.view((S + 1) * per, 16, HK, D).to(dev)
    vp = pool_v.view((S + 1) * per, 16, HK, D).to(dev)
    table = (slots[:, None] * per + torch.arange(per)[None]).to(torch.int32)
    out, lse = tm.decode_paged(q.to(dev), kp, vp, table.to(dev),
                               (pos + 1).to(torch.int32).to(dev), 1.0 / D,
                               window=W, table_wrap=per, rel=rel.to(dev),
                               min_pages=2)
    torch.cuda.synchronize()
    assert_out_close(out, ref_o, f"ring+rel {HQ}/{HK}")
    assert_lse_close(lse, ref_l, f"ring+rel {HQ}/{HK}")


@pytest.mark.parametrize("k,wgs", [(1, 40), (3, 14), (7, 6), (40, 1)])
def test_ring_whole_rows_per_workgroup(tm, dev, k, wgs):
    """The ring decode with whole rows per work-group (seqs_per_workgroup:
    no row split, no merge launch): rows of every fill level (empty, one
    key, a partial first page, full rings, wrapped rings), B = 40 not a
    multiple of k, every row and LSE against the oracle; one work-group
    short of covering B is refused before launch."""
    g = torch.Generator().manual_seed(31)
    B, W, HK, D, HQ = 40, 256, 4, 128, 32
    S = B + 1
    pool_k = torch.randn((S, W, HK, D), generator=g).to(torch.bfloat16)
    pool_v = torch.randn((S, W, HK, D), generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 3 * W, (B,), generator=g)
    pos[:8] = torch.tensor([0, 1, 15, 16, 255, 256, 700, 40])
    slots = torch.randperm(B, generator=g)
    q = torch.randn((B, HQ, D), generator=g).to(torch.bfloat16)
    rel = (torch.randn((B, HQ, W), generator=g) * 0.5).to(torch.bfloat16)
    ref_o, ref_l = attn_ref.decode_reference_semantics(q, pool_k, pool_v,
                                                       slots, pos, rel, W)
    args = (q.to(dev), pool_k.to(dev), pool_v.to(dev), slots.to(dev),
            pos.to(dev), 1.0 / D, W)
    out, lse = tm.decode_ring(*args, rel=rel.to(dev), num_workgroups=wgs,
                              seqs_per_workgroup=k, return_lse=True)
    torch.cuda.synchronize()
    what = f"ring whole rows k={k} wgs={wgs}"
    assert_out_close(out, ref_o, what)
    assert_lse_close(lse, ref_l, what)
    if wgs > 1 and (wgs - 1) * k < B:
        with pytest.raises(tm.TmoptError):
            tm.decode_ring(*args, rel=rel.to(dev), num_workgroups=wgs - 1,
                           seqs_per_workgroup=k)


def test_table_from_flat(tm, dev):
    """attn_global's per-token rows (model.py:938-945) turned into the
    block table and lengths in one launch: bit-exact against the torch
    expressions flat[:, ::16] // 16 and pos + 1, for Lg a multiple of 16
    and not, rows of every length (dead columns 0)."""
    g = torch.Generator().manual_seed(32)
    for Lg in (1536, 1500, 17, 1):
        B = 9
        npg = (Lg + 15) // 16
        table_dev = torch.randperm(B * npg * 2, generator=g)[:B * npg].view(
            B, npg)
        pos = torch.randint(0, Lg, (B,), generator=g)
        pos[0] = Lg - 1
        j = torch.arange(Lg)
        flat = table_dev[:, j // 16] * 16 + (j % 16)[None]
        flat = torch.where(j[None] < (pos + 1)[:, None], flat,
                           torch.zeros((), dtype=torch.int64))
        table, ctx = tm.decode_table_from_flat(flat.contiguous().to(dev),
                                               pos.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(table.cpu(), (flat[:, ::16] // 16).to(torch.int32))
        assert torch.equal(ctx.cpu(), (pos + 1).to(torch.int32))


def test_empty_and_zero_length(tm, dev):
    """B == 0 is a no-op; a zero-length sequence yields 0 and LSE -inf."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("z", 12, 3, 5, 50)
    c = case.to(dev)
    c.ctx_lens[1] = 0
    out, lse = tm.decode_paged(c.q, c.k_pool, c.v_pool, c.block_table,
                               c.ctx_lens, c.scale, min_pages=1)
    torch.cuda.synchronize()
    assert torch.all(out[1].float() == 0)
    assert torch.all(torch.isinf(lse[1])) and torch.all(lse[1] < 0)
    ref_o, ref_l = attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                                         case.block_table,
                                         c.ctx_lens.cpu(), case.scale)
    assert_out_close(out, ref_o, "zero-len")
    e = tm.decode_paged(c.q[:0], c.k_pool, c.v_pool, c.block_table[:0],
                        c.ctx_lens[:0], c.scale)
    assert e[0].shape == (0, 32, 128)
    assert math.isfinite(float(lse[0].max()))


@pytest.mark.parametrize("window", [0, 700])
def test_rising_scores_rescale(tm, dev, window):
    """Scores that climb with the key position, so the running max of every
    split moves past the lazy threshold again and again and the partials
    are merged across very different maxima: key p of a sequence is
    s * 0.02 p + noise, the query 0.5 s + noise (s a +-1 pattern per KV
    head); the score rises ~0.11 per key, up to ~330 at 3000 keys."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    case = wl.make_decode("rise", 12, 6, 200, 3000, window=window)
    B, hq, D = case.q.shape
    hkv = case.k_pool.shape[2]
    g = torch.Generator().manual_seed(6)
    s = torch.where(torch.rand(hkv, D, generator=g) < 0.5, -1.0, 1.0)
    kp = case.k_pool.float()
    for b in range(B):
        n = int(case.ctx_lens[b])
        lo = max(0, n - window) if window else 0
        p = torch.arange(lo, n)
        pages = case.block_table[b, p // 16].long()
        kp[pages, p % 16] = s[None] * (0.02 * p.float())[:, None, None] + \
            0.3 * torch.randn(p.numel(), hkv, D, generator=g)
    case.k_pool.copy_(kp.to(torch.bfloat16))
    case.q.copy_((0.5 * s.repeat_interleave(hq // hkv, 0)[None] +
                  0.1 * torch.randn(B, hq, D, generator=g)).to(torch.bfloat16))
    ref_o, ref_l = _oracle(case)
    for mp, wgs in ((1, 0), (8, 5)):
        out, lse = _run(tm, case, dev, min_pages=mp, num_workgroups=wgs)
        assert_out_close(out, ref_o, f"rising w={window} mp={mp}")
        assert_lse_close(lse, ref_l, f"rising w={window} mp={mp}")


@pytest.mark.parametrize("window", [0, 64])
def test_batch_above_one_scan_pass(tm, dev, window):
    """B = 700: the start-up prefix scan over the batch runs in passes of
    256 sequences, each carrying the previous passes' total. Lengths 0-300
    (zero-length rows at every 50th sequence), so most sequences are one or
    two pages and many work-group boundaries fall inside the second and
    third passes."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    B = 700
    ctx = [0 if b % 50 == 0 else 1 + (b * 37) % 300 for b in range(B)]
    case = wl.make_decode("big-b", 13, B, 0, 0, window=window, ctx=ctx)
    ref_o, ref_l = _oracle(case)
    for mp, wgs in ((1, 0), (3, 97)):
        out, lse = _run(tm, case, dev, min_pages=mp, num_workgroups=wgs)
        what = f"B=700 window={window} min_pages={mp} wgs={wgs}"
        assert_out_close(out, ref_o, what)
        assert_lse_close(lse, ref_l, what)
        zero = torch.tensor([c == 0 for c in ctx])
        assert torch.all(out[zero].float() == 0), what


def test_row_width_bound(tm, dev):
    """ctx_lens reaching past a block-table row: the logical pages beyond
    the row's width count as absent (the result is the attention over the
    keys the row covers), never the next row's pages, which are NaN."""
    g = torch.Generator().manual_seed(71)
    HQ, HKV, D, P = 32, 4, 128, 10
    kp = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    vp = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    kp[6:] = float("nan")
    vp[6:] = float("nan")
    table = torch.tensor([[1, 4, 0, 3], [6, 7, 8, 9]], dtype=torch.int32)
    q = torch.randn((2, HQ, D), generator=g).to(torch.bfloat16)
    ctx = torch.tensor([100, 0], dtype=torch.int32)   # row 0 covers 64 keys
    for mp, wgs in ((1, 0), (2, 3)):
        out, lse = tm.decode_paged(q.to(dev), kp.to(dev), vp.to(dev),
                                   table.to(dev), ctx.to(dev), 0.1,
                                   min_pages=mp, num_workgroups=wgs)
        torch.cuda.synchronize()
        # the covered keys 0..63 seen from query position 99 (no window, no
        # bias: the position enters nowhere else)
        ref_o, ref_l = attn_ref.decode_paged(q[:1], kp, vp, table[:1],
                                             torch.tensor([64]), 0.1)
        assert_out_close(out[:1], ref_o, "row width")
        assert_lse_close(lse[:1], ref_l, "row width")


@pytest.mark.parametrize("window", [0, 4096])
def test_one_very_long_context(tm, dev, window):
    """A 262,143-token context beside a 17-token one (NaN-poisoned pool
    outside the backed pages): the long sequence is split over every
    work-group of the persistent grid and merged from ~190 pieces. Checked
    against an fp32 gather of its pages."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    ctx = [262143, 17]
    case = wl.make_decode("long_ctx", 29, 2, 0, 0, window, device=dev,
                          ctx=ctx)
    out, lse = tm.decode_paged(case.q, case.k_pool, case.v_pool,
                               case.block_table, case.ctx_lens, case.scale,
                               window=window)
    torch.cuda.synchronize()
    out, lse = out.cpu(), lse.cpu()
    HQ, HKV = case.q.shape[1], case.k_pool.shape[2]
    rep = HQ // HKV
    table = case.block_table.cpu().long()
    for b, n in enumerate(ctx):
        lo = max(0, n - window) if window else 0
        pages = table[b, lo // 16:(n + 15) // 16].to(case.k_pool.device)
        K = case.k_pool[pages].reshape(-1, HKV, 128)[lo % 16:][:n - lo]
        V = case.v_pool[pages].reshape(-1, HKV, 128)[lo % 16:][:n - lo]
        K, V = K.float().cpu(), V.float().cpu()
        qv = case.q[b].float().cpu().view(HKV, rep, -1)
        s = torch.einsum("grd,ngd->grn", qv, K) * case.scale
        ref_l = torch.logsumexp(s, -1).reshape(HQ)
        ref_o = torch.einsum("grn,ngd->grd", torch.softmax(s, -1),
                             V).reshape(HQ, -1)
        assert_out_close(out[b], ref_o, f"ctx {n} w={window}")
        assert_lse_close(lse[b], ref_l, f"ctx {n} w={window}")
