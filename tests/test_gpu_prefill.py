"""Parity of the HIP varlen prefill kernel against the fp32 oracle.

Tolerances: outputs max-abs 2e-2 / rtol 1e-2, LSE 1e-3.
Covers ragged lengths around the 32-query / 64-key tile edges, causal and
windowed masks, GQA 1, 2, 4 and 8 (and 3, 5, 6, 12, 16, 24, run as groups
of 8, 4, 2 or 1 query heads per stored KV head), strided inputs, chunked prefill reading prior
context from a shuffled paged cache, the fused relative bias (band shorter
than the runs, so most key tiles carry none; packed and paged sources), the
q = 0 closed form (LSE = ln(#visible keys)), determinism, config 4 at full
size checked on sampled query rows, and repeated launches back to back and
on two streams at once.
"""
import math

import pytest
import torch

from helpers import assert_lse_close, assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu

LENS = [1, 5, 31, 32, 33, 63, 64, 65, 129, 200]


def _wl():
    from importlib import import_module
    return import_module("tm-opt_amd.workloads")


def _gpu(tm, case, dev, **kw):
    out, lse = tm.prefill_varlen(case.q.to(dev), case.k.to(dev),
                                 case.v.to(dev), case.cu_seqlens.to(dev),
                                 case.scale, window=case.window, **kw)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


@pytest.mark.parametrize("window", [0, 1, 17, 64, 100])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (64, 16), (8, 8), (16, 8),
                                    (12, 4), (64, 4), (5, 1)])
def test_ragged_lengths(tm, dev, window, hq, hkv):
    case = _wl().make_prefill("ragged", 21, lens=LENS, window=window, hq=hq,
                              hkv=hkv)
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale,
                                           window=window)
    out, lse = _gpu(tm, case, dev)
    assert_out_close(out, ref_o, f"ragged w={window} {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"ragged w={window} {hq}/{hkv}")


@pytest.mark.parametrize("hq,hkv", [(8, 1), (16, 2), (24, 3), (32, 4),
                                    (64, 16), (4, 4), (6, 3), (16, 16),
                                    (24, 12), (12, 4), (40, 8), (96, 4)])
def test_every_row_written(tm, dev, hq, hkv):
    """The work-group -> (KV head, run, query block) schedule covers every
    row: 70 runs (more than one wave's worth of runs) of ragged lengths,
    outputs and LSE pre-filled with NaN, every head count branch of the
    XCD mapping (8 % HKV == 0, HKV % 8 == 0, neither)."""
    g = torch.Generator().manual_seed(31)
    lens = torch.randint(1, 90, (70,), generator=g).tolist()
    lens[5] = 300                     # one long run: many empty levels
    case = _wl().make_prefill("sched", 24, lens=lens, window=0, hq=hq,
                              hkv=hkv)
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale)
    T = case.q.shape[0]
    out = torch.full((T, hq, 128), float("nan"), dtype=torch.bfloat16,
                     device=dev)
    lse = torch.full((hq, T), float("nan"), dtype=torch.float32, device=dev)
    tm.prefill_varlen(case.q.to(dev), case.k.to(dev), case.v.to(dev),
                      case.cu_seqlens.to(dev), case.scale, out=out, lse=lse)
    torch.cuda.synchronize()
    assert_out_close(out.cpu(), ref_o, f"schedule {hq}/{hkv}")
    assert_lse_close(lse.cpu(), ref_l, f"schedule {hq}/{hkv}")


def test_strided_inputs(tm, dev):
    """K/V as head slices of a wider tensor and Q with padded rows; the
    output written into a strided view."""
    g = torch.Generator().manual_seed(3)
    lens = [70, 33, 128]
    T = sum(lens)
    cu = torch.tensor([0, 70, 103, 231], dtype=torch.int32)
    qw = torch.randn((T, 40, 128), generator=g).to(torch.bfloat16)
    kvw = torch.randn((T, 12, 128), generator=g).to(torch.bfloat16)
    q, k, v = qw[:, 4:36], kvw[:, 0:4], kvw[:, 6:10]
    ref_o, ref_l = attn_ref.prefill_varlen(q, k, v, cu, 0.1, window=50)
    qd, kvd = qw.to(dev), kvw.to(dev)
    outw = torch.zeros((T, 48, 128), dtype=torch.bfloat16, device=dev)
    out, lse = tm.prefill_varlen(qd[:, 4:36], kvd[:, 0:4], kvd[:, 6:10],
                                 cu.to(dev), 0.1, window=50,
                                 out=outw[:, 8:40])
    torch.cuda.synchronize()
    assert_out_close(outw[:, 8:40].cpu(), ref_o, "strided")
    assert_lse_close(lse.cpu(), ref_l, "strided")
    assert torch.all(outw[:, :8] == 0) and torch.all(outw[:, 40:] == 0)


def test_output_rows_8_byte_aligned(tm, dev):
    """Output head rows 132 elements apart (8-byte but not 16-byte
    aligned): the row-wise store falls back to 8-byte stores, and the 4
    padding elements after every row stay untouched."""
    case = _wl().make_prefill("o8", 24, lens=[45, 130, 1])
    T, HQ, D = case.q.shape
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale)
    outw = torch.full((T, HQ, D + 4), 7.0, dtype=torch.bfloat16, device=dev)
    out, lse = tm.prefill_varlen(case.q.to(dev), case.k.to(dev),
                                 case.v.to(dev), case.cu_seqlens.to(dev),
                                 case.scale, out=outw[:, :, :D])
    torch.cuda.synchronize()
    assert outw[:, :, :D].stride(1) % 8 == 4
    assert_out_close(outw[:, :, :D].cpu(), ref_o, "8-byte rows")
    assert_lse_close(lse.cpu(), ref_l, "8-byte rows")
    assert torch.all(outw[:, :, D:] == 7.0)


@pytest.mark.parametrize("window", [0, 48])
@pytest.mark.parametrize("HQ,HKV", [(32, 4), (8, 8), (8, 4), (24, 2),
                                    (6, 2)])
def test_paged_prior_context(tm, dev, window, HQ, HKV):
    """Chunked prefill: each run's keys = prior context + its own tokens,
    all in a shuffled page pool (written by the KV-write kernel)."""
    g = torch.Generator().manual_seed(17)
    wl = _wl()
    prior = [0, 16, 100, 37, 300]
    lens = [17, 64, 129, 1, 90]
    S, D = len(lens), 128
    table, P = wl.paged_layout(lens, g, pool_factor=2, prior=prior)
    tot = [p + t for p, t in zip(prior, lens)]
    kp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    vp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    k_all = [torch.randn((n, HKV, D), generator=g).to(torch.bfloat16)
             for n in tot]
    v_all = [torch.randn((n, HKV, D), generator=g).to(torch.bfloat16)
             for n in tot]
    for i in range(S):
        pos = torch.arange(tot[i])
        pages = table[i][pos // 16].long()
        kp[pages, pos % 16] = k_all[i]
        vp[pages, pos % 16] = v_all[i]
    cu = torch.zeros(S + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q = torch.randn((int(cu[-1]), HQ, D), generator=g).to(torch.bfloat16)
    pr = torch.tensor(prior, dtype=torch.int32)
    ref_o, ref_l = attn_ref.prefill_varlen(q, None, None, cu, 0.08,
                                           window=window, prior_lens=pr,
                                           k_pool=kp, v_pool=vp,
                                           block_table=table)
    out, lse = tm.prefill_varlen(q.to(dev), None, None, cu.to(dev), 0.08,
                                 window=window, prior_lens=pr.to(dev),
                                 k_pool=kp.to(dev), v_pool=vp.to(dev),
                                 block_table=table.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref_o, f"paged w={window} {HQ}/{HKV}")
    assert_lse_close(lse, ref_l, f"paged w={window} {HQ}/{HKV}")


def test_zero_query_closed_form(tm, dev):
    """q = 0: LSE = ln(number of visible keys) exactly."""
    case = _wl().make_prefill("q0", 22, lens=[40, 130, 7], window=50)
    case.q.zero_()
    _, lse = _gpu(tm, case, dev)
    want = []
    for T in case.lens:
        j = torch.arange(T, dtype=torch.float64)
        want.append(torch.log(torch.minimum(j + 1, torch.tensor(50.0))))
    want = torch.cat(want)[None].expand(lse.shape[0], -1)
    assert (lse.double() - want).abs().max() <= 1e-4


def test_determinism(tm, dev):
    case = _wl().make_prefill("det", 23, lens=[300, 77, 1000], window=0)
    a = _gpu(tm, case, dev)
    b = _gpu(tm, case, dev)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("make,window", [("config4", 0), ("config4", 4096),
                                         ("config4_long", 4096)])
def test_config4_sampled_rows(tm, dev, make, window):
    """BASELINE config 4 at full size, and its head config on 4 runs of 8192
    tokens with window 4096 (half of each run's queries see a full window);
    the oracle checks 48 sampled query rows per sequence (first, last,
    around the 4096 window edge, random)."""
    wl = _wl()
    case = getattr(wl, make)(window=window)
    out, lse = _gpu(tm, case, dev)
    assert torch.isfinite(out.float()).all()
    g = torch.Generator().manual_seed(99)
    cu = case.cu_seqlens.tolist()
    for i, T in enumerate(case.lens):
        t0 = cu[i]
        pick = {0, T - 1, min(T - 1, 4095), min(T - 1, 4096)}
        pick |= set(torch.randint(0, T, (44,), generator=g).tolist())
        rows = sorted(pick)
        for j in rows:
            lo = max(0, j - window + 1) if window else 0
            qv = case.q[t0 + j].float()                     # [HQ, D]
            K = case.k[t0 + lo:t0 + j + 1].float()          # [n, HKV, D]
            V = case.v[t0 + lo:t0 + j + 1].float()
            rep = qv.shape[0] // K.shape[1]
            s = torch.einsum("hd,nhd->hn", qv,
                             K.repeat_interleave(rep, 1)) * case.scale
            ref_l = torch.logsumexp(s, -1)
            ref_o = torch.einsum("hn,nhd->hd", torch.softmax(s, -1),
                                 V.repeat_interleave(rep, 1))
            assert_out_close(out[t0 + j], ref_o, f"C4 w={window} seq{i} q{j}")
            assert_lse_close(lse[:, t0 + j], ref_l,
                             f"C4 w={window} seq{i} q{j}")


def test_one_long_run_sampled_rows(tm, dev):
    """One run of 131,069 tokens (a long-context prompt; not a multiple of
    the 32-query block or the 64-key tile), global: 4,096 key tiles for the
    last query blocks, 16,384 work-groups. The oracle checks sampled rows
    (first, last, tile and block edges, random) per KV-head group in
    fp32."""
    T = 131069
    case = _wl().make_prefill("long1", 28, lens=[T], window=0, device=dev)
    out, lse = tm.prefill_varlen(case.q, case.k, case.v, case.cu_seqlens,
                                 case.scale, max_seqlen=T)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    K = case.k.float().cpu()                    # [T, HKV, D]
    V = case.v.float().cpu()
    HQ, HKV = case.q.shape[1], case.k.shape[1]
    rep = HQ // HKV
    g = torch.Generator().manual_seed(7)
    rows = {0, 1, 31, 32, 63, 64, 4095, 65535, T - 33, T - 2, T - 1}
    rows |= set(torch.randint(0, T, (5,), generator=g).tolist())
    for j in sorted(rows):
        qv = case.q[j].float().cpu().view(HKV, rep, -1)       # [HKV, rep, D]
        s = torch.einsum("grd,ngd->grn", qv, K[:j + 1]) * case.scale
        ref_l = torch.logsumexp(s, -1).reshape(HQ)
        ref_o = torch.einsum("grn,ngd->grd", torch.softmax(s, -1),
                             V[:j + 1]).reshape(HQ, -1)
        assert_out_close(out[j].cpu(), ref_o, f"long run q{j}")
        assert_lse_close(lse[:, j].cpu(), ref_l, f"long run q{j}")


@pytest.mark.parametrize("E,window", [(95, 0), (1, 0), (80, 256), (300, 64)])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (64, 16), (8, 8), (8, 4),
                                    (12, 4), (64, 4)])
def test_bias_band_shorter_than_runs(tm, dev, E, window, hq, hkv):
    """Fused bias rel[t, h, dist] inside 0 <= dist < E: with E well below
    the run lengths most key tiles lie wholly outside the band and skip the
    bias, so one item mixes tiles with and without it; odd E and query
    positions of both parities exercise the realigned bias loads."""
    g = torch.Generator().manual_seed(31)
    case = _wl().make_prefill("bias", 23, lens=[700, 333, 65, 1],
                              window=window, hq=hq, hkv=hkv)
    total = case.q.shape[0]
    rel = (torch.randn((total, hq, E), generator=g) * 2.0).to(torch.bfloat16)
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale,
                                           window=window, rel=rel)
    out, lse = _gpu(tm, case, dev, rel=rel.to(dev))
    assert_out_close(out, ref_o, f"bias E={E} w={window} {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"bias E={E} w={window} {hq}/{hkv}")


def test_bias_paged_prior_context(tm, dev):
    """Fused bias on the paged source with prior context: dist counts from
    the query's position (prior + j), so the band reaches into the prior
    keys."""
    g = torch.Generator().manual_seed(19)
    wl = _wl()
    prior = [0, 40, 300, 5]
    lens = [150, 64, 97, 1]
    S, HQ, HKV, D, E = len(lens), 32, 4, 128, 70
    table, P = wl.paged_layout(lens, g, pool_factor=2, prior=prior)
    tot = [p + t for p, t in zip(prior, lens)]
    kp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    vp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    for i in range(S):
        pos = torch.arange(tot[i])
        pages = table[i][pos // 16].long()
        kp[pages, pos % 16] = torch.randn((tot[i], HKV, D),
                                          generator=g).to(torch.bfloat16)
        vp[pages, pos % 16] = torch.randn((tot[i], HKV, D),
                                          generator=g).to(torch.bfloat16)
    cu = torch.zeros(S + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q = torch.randn((int(cu[-1]), HQ, D), generator=g).to(torch.bfloat16)
    rel = torch.randn((int(cu[-1]), HQ, E), generator=g).to(torch.bfloat16)
    pr = torch.tensor(prior, dtype=torch.int32)
    ref_o, ref_l = attn_ref.prefill_varlen(q, None, None, cu, 0.08,
                                           prior_lens=pr, k_pool=kp,
                                           v_pool=vp, block_table=table,
                                           rel=rel)
    out, lse = tm.prefill_varlen(q.to(dev), None, None, cu.to(dev), 0.08,
                                 prior_lens=pr.to(dev), k_pool=kp.to(dev),
                                 v_pool=vp.to(dev), block_table=table.to(dev),
                                 rel=rel.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref_o, "paged bias")
    assert_lse_close(lse, ref_l, "paged bias")


@pytest.mark.parametrize("window", [0, 300])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (64, 16)])
def test_rising_scores_rescale(tm, dev, window, hq, hkv):
    """Scores that climb along the keys, so the running max moves past the
    lazy threshold on every key tile and the accumulated O^T and row sum are
    rescaled over and over (with factors that underflow to 0 for the oldest
    terms): key t of a run is s * 0.02 t + noise, every query 0.5 s + noise
    (s a +-1 pattern per KV head), i.e. the score rises ~0.11 per key, ~7
    per 64-key tile, up to ~110 at the end of a 1000-token run."""
    case = _wl().make_prefill("rise", 24, lens=[1000, 130, 65, 700],
                              window=window, hq=hq, hkv=hkv)
    g = torch.Generator().manual_seed(5)
    s = torch.where(torch.rand(hkv, 128, generator=g) < 0.5, -1.0, 1.0)
    cu = case.cu_seqlens.tolist()
    pos = torch.cat([torch.arange(cu[i + 1] - cu[i])
                     for i in range(len(cu) - 1)]).float()
    k = s[None] * (0.02 * pos)[:, None, None] + \
        0.3 * torch.randn(pos.numel(), hkv, 128, generator=g)
    q = 0.5 * s.repeat_interleave(hq // hkv, 0)[None] + \
        0.1 * torch.randn(pos.numel(), hq, 128, generator=g)
    case.k.copy_(k.to(torch.bfloat16))
    case.q.copy_(q.to(torch.bfloat16))
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale,
                                           window=window)
    out, lse = _gpu(tm, case, dev)
    assert_out_close(out, ref_o, f"rising w={window} {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"rising w={window} {hq}/{hkv}")


def test_score_spike_underflows_old_terms(tm, dev):
    """One key per run scores ~150 above the rest (a jump of ~215 in the
    log2 domain): the running max leaps once, the rescale factor of
    everything before underflows to 0, and later keys add terms ~e^-150
    relative to it. Queries before the spike see ordinary scores."""
    case = _wl().make_prefill("spike", 25, lens=[900, 300], window=0)
    g = torch.Generator().manual_seed(7)
    hq, hkv = case.q.shape[1], case.k.shape[1]
    s = torch.where(torch.rand(hkv, 128, generator=g) < 0.5, -1.0, 1.0)
    cu = case.cu_seqlens.tolist()
    q = s.repeat_interleave(hq // hkv, 0)[None].expand(
        case.q.shape[0], -1, -1)
    k = case.k.float()
    for i, at in ((0, 517), (1, 70)):
        k[cu[i] + at] = s * 13.25      # q.k * scale = 128 * 13.25 / 11.3
    case.q.copy_(q.to(torch.bfloat16))
    case.k.copy_(k.to(torch.bfloat16))
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale)
    out, lse = _gpu(tm, case, dev)
    assert_out_close(out, ref_o, "spike")
    assert_lse_close(lse, ref_l, "spike")


def _chunked_pool(g, lens, prior, HKV, D, poison_before=None, nan_page=False,
                  extra_pages=0):
    """Shuffled page pool holding every key (prior context + each run's own
    tokens) of the runs; positions before poison_before[i] hold NaN rows
    and, with nan_page, table entries of pages wholly before it point at a
    NaN page (as a windowed table may). Returns (k_pool, v_pool, table,
    k_all, v_all) with k_all[i] the run's keys in position order."""
    wl = _wl()
    table, P = wl.paged_layout(lens, g, pool_factor=2, prior=prior)
    P += 1 + extra_pages
    tot = [p + t for p, t in zip(prior, lens)]
    kp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    vp = torch.full((P, 16, HKV, D), float("nan"), dtype=torch.bfloat16)
    k_all, v_all = [], []
    for i in range(len(lens)):
        ka = torch.randn((tot[i], HKV, D), generator=g).to(torch.bfloat16)
        va = torch.randn((tot[i], HKV, D), generator=g).to(torch.bfloat16)
        if poison_before is not None:
            ka[:poison_before[i]] = float("nan")
            va[:poison_before[i]] = float("nan")
        pos = torch.arange(tot[i])
        pages = table[i][pos // 16].long()
        kp[pages, pos % 16] = ka
        vp[pages, pos % 16] = va
        if nan_page and poison_before is not None:
            table[i, :poison_before[i] // 16] = P - 1 - extra_pages
        k_all.append(ka)
        v_all.append(va)
    return kp, vp, table, k_all, v_all


def _packed_own(k_all, lens, prior):
    return torch.cat([ka[p:p + t] for ka, p, t in zip(k_all, prior, lens)])


@pytest.mark.parametrize("source", ["paged", "mixed"])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (64, 16), (12, 4)])
def test_window_never_reads_before_it(tm, dev, source, hq, hkv):
    """Windowed chunked prefill over a pool whose keys before each run's
    first visible position (prior - W + 1) are NaN, pages wholly before it
    mapped to a NaN page: the tile grid starts up to 63 keys (3 pages)
    before the window, and those rows must never be read (a masked
    probability of 0 times a NaN value is NaN)."""
    g = torch.Generator().manual_seed(61)
    W, D = 48, 128
    prior = [300, 70, 49, 1000, 0]
    lens = [90, 200, 1, 33, 64]
    first = [max(0, p - W + 1) for p in prior]
    kp, vp, table, k_all, v_all = _chunked_pool(g, lens, prior, hkv, D,
                                                poison_before=first,
                                                nan_page=True)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q = torch.randn((int(cu[-1]), hq, D), generator=g).to(torch.bfloat16)
    pr = torch.tensor(prior, dtype=torch.int32)
    k_own = _packed_own(k_all, lens, prior)
    v_own = _packed_own(v_all, lens, prior)
    ref_o, ref_l = attn_ref.prefill_varlen(q, k_own, v_own, cu, 0.08,
                                           window=W, prior_lens=pr,
                                           k_pool=kp, v_pool=vp,
                                           block_table=table)
    own = source == "mixed"
    out, lse = tm.prefill_varlen(q.to(dev), k_own.to(dev) if own else None,
                                 v_own.to(dev) if own else None, cu.to(dev),
                                 0.08, window=W, prior_lens=pr.to(dev),
                                 k_pool=kp.to(dev), v_pool=vp.to(dev),
                                 block_table=table.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref_o, f"pre-window NaN {source} {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"pre-window NaN {source} {hq}/{hkv}")


@pytest.mark.parametrize("window", [0, 100])
def test_mixed_source_equals_paged_bitwise(tm, dev, window):
    """The mixed source (prior keys from the pool, the run's own from packed
    rows) feeds the same bytes to the same tiles as the all-paged source
    when the pool also holds the run's keys: the outputs are identical.
    Priors of every residue mod 4 put the source boundary inside a 4-row
    load block (split by exec mask)."""
    g = torch.Generator().manual_seed(62)
    HQ, HKV, D = 32, 4, 128
    prior = [0, 1, 2, 3, 17, 250, 511, 64]
    lens = [70, 33, 5, 129, 64, 300, 1, 66]
    kp, vp, table, k_all, v_all = _chunked_pool(g, lens, prior, HKV, D)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q = torch.randn((int(cu[-1]), HQ, D), generator=g).to(torch.bfloat16)
    args = dict(window=window, prior_lens=torch.tensor(
        prior, dtype=torch.int32, device=dev), k_pool=kp.to(dev),
        v_pool=vp.to(dev), block_table=table.to(dev))
    a = tm.prefill_varlen(q.to(dev), None, None, cu.to(dev), 0.08, **args)
    b = tm.prefill_varlen(q.to(dev),
                          _packed_own(k_all, lens, prior).to(dev),
                          _packed_own(v_all, lens, prior).to(dev),
                          cu.to(dev), 0.08, **args)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    ref_o, ref_l = attn_ref.prefill_varlen(q, None, None, cu, 0.08,
                                           window=window,
                                           prior_lens=args["prior_lens"].cpu(),
                                           k_pool=kp, v_pool=vp,
                                           block_table=table)
    assert_out_close(a[0], ref_o, f"mixed==paged w={window}")
    assert_lse_close(a[1], ref_l, f"mixed==paged w={window}")


@pytest.mark.parametrize("hq,hkv", [(64, 16), (32, 4)])
def test_ring_prior_context_chunks_longer_than_window(tm, dev, hq, hkv):
    """SWA chunked prefill over the reference's ring storage (SwaPool rows
    [S + 1, W, HK, D], RingKV slot p % W): the ring holds each sequence's
    last W positions before the chunk; the chunk's own keys come from
    packed k/v (chunks up to 3x the ring), then the chunk is appended to
    the ring and the ring state is checked bit-exact against RingKV's rule
    (only the last W positions survive)."""
    from oracle import kv_ref
    import numpy as np
    g = torch.Generator().manual_seed(63)
    W, D = 512, 128
    per = W // 16
    prior = [0, 100, 511, 512, 513, 4000, 700]
    lens = [300, 1500, 1, 700, 64, 520, 1]
    S = len(lens)
    slots = [4, 0, 6, 2, 1, 5, 3]
    # ring state before the chunk: stale random rows everywhere, then each
    # sequence's last min(prior, W) positions written at p % W
    pool_k = torch.randn((S + 1, W, hkv, D), generator=g).to(torch.bfloat16)
    pool_v = torch.randn((S + 1, W, hkv, D), generator=g).to(torch.bfloat16)
    table = (torch.tensor(slots)[:, None] * per +
             torch.arange(per)[None]).to(torch.int32)
    cu = torch.zeros(S + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    T = int(cu[-1])
    q = torch.randn((T, hq, D), generator=g).to(torch.bfloat16)
    k = torch.randn((T, hkv, D), generator=g).to(torch.bfloat16)
    v = torch.randn((T, hkv, D), generator=g).to(torch.bfloat16)
    kp = pool_k.view((S + 1) * per, 16, hkv, D)
    vp = pool_v.view((S + 1) * per, 16, hkv, D)
    pr = torch.tensor(prior, dtype=torch.int32)
    ref_o, ref_l = attn_ref.prefill_varlen(q, k, v, cu, 1.0 / D, window=W,
                                           prior_lens=pr, k_pool=kp,
                                           v_pool=vp, block_table=table,
                                           table_wrap=per)
    kd, vd = kp.to(dev), vp.to(dev)
    out, lse = tm.prefill_varlen(q.to(dev), k.to(dev), v.to(dev), cu.to(dev),
                                 1.0 / D, window=W, prior_lens=pr.to(dev),
                                 k_pool=kd, v_pool=vd,
                                 block_table=table.to(dev), table_wrap=per)
    # then the append, after the attention (it overwrites the ring)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev), pr.to(dev), kd, vd,
                      cu_seqlens=cu.to(dev), table_wrap=per)
    torch.cuda.synchronize()
    assert_out_close(out, ref_o, f"ring chunks {hq}/{hkv}")
    assert_lse_close(lse, ref_l, f"ring chunks {hq}/{hkv}")
    want = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                              cu.numpy(), prior, table.numpy(), 16, per)
    assert np.array_equal(kv_ref.as_u16(kd), want)


def test_paged_row_width_bound(tm, dev):
    """A block-table row narrower than the run's keys: the logical pages
    past its width read as zero rows (score 0, value 0) instead of the next
    row's pages, which hold NaN here."""
    g = torch.Generator().manual_seed(64)
    HQ, HKV, D = 32, 4, 128
    P = 12
    kp = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    vp = torch.randn((P, 16, HKV, D), generator=g).to(torch.bfloat16)
    kp[7:] = float("nan")
    vp[7:] = float("nan")
    # run 0 needs 3 pages (40 keys) but its row holds 2; row 1 = NaN pages
    table = torch.tensor([[2, 5], [7, 8]], dtype=torch.int32)
    cu = torch.tensor([0, 40], dtype=torch.int32)
    q = torch.randn((40, HQ, D), generator=g).to(torch.bfloat16)
    out, lse = tm.prefill_varlen(q.to(dev), None, None, cu.to(dev), 0.1,
                                 prior_lens=None, k_pool=kp.to(dev),
                                 v_pool=vp.to(dev), block_table=table.to(dev))
    torch.cuda.synchronize()
    # expected: the third page is a zero page
    kz = torch.cat([kp[:7], torch.zeros((1, 16, HKV, D),
                                        dtype=torch.bfloat16)])
    vz = torch.cat([vp[:7], torch.zeros((1, 16, HKV, D),
                                        dtype=torch.bfloat16)])
    ref_o, ref_l = attn_ref.prefill_varlen(
        q, None, None, cu, 0.1, prior_lens=torch.zeros(1, dtype=torch.int32),
        k_pool=kz, v_pool=vz, block_table=torch.tensor([[2, 5, 7]]))
    assert_out_close(out, ref_o, "row width")
    assert_lse_close(lse, ref_l, "row width")


def test_reject_flag_writes_nan(tm, dev):
    """A nonzero device reject flag turns every output row and LSE entry of
    the launch into NaN; a zero flag changes nothing."""
    case = _wl().make_prefill("rej", 26, lens=[70, 1, 300], window=0)
    base = _gpu(tm, case, dev)
    zero = torch.zeros(1, dtype=torch.int32, device=dev)
    one = torch.ones(1, dtype=torch.int32, device=dev)
    a = _gpu(tm, case, dev, reject=zero)
    b = _gpu(tm, case, dev, reject=one)
    assert torch.equal(a[0], base[0]) and torch.equal(a[1], base[1])
    assert torch.isnan(b[0].float()).all() and torch.isnan(b[1]).all()


def _dev_case(case, dev):
    return (case.q.to(dev), case.k.to(dev), case.v.to(dev),
            case.cu_seqlens.to(dev))


def test_repeated_launches_write_every_row(tm, dev):
    """300 launches in a row, outputs pre-filled with NaN each time: every
    launch writes every row and LSE entry, bitwise equal to the first, which
    is within tolerance of the oracle (no state carries from one launch to
    the next)."""
    case = _wl().make_prefill("pers", 25, lens=[1, 100, 37, 500, 64],
                              window=0)
    q, k, v, cu = _dev_case(case, dev)
    T, HQ = case.q.shape[0], case.q.shape[1]
    out0, lse0 = tm.prefill_varlen(q, k, v, cu, case.scale)
    outs = [torch.empty_like(out0) for _ in range(3)]
    lses = [torch.empty_like(lse0) for _ in range(3)]
    for i in range(300):
        o, l = outs[i % 3], lses[i % 3]
        o.fill_(float("nan"))
        l.fill_(float("nan"))
        tm.prefill_varlen(q, k, v, cu, case.scale, out=o, lse=l)
    torch.cuda.synchronize()
    for o, l in zip(outs, lses):
        assert torch.equal(o, out0) and torch.equal(l, lse0)
    ref_o, ref_l = attn_ref.prefill_varlen(case.q, case.k, case.v,
                                           case.cu_seqlens, case.scale)
    assert_out_close(out0.cpu(), ref_o, "persistent")
    assert_lse_close(lse0.cpu(), ref_l, "persistent")
    assert out0.shape == (T, HQ, 128)


def test_two_streams_at_once(tm, dev):
    """Launches in flight on two streams at once (sharing the GPU's compute
    units) give each stream's one-stream results, bitwise."""
    ca = _wl().make_prefill("pa", 26, lens=[700, 45, 1300], window=0)
    cb = _wl().make_prefill("pb", 27, lens=[90, 2000], window=256, hq=64,
                            hkv=8)
    da, db = _dev_case(ca, dev), _dev_case(cb, dev)
    ref_a = tm.prefill_varlen(*da, ca.scale)
    ref_b = tm.prefill_varlen(*db, cb.scale, window=256)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    res_a, res_b = [], []
    for _ in range(10):
        with torch.cuda.stream(sa):
            res_a.append(tm.prefill_varlen(*da, ca.scale))
        with torch.cuda.stream(sb):
            res_b.append(tm.prefill_varlen(*db, cb.scale, window=256))
    torch.cuda.synchronize()
    for o, l in res_a:
        assert torch.equal(o, ref_a[0]) and torch.equal(l, ref_a[1])
    for o, l in res_b:
        assert torch.equal(o, ref_b[0]) and torch.equal(l, ref_b[1])
