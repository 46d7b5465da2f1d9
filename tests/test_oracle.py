"""CPU tests that pin the oracle (oracle/attn_ref.py, oracle/kv_ref.py,
oracle/geometry.py) before anything is compared against it.

Pins, each independent of the oracle's own code:
  * golden vectors from plain-Python loops (tests/golden/make_golden.py);
  * torch.nn.functional.scaled_dot_product_attention with an explicit mask;
  * closed forms: q = 0 -> LSE = ln(#visible), out = mean of visible V;
    a single visible key -> its V row and its score; one-hot V rows -> the
    attention weights; SWA == global when ctx <= W;
  * the reference's structural pins (t_b3.py:81-130, t_graphrun.py:17-76);
  * planted mistakes (wrong GQA map, window off by one, missing scale,
    K/V swapped, log base, in-page order) must each fail a pin.
"""
import math

import numpy as np
import pytest
import torch

from golden import load as golden
from oracle import attn_ref, geometry, kv_ref

TOL = 1e-5


def _decode_golden(c, q=None, k_pool=None, v_pool=None, window=None,
                   scale=None):
    table = torch.tensor(c["block_table"], dtype=torch.int64)
    return attn_ref.decode_paged(
        c["q"] if q is None else q,
        c["k_pool"] if k_pool is None else k_pool,
        c["v_pool"] if v_pool is None else v_pool, table,
        torch.tensor(c["ctx"]), c["scale"] if scale is None else scale,
        window=c["window"] if window is None else window,
        table_wrap=c["table_wrap"], rel=c["rel"])


def _close(a, b):
    return bool((a.float() - b.float()).abs().max() <= TOL)


# --------------------------------------------------------------------------
# golden vectors
# --------------------------------------------------------------------------

@pytest.mark.parametrize("c", golden.cases("decode"), ids=lambda c: c["name"])
def test_decode_oracle_matches_golden(c):
    out, lse = _decode_golden(c)
    assert _close(out, c["out"]) and _close(lse, c["lse"])


@pytest.mark.parametrize("c", golden.cases("prefill"),
                         ids=lambda c: c["name"])
def test_prefill_oracle_matches_golden(c):
    out, lse = attn_ref.prefill_varlen(c["q"], c["k"], c["v"],
                                       torch.tensor(c["cu"]), c["scale"],
                                       window=c["window"])
    assert _close(out, c["out"]) and _close(lse, c["lse"])


def test_kv_write_oracle_matches_golden():
    c = golden.cases("kv_write")[0]
    pool = kv_ref.as_u16(c["pool"].to(torch.bfloat16)).copy()
    kv_ref.write_paged(pool, kv_ref.as_u16(c["k"]), c["cu"], c["start"],
                       np.array(c["block_table"]))
    assert np.array_equal(pool, kv_ref.as_u16(c["want"].to(torch.bfloat16)))


# --------------------------------------------------------------------------
# planted mistakes: each must break at least one golden comparison
# --------------------------------------------------------------------------

def _mutants(c):
    HQ, HKV = c["HQ"], c["HKV"]
    rep = HQ // HKV

    def gqa_modulo():
        # head h reads KV head h % HKV instead of h // REP: same as the
        # correct map applied to permuted query heads
        perm = [(h % HKV) * rep + h // HKV for h in range(HQ)]
        inv = [perm.index(h) for h in range(HQ)]
        o, l = _decode_golden(c, q=c["q"][:, perm])
        return o[:, inv], l[:, inv]

    def in_page_reversed():
        return _decode_golden(c, k_pool=c["k_pool"].flip(1),
                              v_pool=c["v_pool"].flip(1))

    muts = {
        "no_scale": lambda: _decode_golden(c, scale=1.0),
        "kv_swapped": lambda: _decode_golden(c, k_pool=c["v_pool"],
                                             v_pool=c["k_pool"]),
        "log2_lse": lambda: tuple(
            x / math.log(2) if i else x
            for i, x in enumerate(_decode_golden(c))),
        "in_page_reversed": in_page_reversed,
    }
    if rep > 1 and HKV > 1:   # with one KV head both maps coincide
        muts["gqa_modulo"] = gqa_modulo
    if c["window"]:
        muts["window_plus_1"] = lambda: _decode_golden(
            c, window=c["window"] + 1)
    return muts


@pytest.mark.parametrize("c", golden.cases("decode"), ids=lambda c: c["name"])
def test_planted_mistakes_fail_golden(c):
    for name, fn in _mutants(c).items():
        out, lse = fn()
        caught = not (_close(out, c["out"]) and _close(lse, c["lse"]))
        assert caught, f"planted mistake {name} passed the golden check"


# --------------------------------------------------------------------------
# library routine: torch SDPA with an explicit boolean mask
# --------------------------------------------------------------------------

@pytest.mark.parametrize("window", [0, 5, 40])
def test_prefill_oracle_matches_sdpa(window):
    g = torch.Generator().manual_seed(4)
    lens, HQ, HKV, D = [3, 70, 17], 8, 2, 32
    cu = torch.tensor([0, 3, 73, 90])
    q = torch.randn((90, HQ, D), generator=g).to(torch.bfloat16)
    k = torch.randn((90, HKV, D), generator=g).to(torch.bfloat16)
    v = torch.randn((90, HKV, D), generator=g).to(torch.bfloat16)
    out, _ = attn_ref.prefill_varlen(q, k, v, cu, 0.3, window=window,
                                     q_block=16)
    F = torch.nn.functional
    for i, T in enumerate(lens):
        t0 = int(cu[i])
        qi = q[t0:t0 + T].float().permute(1, 0, 2)
        ki = k[t0:t0 + T].float().repeat_interleave(HQ // HKV, 1).permute(
            1, 0, 2)
        vi = v[t0:t0 + T].float().repeat_interleave(HQ // HKV, 1).permute(
            1, 0, 2)
        d = torch.arange(T)[:, None] - torch.arange(T)[None, :]
        mask = d >= 0
        if window:
            mask &= d < window
        ref = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=mask,
                                             scale=0.3)
        assert (out[t0:t0 + T].permute(1, 0, 2) - ref).abs().max() < 1e-5


# --------------------------------------------------------------------------
# closed forms and identities
# --------------------------------------------------------------------------

def _wl():
    from importlib import import_module
    return import_module("tm-opt_amd.workloads")


def test_zero_query_uniform_weights():
    case = _wl().make_decode("z", 31, 6, 1, 300, window=50, poison=True)
    case.q.zero_()
    out, lse = attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                                     case.block_table, case.ctx_lens,
                                     case.scale, window=50)
    nv = case.visible().double()
    assert torch.allclose(lse.double(), torch.log(nv)[:, None].expand_as(lse),
                          atol=1e-6)
    for b in range(case.B):
        n = int(case.ctx_lens[b])
        lo = max(0, n - 50)
        rows = kv_ref.gather(kv_ref.as_u16(case.v_pool),
                             case.block_table[b].numpy(), n, lo=lo)
        vr = torch.from_numpy(rows.astype(np.int16)).view(
            torch.bfloat16).float()
        mean = vr.mean(0)                                   # [HKV, D]
        rep = case.q.shape[1] // mean.shape[0]
        assert torch.allclose(out[b], mean.repeat_interleave(rep, 0),
                              atol=1e-5)


def test_single_visible_key():
    case = _wl().make_decode("one", 32, 5, 1, 200, window=1, poison=True)
    out, lse = attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                                     case.block_table, case.ctx_lens,
                                     case.scale, window=1)
    for b in range(case.B):
        p = int(case.ctx_lens[b]) - 1
        pg = int(case.block_table[b, p // 16])
        kv = case.k_pool[pg, p % 16].float()
        vv = case.v_pool[pg, p % 16].float()
        rep = case.q.shape[1] // kv.shape[0]
        s = (case.q[b].float() * kv.repeat_interleave(rep, 0)).sum(-1) * \
            case.scale
        assert torch.allclose(lse[b], s, atol=1e-5)
        assert torch.allclose(out[b], vv.repeat_interleave(rep, 0), atol=1e-6)


def test_one_hot_values_give_weights():
    """V row of key j = e_j: out[h, j] is the softmax weight of key j."""
    g = torch.Generator().manual_seed(8)
    n, HQ, HKV, D = 40, 4, 1, 64
    q = torch.randn((1, HQ, D), generator=g).to(torch.bfloat16)
    k_pool = torch.randn((3, 16, HKV, D), generator=g).to(torch.bfloat16)
    v_pool = torch.zeros((3, 16, HKV, D), dtype=torch.bfloat16)
    table = torch.tensor([[2, 0, 1]])
    for j in range(n):
        v_pool[table[0, j // 16], j % 16, 0, j] = 1.0
    out, _ = attn_ref.decode_paged(q, k_pool, v_pool, table,
                                   torch.tensor([n]), 0.2)
    K = torch.stack([k_pool[table[0, j // 16], j % 16, 0].float()
                     for j in range(n)])
    w = torch.softmax(q[0].float() @ K.T * 0.2, -1)
    assert torch.allclose(out[0, :, :n], w, atol=1e-6)
    assert torch.all(out[0, :, n:] == 0)


def test_swa_equals_global_when_short():
    case = _wl().make_decode("s", 33, 5, 1, 300, window=0, poison=True)
    a = attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                              case.block_table, case.ctx_lens, case.scale)
    b = attn_ref.decode_paged(case.q, case.k_pool, case.v_pool,
                              case.block_table, case.ctx_lens, case.scale,
                              window=300)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_ring_pool_as_block_table():
    """RingKV keeps position p at slot p % W (kv.py:75-76); viewing the ring
    row as W/16 pages and wrapping the logical page reproduces that map."""
    W, per = 64, 4
    for n in range(1, 200):
        for p in range(max(0, n - W), n):
            lp = (p // 16) % per
            assert lp * 16 + p % 16 == p % W


def test_ring_geometry_restated():
    """decode_batch_ctx #1 (model.py:842-848) brute force: every live slot
    s holds the unique p in [n-W, n) with p % W == s."""
    for W in (4, 8, 12):
        for n in range(0, 3 * W + 2):
            p, live = geometry.ring_positions(n, W)
            for s in range(W):
                if live[s]:
                    assert p[s] % W == s and max(0, n - W) <= p[s] < n
            assert int(live.sum()) == min(n, W)


def test_global_geometry_and_bucket():
    """decode_batch_ctx #2 and the 512-bucket high-water (t_graphrun.py
    restated): padded columns are dead, buckets are monotone."""
    pg, off, valid = geometry.global_valid(21, 32)
    assert valid.sum() == 21 and not valid[21:].any()
    assert (pg * 16 + off == np.arange(32)).all()
    hw = 0
    for mp in (10, 600, 300, 2000, 1000):
        L = geometry.bucket_len(mp, hw)
        assert L >= hw and L % 512 == 0 and L >= mp + 1
        hw = L


# --------------------------------------------------------------------------
# the reference's structural KV pins (t_b3.py:81-130), restated
# --------------------------------------------------------------------------

def test_kv_paged_pin():
    rng = np.random.default_rng(1)
    ks = rng.integers(0, 1 << 15, size=(13, 2, 8)).astype(np.uint16)
    order = list(rng.permutation(8))
    pool = np.zeros((8, 4, 2, 8), dtype=np.uint16)
    table = [order[:4]]
    kv_ref.write_paged(pool, ks[:5], [0, 5], [0], table, page=4)
    kv_ref.write_paged(pool, ks[5:], [0, 8], [5], table, page=4)
    assert np.array_equal(kv_ref.gather(pool, order[:4], 13, page=4), ks)


def test_kv_ring_pin():
    rng = np.random.default_rng(2)
    ks = rng.integers(0, 1 << 15, size=(13, 2, 8)).astype(np.uint16)
    for chunks in (((0, 3), (3, 13)), ((0, 13),)):
        pool = np.zeros((8, 4, 2, 8), dtype=np.uint16)
        for s0, s1 in chunks:
            kv_ref.write_paged(pool, ks[s0:s1], [0, s1 - s0], [s0], [[6, 2]],
                               page=4, table_wrap=2)
        got = kv_ref.gather(pool, [6, 2], 13, page=4, table_wrap=2, lo=5)
        assert np.array_equal(got, ks[5:])


def test_write_slots_index_put_semantics():
    rng = np.random.default_rng(3)
    pool = rng.integers(0, 100, size=(4, 16, 2, 8)).astype(np.uint16)
    rows = rng.integers(0, 100, size=(5, 2, 8)).astype(np.uint16)
    ref = torch.from_numpy(pool.astype(np.int64)).view(-1, 2, 8).clone()
    slots = [3, -1, 63, 70, 10]
    for t, s in enumerate(slots):
        if 0 <= s < 64:
            ref[s] = torch.from_numpy(rows[t].astype(np.int64))
    got = kv_ref.write_slots(pool.copy(), rows, slots)
    assert np.array_equal(got.reshape(-1, 2, 8), ref.numpy())


# --------------------------------------------------------------------------
# work counters used by the roofline figures
# --------------------------------------------------------------------------

@pytest.mark.parametrize("window", [0, 7, 64])
def test_visible_pairs_brute_force(window):
    wl = _wl()
    lens, prior = [1, 9, 100, 65], [0, 3, 50, 7]
    want = 0
    for T, p in zip(lens, prior):
        for j in range(T):
            qp = p + j
            for kp in range(qp + 1):
                if not window or qp - kp < window:
                    want += 1
    assert wl.visible_pairs(lens, window, prior) == want


def test_decode_algorithmic_bytes():
    wl = _wl()
    c = wl.make_decode("b", 34, 3, 1, 1, window=20, ctx=[5, 40, 100])
    nv = [5, 20, 20]
    want = sum(nv) * 4 * 128 * 4 + 3 * 32 * 128 * 4 + 3 * 32 * 4 + \
        sum((n + 15) // 16 for n in nv) * 4 + 3 * 4
    assert c.algorithmic_bytes() == want


def test_workload_tables_are_valid():
    wl = _wl()
    c = wl.config1()
    P = c.k_pool.shape[0]
    used = []
    for b in range(c.B):
        n = int(c.ctx_lens[b])
        row = c.block_table[b, :(n + 15) // 16]
        assert ((row >= 0) & (row < P - 1)).all()
        used += row.tolist()
    assert len(used) == len(set(used))               # pages are distinct
    assert torch.isnan(c.k_pool[P - 1].float()).all()   # poison page


# --------------------------------------------------------------------------
# model-semantics restatements used by the adapter tests
# --------------------------------------------------------------------------

def test_prefill_semantics_zero_bias_equals_packed_oracle():
    g = torch.Generator().manual_seed(41)
    B, H, HK, T, D = 2, 8, 2, 37, 32
    q = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    k = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    v = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    rel = torch.zeros((B, H, T, 16), dtype=torch.bfloat16)
    a = attn_ref.prefill_reference_semantics(q, k, v, rel, torch.arange(T),
                                             9)
    cu = torch.tensor([0, T, 2 * T])
    pk = lambda x: x.transpose(1, 2).reshape(B * T, x.shape[1], D)
    b, _ = attn_ref.prefill_varlen(pk(q), pk(k), pk(v), cu, 1.0 / D,
                                   window=9)
    assert (a.reshape(B * T, H, D) - b).abs().max() < 1e-5


def test_prefill_semantics_bias_closed_form():
    """q = 0: weights are exp(bias(dist)); bias = ln(dist + 1) inside the
    band E, 0 outside, so w = dist + 1 for dist < E and 1 beyond."""
    B, H, HK, T, D, E = 1, 2, 1, 20, 16, 6
    g = torch.Generator().manual_seed(42)
    q = torch.zeros((B, H, T, D), dtype=torch.bfloat16)
    k = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    v = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    lnw = torch.log(torch.arange(E, dtype=torch.float32) + 1)
    rel = lnw.expand(B, H, T, E).to(torch.bfloat16)
    out = attn_ref.prefill_reference_semantics(q, k, v, rel, torch.arange(T),
                                               None)
    vb = v.float()[0, 0]
    for t in (0, 3, 5, 6, 19):
        d = t - torch.arange(t + 1)
        w = torch.where(d < E, torch.exp(rel.float()[0, 0, 0, d.clamp(
            max=E - 1)]), torch.ones(()))
        want = (w[:, None] * vb[:t + 1]).sum(0) / w.sum()
        assert torch.allclose(out[0, t, 0], want, atol=1e-5)


def test_varlen_bias_matches_padded_semantics():
    """The packed oracle's fused bias (rel [total, HQ, E]) against the
    padded-batch restatement of the model semantics, which gathers the
    bias independently (torch.gather over [B, H, T, E]): E shorter than the
    runs, with and without a window."""
    g = torch.Generator().manual_seed(43)
    B, H, HK, T, D, E = 2, 4, 2, 45, 16, 11
    q = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    k = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    v = torch.randn((B, HK, T, D), generator=g).to(torch.bfloat16)
    rel = torch.randn((B, H, T, E), generator=g).to(torch.bfloat16)
    cu = torch.tensor([0, T, 2 * T])
    pk = lambda x: x.transpose(1, 2).reshape(B * T, x.shape[1], x.shape[3])
    for window in (None, 7, 30):
        a = attn_ref.prefill_reference_semantics(q, k, v, rel,
                                                 torch.arange(T), window)
        b, _ = attn_ref.prefill_varlen(pk(q), pk(k), pk(v), cu, 1.0 / D,
                                       window=window or 0, rel=pk(rel))
        assert (a.reshape(B * T, H, D) - b).abs().max() < 1e-5, window
        # sampled query rows (the form the model-shape GPU tests use) are
        # the same rows of the whole-batch result
        rows = [44, 0, 10, 11, 29]
        sub = attn_ref.prefill_reference_semantics(
            q, k, v, rel, torch.arange(T), window, rows=rows)
        assert (sub - a[:, rows]).abs().max() < 1e-5, window


# --------------------------------------------------------------------------
# chunked prefill: prior context from the paged pools / a ring
# --------------------------------------------------------------------------

def _prefill_paged_golden(c, source, prior_shift=0, wrap=None, window=None,
                          q=None):
    prior = torch.tensor(c["prior"], dtype=torch.int32) + prior_shift
    table = torch.tensor(c["block_table"], dtype=torch.int64)
    own = source == "mixed"
    return attn_ref.prefill_varlen(
        c["q"] if q is None else q, c["k"] if own else None,
        c["v"] if own else None, torch.tensor(c["cu"]), c["scale"],
        window=c["window"] if window is None else window, prior_lens=prior,
        k_pool=c["k_pool"], v_pool=c["v_pool"], block_table=table,
        table_wrap=c["table_wrap"] if wrap is None else wrap)


def _paged_sources(c):
    # a ring holds the prior context only: the mixed source alone reads it
    return ("mixed",) if c["table_wrap"] else ("paged", "mixed")


@pytest.mark.parametrize("c", golden.cases("prefill_paged"),
                         ids=lambda c: c["name"])
def test_prefill_paged_oracle_matches_golden(c):
    """The oracle's prior-context branches (all keys from the pools; prior
    keys from the pools or a ring and the run's own from packed rows)
    against the plain-Python brute force."""
    for source in _paged_sources(c):
        out, lse = _prefill_paged_golden(c, source)
        assert _close(out, c["out"]) and _close(lse, c["lse"]), source


@pytest.mark.parametrize("c", golden.cases("prefill_paged"),
                         ids=lambda c: c["name"])
def test_prefill_paged_planted_mistakes(c):
    """Plausible mistakes in the prior-context branch each fail the golden
    comparison: query positions off by one, the ring wrap ignored, the
    window one wider."""
    muts = {"prior_plus_1": dict(prior_shift=1)}
    if c["table_wrap"]:
        muts["no_ring_wrap"] = dict(wrap=0)
    if c["window"]:
        muts["window_plus_1"] = dict(window=c["window"] + 1)
    for name, kw in muts.items():
        for source in _paged_sources(c):
            try:
                out, lse = _prefill_paged_golden(c, source, **kw)
            except (IndexError, RuntimeError):
                continue          # an out-of-table read also catches it
            caught = not (_close(out, c["out"]) and _close(lse, c["lse"]))
            assert caught, f"planted mistake {name} ({source}) passed"


@pytest.mark.parametrize("c", golden.cases("prefill_paged"),
                         ids=lambda c: c["name"])
def test_prefill_paged_zero_query_closed_form(c):
    """q = 0: uniform weights over the visible keys, so LSE = ln(number of
    visible keys) = ln(min(prior + j + 1, W)) whatever the keys, the table
    or the ring, and out = the mean of the visible V rows."""
    q0 = torch.zeros_like(c["q"])
    W = c["window"]
    for source in _paged_sources(c):
        out, lse = _prefill_paged_golden(c, source, q=q0)
        want = []
        for p, T in zip(c["prior"], c["lens"]):
            n = torch.arange(p + 1, p + T + 1, dtype=torch.float64)
            want.append(torch.log(torch.clamp(n, max=W) if W else n))
        want = torch.cat(want)[None].expand(lse.shape[0], -1)
        assert (lse.double() - want).abs().max() < 1e-5, source
    # the mean of V: run 0, last query, head 0, through the brute-force rows
    out, _ = _prefill_paged_golden(c, _paged_sources(c)[-1], q=q0)
    i, T, p0 = 0, c["lens"][0], c["prior"][0]
    pos = p0 + T - 1
    lo = max(0, pos - W + 1) if W else 0
    rows = []
    for p in range(lo, pos + 1):
        if p < p0:
            lp = p // 16
            if c["table_wrap"]:
                lp %= c["table_wrap"]
            rows.append(c["v_pool"][c["block_table"][i][lp], p % 16, 0])
        else:
            rows.append(c["v"][c["cu"][i] + p - p0, 0])
    want = torch.stack(rows).float().mean(0)
    assert (out[c["cu"][i] + T - 1, 0] - want).abs().max() < 1e-5

