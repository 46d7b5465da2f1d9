"""fp32 CPU oracle of the paged attention math (TEST INFRASTRUCTURE ONLY —
see oracle/__init__.py; never imported by the product path).

Every function computes in float32 from the bf16 inputs upcast exactly (not
regenerated), the oracle BASELINE.json asks for: softmax(scale * Q K^T + bias +
mask) V with a natural-log LSE. The reference rounds the probabilities to
bf16 before P.V (engine/pyengine/kernels/attn_swa.py:110-112); the oracle
does not, and the tolerance absorbs that rounding.
"""
import math

import torch

PAGE = 16


def _key_rows(block_table_row, positions, table_wrap, page=PAGE):
    """Logical positions -> (physical page, in-page offset), following
    PagedKV._flat_slots (engine/pyengine/kv.py:161-168); a ring table of
    table_wrap pages reuses its pages cyclically (RingKV slot p % W,
    kv.py:75-76 and :99-100, with W = table_wrap * page)."""
    lp = positions // page
    if table_wrap:
        lp = lp % table_wrap
    pages = block_table_row[lp].to(torch.int64)
    return pages, positions % page


def rel_bias_gather(rel_row, dist):
    """rel[b, h, clamp(dist, 0, E-1)] zeroed outside 0 <= dist < E
    (engine/pyengine/model.py:137-158 steps #2-#4; attn_swa.py:97-102).
    rel_row [H, E] -> [H, len(dist)] fp32."""
    E = rel_row.shape[-1]
    idx = dist.clamp(0, E - 1)
    g = rel_row.float()[:, idx]
    band = (dist >= 0) & (dist < E)
    return torch.where(band[None, :], g, torch.zeros((), dtype=g.dtype))


def decode_paged(q, k_pool, v_pool, block_table, ctx_lens, scale, window=0,
                 table_wrap=0, rel=None):
    """One query per sequence at position n-1 against its cached keys.

    Follows _attn_decode_kernel (engine/pyengine/kernels/attn_swa.py:57-117)
    and the eager chain it replaced (engine/pyengine/model.py:978-1014):
    visible keys are positions [lo, n) with lo = max(0, n - W) on windowed
    layers (attn_swa.py:71-72, :83-85: live iff 0 <= pos - p < W) and 0 on
    global ones (:90-91: live iff l < n); GQA head h reads KV head h // REP
    (model.py:995-998); score = q.k * scale + bias, softmax in fp32.

    q [B, HQ, D]; pools [P, 16, HKV, D]; block_table [B, >=pages] int;
    ctx_lens [B] int. Returns (out [B, HQ, D] fp32, lse [B, HQ] fp32)."""
    B, HQ, D = q.shape
    HKV = k_pool.shape[2]
    rep = HQ // HKV
    out = torch.zeros((B, HQ, D), dtype=torch.float32)
    lse = torch.full((B, HQ), -math.inf, dtype=torch.float32)
    bt = block_table.cpu()
    for b in range(B):
        n = int(ctx_lens[b])
        if n <= 0:
            continue
        lo = max(0, n - window) if window else 0
        pos = torch.arange(lo, n, dtype=torch.int64)
        pages, offs = _key_rows(bt[b], pos, table_wrap)
        K = k_pool[pages, offs].float()            # [n_vis, HKV, D]
        V = v_pool[pages, offs].float()
        # head h = kvh * REP + r reads KV head kvh: group the query heads
        qb = q[b].float().view(HKV, rep, D)        # [HKV, REP, D]
        s = torch.matmul(qb, K.permute(1, 2, 0)).reshape(HQ, -1) * scale
        if rel is not None:
            s = s + rel_bias_gather(rel[b].cpu(), (n - 1) - pos)
        lse[b] = torch.logsumexp(s, dim=-1)
        p = torch.softmax(s, dim=-1)               # [HQ, n_vis]
        out[b] = torch.matmul(p.view(HKV, rep, -1),
                              V.permute(1, 0, 2)).reshape(HQ, D)
    return out, lse


def prefill_varlen(q, k, v, cu_seqlens, scale, window=0, prior_lens=None,
                   k_pool=None, v_pool=None, block_table=None, q_block=256,
                   rel=None, table_wrap=0):
    """Causal (optionally windowed) attention over packed runs.

    Follows _attn_prefill_kernel (engine/pyengine/kernels/attn_prefill.py:
    80-141) and the eager chain of attn_prefill (engine/pyengine/model.py:
    530-556): query j of run i sits at position p_i + j (p_i = prior tokens),
    keys at positions 0..p_i+len_i-1, kept iff 0 <= qpos - kpos (< W on
    windowed layers) — the additive_causal_mask predicate (model.py:228-246).
    GQA head h reads KV head h // REP. With a block table and no k/v every
    key comes from the paged pools (PagedKV.gather, kv.py:207-212); with a
    block table and k/v the prior keys come from the pools (a ring of
    table_wrap pages when table_wrap > 0: RingKV slot p % W, kv.py:75-76,
    :105-114) and the run's own keys from the packed rows; without a table
    every key is a packed row (no prior context).
    rel (optional, [total, HQ, E]): query row t of head h adds
    rel[t, h, qpos - kpos] to the scaled score inside 0 <= qpos - kpos < E
    and nothing outside (attn_prefill.py:114-120, rel_bias model.py:137-158).

    Returns (out [total, HQ, D] fp32, lse [HQ, total] fp32)."""
    total, HQ, D = q.shape
    cu = cu_seqlens.to(torch.int64).cpu()
    S = cu.shape[0] - 1
    if block_table is not None and k is None:
        HKV = k_pool.shape[2]
    else:
        HKV = k.shape[1]
    rep = HQ // HKV
    out = torch.zeros((total, HQ, D), dtype=torch.float32)
    lse = torch.full((HQ, total), -math.inf, dtype=torch.float32)
    for i in range(S):
        t0, t1 = int(cu[i]), int(cu[i + 1])
        T = t1 - t0
        if T <= 0:
            continue
        p0 = 0 if prior_lens is None else int(prior_lens[i])
        nk = p0 + T
        if block_table is not None and k is None:
            assert not table_wrap, "a ring holds the prior context only"
            kpos = torch.arange(nk, dtype=torch.int64)
            pages, offs = _key_rows(block_table[i].cpu(), kpos, 0)
            K = k_pool[pages, offs].float()
            V = v_pool[pages, offs].float()
        elif block_table is not None:
            # prior keys the window can reach (a ring keeps the last W only;
            # older positions are never visible to this run's queries)
            lo = max(0, p0 - window + 1) if window else 0
            kpos = torch.arange(lo, p0, dtype=torch.int64)
            pages, offs = _key_rows(block_table[i].cpu(), kpos, table_wrap)
            HKV_ = k.shape[1]
            K = torch.zeros((nk, HKV_, D), dtype=torch.float32)
            V = torch.zeros((nk, HKV_, D), dtype=torch.float32)
            K[lo:p0] = k_pool[pages, offs].float()
            V[lo:p0] = v_pool[pages, offs].float()
            K[p0:] = k[t0:t1].float()
            V[p0:] = v[t0:t1].float()
        else:
            assert p0 == 0
            K = k[t0:t1].float()
            V = v[t0:t1].float()
        Kh = K.repeat_interleave(rep, dim=1).permute(1, 0, 2)   # [HQ, nk, D]
        Vh = V.repeat_interleave(rep, dim=1).permute(1, 0, 2)
        for j0 in range(0, T, q_block):
            j1 = min(T, j0 + q_block)
            qp = p0 + torch.arange(j0, j1, dtype=torch.int64)
            k_lo = max(0, p0 + j0 - window + 1) if window else 0
            k_hi = p0 + j1                       # exclusive
            kp = torch.arange(k_lo, k_hi, dtype=torch.int64)
            qb = q[t0 + j0:t0 + j1].float().permute(1, 0, 2)    # [HQ, m, D]
            s = torch.matmul(qb, Kh[:, k_lo:k_hi].transpose(1, 2)) * scale
            d = qp[:, None] - kp[None, :]
            if rel is not None:
                E = rel.shape[2]
                r = rel[t0 + j0:t0 + j1].float().permute(1, 0, 2)  # [HQ,m,E]
                band = (d >= 0) & (d < E)
                idx = d.clamp(0, E - 1)[None].expand(HQ, -1, -1)
                s = s + torch.where(band[None], torch.gather(r, 2, idx),
                                    torch.zeros(()))
            keep = d >= 0
            if window:
                keep &= d < window
            s = s.masked_fill(~keep[None], -math.inf)
            lse[:, t0 + j0:t0 + j1] = torch.logsumexp(s, dim=-1)
            p = torch.softmax(s, dim=-1)
            out[t0 + j0:t0 + j1] = torch.matmul(
                p, Vh[:, k_lo:k_hi]).permute(1, 0, 2)
    return out, lse


def decode_reference_semantics(q, pool_k, pool_v, slots, pos, rel, window):
    """attn_swa's model semantics (engine/pyengine/kernels/attn_swa.py:
    120-141): ring pool [S, W, HK, D], scale 1/D, rel extent == W.
    Restated through the paged oracle with the ring viewed as pages."""
    B, HQ, D = q.shape
    S, W, HK, _ = pool_k.shape
    per = W // PAGE
    kp = pool_k.reshape(S * per, PAGE, HK, D)
    vp = pool_v.reshape(S * per, PAGE, HK, D)
    table = slots.to(torch.int64)[:, None] * per + torch.arange(per)[None]
    ctx = pos.to(torch.int64) + 1
    return decode_paged(q, kp, vp, table, ctx, 1.0 / D, window=W,
                        table_wrap=per, rel=rel)


def prefill_reference_semantics(q, k, v, rel, positions, window,
                                rows=None):
    """attn_prefill_fused's model semantics on the padded batch
    (engine/pyengine/kernels/attn_prefill.py:114-124, the eager chain
    model.py:530-556 with rel_bias model.py:137-158): score = q.k / D +
    rel[b, h, q, clamp(dist, 0, E-1)] zeroed outside 0 <= dist < E, kept
    iff 0 <= dist (< window on SWA layers), fp32 softmax.
    q [B, H, T, D], k/v [B, HK, T, D], rel [B, H, T, E], positions [T].
    rows: optional query indices; only those query rows are computed (the
    same expressions restricted to them, for shapes whose full [T, T]
    scores would not fit).
    Returns [B, T, H, D] fp32 ([B, len(rows), H, D] with rows)."""
    B, H, T, D = q.shape
    HK = k.shape[1]
    E = rel.shape[3]
    rep = H // HK
    pos = positions.to(torch.int64).cpu()
    qsel = torch.arange(T) if rows is None else torch.as_tensor(rows)
    M = qsel.shape[0]
    dist = pos[qsel, None] - pos[None, :]                    # [M, T]
    idx = dist.clamp(0, E - 1)
    band = (dist >= 0) & (dist < E)
    keep = dist >= 0
    if window is not None:
        keep &= dist < window
    kh = k.float().repeat_interleave(rep, 1)
    vh = v.float().repeat_interleave(rep, 1)
    qf = q[:, :, qsel].float()
    s = torch.matmul(qf, kh.transpose(2, 3)) / D             # [B,H,M,T]
    r = rel[:, :, qsel].float()
    bias = torch.gather(r, 3, idx[None, None].expand(B, H, M, T))
    s = s + torch.where(band[None, None], bias, torch.zeros(()))
    s = s.masked_fill(~keep[None, None], -math.inf)
    p = torch.softmax(s, -1)
    return torch.matmul(p, vh).transpose(1, 2)
