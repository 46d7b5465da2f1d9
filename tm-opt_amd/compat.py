"""The reference engine's attention call signatures over the native kernels.

attn_swa / attn_global / attn_prefill_fused take exactly the arguments of
engine/pyengine/kernels/attn_swa.py:120, attn_global.py:15 and
attn_prefill.py:144, keep their contract asserts, their model semantics
(scale 1/head_dim because q/k are RMS-normed, the fused relative bias
gathered at the clamped backward distance and zeroed out of band) and their
output layouts, and run the gfx950 kernels of this package:

  * the SWA ring pool [S, W, HK, D] is viewed as W/16 pages per slot and
    walked as a ring block table (table_wrap = W/16): position p lives in
    ring slot p % W, exactly RingKV's rule (kv.py:75-76, :99-100);
  * the global path's per-token flat rows `flat` [B, Lg] (model.py:938-945)
    are turned back into a block table: rows of one page are consecutive,
    so page i of row b is flat[b, 16 i] // 16;
  * the padded [B, H, T, D] prefill batch becomes B runs of T tokens
    (cu_seqlens = 0, T, 2T, ...): queries as packed rows, K/V one run per
    batch row at the batch stride, token-major or channel-major (the sconv
    output) read in place, other layouts copied;
  * the prefill's position contract is checked on the device
    (tmopt_prefill_check_positions feeds the kernel's reject flag).

No host synchronisation in attn_swa, attn_global, attn_prefill_fused
without caches and the pooled chunk adapters given max_seqlen (or one
sequence, cu_seqlens None): every helper tensor is built with device ops,
so they can run inside hipGraph capture. The
cache-populating paths take the rows' lengths from the host cache
objects, as the reference's appends do (their small metadata tensors go
through pinned memory, without a stream synchronisation).
"""
import os

import torch

from . import attn

PAGE = attn.PAGE_SIZE


def _ring_grid(B, HKV, dev):
    """Work split of a ring decode: k whole rings per work-group (k the
    fewest that keep to one work-group per compute unit), so no row is
    split between work-groups and the merge launch is skipped. Every row
    holds at most W/16 pages, so full rings balance exactly. Measured at
    B = 64, W = 512, 64Q/16KV: 52 us against 62 us with the default grid
    (which splits rings and merges the pieces). Returns (work-groups, k)."""
    groups = max(1, HKV // 4)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    per_group = max(1, cus // groups)
    k = -(-B // per_group)
    return -(-B // k), k


def attn_swa(q, pool_k, pool_v, slots, pos, rel):
    """SWA decode attention over a ring pool, in place (attn_swa.py:120).
    q [B, HQ, D] bf16, pool_k/pool_v [S, W, HK, D] bf16, slots/pos [B] i64,
    rel [B, HQ, W] bf16. Returns [B, HQ, D]. One native launch reads the
    ring rows through `slots` and the lengths from `pos` directly."""
    B, HQ, D = q.shape
    S, W, HK, _ = pool_k.shape
    assert q.is_contiguous() and rel.is_contiguous()
    assert pool_k.is_contiguous() and pool_v.is_contiguous()
    assert rel.shape == (B, HQ, W), (rel.shape, (B, HQ, W))
    assert slots.dtype == torch.int64 and pos.dtype == torch.int64
    assert W % PAGE == 0, "ring length must be a whole number of pages"
    wgs, k = _ring_grid(B, HK, q.device)
    out, _ = attn.decode_ring(q, pool_k, pool_v, slots.contiguous(),
                              pos.contiguous(), 1.0 / D, W, rel=rel,
                              num_workgroups=wgs, seqs_per_workgroup=k)
    return out


def attn_global(q, pool_kp, pool_vp, flat, pos, rel, Lg):
    """Global decode attention over a page pool, in place (attn_global.py:15).
    q [B, HQ, D] bf16, pool_kp/pool_vp [(P+1), 16, HK, D] bf16, flat [B, Lg]
    i64 per-token rows (dead columns 0), pos [B] i64, rel [B, HQ, E] bf16.
    Returns [B, HQ, D]. The block table is recovered from `flat` in one
    launch (rows of one page are consecutive, so page i of row b is
    flat[b, 16 i] // 16) together with the lengths pos + 1."""
    B, HQ, D = q.shape
    assert q.is_contiguous() and rel.is_contiguous()
    assert pool_kp.is_contiguous() and pool_vp.is_contiguous()
    assert flat.is_contiguous() and flat.shape == (B, Lg)
    assert flat.dtype == torch.int64 and pos.dtype == torch.int64
    ps = pool_kp.shape[1]
    assert ps == PAGE
    table, ctx = attn.decode_table_from_flat(flat, pos.contiguous())
    out, _ = attn.decode_paged(q, pool_kp, pool_vp, table, ctx, 1.0 / D,
                               window=0, rel=rel, return_lse=False)
    return out


def _packed(x, B, T, H, D):
    """[B, H, T, D] view -> [B*T, H, D] with D contiguous and token stride
    uniform across the batch boundary (a view when possible)."""
    xt = x.transpose(1, 2)                       # [B, T, H, D]
    if not (xt.stride(3) == 1 and (B == 1 or xt.stride(0) == T * xt.stride(1))
            and xt.stride(1) % 8 == 0 and xt.stride(2) % 8 == 0):
        xt = xt.contiguous()
    return xt.as_strided((B * T, H, D), (xt.stride(1), xt.stride(2), 1))


def _kv_rows(x):
    """[B, HK, T, D] K or V (any strides) -> a [B, T, HK, D] view that the
    prefill and the KV write both read in place: token-major rows (head_dim
    contiguous) or channel-major ones (tokens contiguous, head_dim strided:
    the sconv output, experiments/DEADENDS.md:631-645), with 16-byte
    aligned rows, dim rows and heads. Anything else (e.g. channel-major with
    T % 8 != 0) becomes a token-major copy, so a caller can rely on both
    kernels accepting the result before it changes any cache."""
    xt = x.transpose(1, 2)                       # [B, T, HK, D]
    B, T, _, D = xt.shape
    if B == 1 and xt.stride(0) % 8 != 0:
        # a size-1 axis: its stride never moves an address
        xt = xt.as_strided(xt.shape, (8,) + tuple(xt.stride()[1:]))
    st = xt.stride()
    aligned = (xt.data_ptr() % 16 == 0 and st[0] % 8 == 0 and
               st[2] % 8 == 0)
    token_major = st[3] == 1 and st[1] % 8 == 0
    channel_major = (st[1] == 1 and D == attn.HEAD_DIM and st[3] % 8 == 0 and
                     st[3] >= T)
    if aligned and (token_major or channel_major):
        return xt
    return xt.contiguous()


def _to_device(rows, dev):
    """int32 rows (a host list) on the device through pinned memory: the
    copy is queued on the stream instead of synchronising it (the caching
    host allocator keeps the staging buffer until the copy has run)."""
    t = torch.tensor(rows, dtype=torch.int32)
    if dev.type != "cuda":
        return t.to(dev)
    return t.pin_memory().to(dev, non_blocking=True)


def _ring_pool(caches):
    """Rings that are rows of one SwaPool (kv.py:231-245: LayerKV hands
    RingKV views of pool rows): (k_pool, v_pool, slots, pages_per_ring),
    the pools as [rows * W / 16, 16, HK, D] page views of the whole pool
    storage and each cache's pool row, so that their appends take one
    launch; None when the rings are not such views."""
    c0 = caches[0]
    if not all(hasattr(c, "k") and hasattr(c, "v") for c in caches):
        return None
    W, HK, D = c0.k.shape
    if W % PAGE:
        return None
    row = W * HK * D
    out = []
    for name in ("k", "v"):
        x0 = getattr(c0, name)
        st = x0.untyped_storage()
        slots = []
        for c in caches:
            x = getattr(c, name)
            if (x.shape != (W, HK, D) or not x.is_contiguous() or
                    x.dtype != x0.dtype or x.device != x0.device or
                    x.untyped_storage().data_ptr() != st.data_ptr() or
                    x.storage_offset() % row):
                return None
            slots.append(x.storage_offset() // row)
        nrow = st.nbytes() // (row * x0.element_size())
        out.append((x0.as_strided((nrow * (W // PAGE), PAGE, HK, D),
                                  (PAGE * HK * D, HK * D, D, 1), 0), slots))
    (kpool, ks), (vpool, vs) = out
    if ks != vs or len(set(ks)) != len(ks):
        return None
    return kpool, vpool, ks, W // PAGE


def _append_rows(k, v, caches, lens):
    """The prefill's cache population (model.py:507-512:
    st.cache.append(kn[i, :lens[i]], vv[i, :lens[i]])) done natively: each
    row's K/V [lens[i], HK, D] is appended to its cache straight from the
    [B, T, HK, D] rows of _kv_rows (channel-major or token-major, a layout
    the write kernels accept, checked before any cache changes), pages
    allocated on the host as
    PagedKV.append does (kv.py:196-198), ring rows as RingKV.append keeps
    them (kv.py:89-103); cache.n advances. Page caches that share one pool
    (GlobalPool rows) take one batched launch for all rows, and so do
    rings that are rows of one SwaPool; other rings and caches with pools
    of their own take one launch each. Returns the int32 block-table rows
    of page caches ([B, num_pages]) or None for rings."""
    B = k.shape[0]
    dev = k.device
    n0 = [int(c.n) for c in caches]
    T = [int(x) for x in lens]
    # every row's start position, length and [0, length] run bounds in one
    # host-to-device copy, from pinned memory so that it does not
    # synchronise the stream
    flat = n0 + T + [x for t in T for x in (0, t)]
    meta = _to_device(flat, dev)
    start, lens_d = meta[:B], meta[B:2 * B]
    paged = all(hasattr(c, "kp") for c in caches)
    for i, c in enumerate(caches):
        if hasattr(c, "kp"):
            c.ensure_pages((n0[i] + T[i] - 1) // c.page_size)
    rows = None
    if paged:
        # the host tables (PagedKV.table, which ensure_pages just extended;
        # a pool's device mirror holds the same ids) in one staged copy
        width = max(len(c.table) for c in caches)
        rows = _to_device([list(c.table) + [-1] * (width - len(c.table))
                           for c in caches], dev)
    shared = paged and all(c.kp is caches[0].kp and c.vp is caches[0].vp
                           for c in caches)
    pooled = None if paged else _ring_pool(caches)
    if shared:
        c0 = caches[0]
        attn.kv_append_rows(k, v, lens_d, start, rows, c0.kp, c0.vp,
                            max_len=max(T))
    elif pooled is not None:
        kpool, vpool, slots, per = pooled
        table = _to_device([[s * per + j for j in range(per)] for s in slots],
                           dev)
        attn.kv_append_rows(k, v, lens_d, start, table, kpool, vpool,
                            max_len=max(T), table_wrap=per)
    else:
        for i, c in enumerate(caches):
            kt = k[i, :T[i]]                     # [T, HK, D] view
            vt = v[i, :T[i]]
            cu = meta[2 * B + 2 * i:2 * B + 2 * i + 2]
            if hasattr(c, "kp"):
                row = (rows[i:i + 1].contiguous() if rows is not None else
                       _to_device([list(c.table)], dev))
                attn.kv_write_paged(kt, vt, row, start[i:i + 1], c.kp, c.vp,
                                    cu_seqlens=cu, max_seqlen=T[i])
            else:
                W = c.k.shape[0]
                per = W // PAGE
                ring = torch.arange(per, dtype=torch.int32, device=dev)[None]
                attn.kv_write_paged(kt, vt, ring, start[i:i + 1],
                                    c.k.view(per, PAGE, *c.k.shape[1:]),
                                    c.v.view(per, PAGE, *c.v.shape[1:]),
                                    cu_seqlens=cu, max_seqlen=T[i],
                                    table_wrap=per)
    for i, c in enumerate(caches):
        c.n = n0[i] + T[i]
    return rows


_CU = {}


def _uniform_cu(B, T, dev):
    """cu_seqlens of B runs of T rows (0, T, .., B*T) as an int32 device
    tensor, made once per (B, T, device) and reused, so that a call does not
    spend a launch on it. Not kept when first made under a graph capture
    (its memory would belong to that graph's pool)."""
    key = (B, T, dev)
    cu = _CU.get(key)
    if cu is None:
        cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=dev)
        if not (dev.type == "cuda" and
                torch.cuda.is_current_stream_capturing()):
            _CU[key] = cu
    return cu


def attn_prefill_fused(q, k, v, rel, q_positions, kv_positions, window,
                       block_m=64, block_n=64, caches=None, lens=None):
    """Fused prefill attention over in-batch K/V (attn_prefill.py:144).
    q [B, H, T, D], k/v [B, HK, T, D] bf16 (any strides), rel [B, H, T, E]
    bf16 with rel.stride(3) == 1, q_positions/kv_positions [T] i64 (the
    engine's arange), window None (global) or W (SWA, E == W).
    Returns [B, T, H, D] bf16. block_m / block_n are accepted for signature
    compatibility; the kernel's tiles are fixed for gfx950.

    K/V are read in place in the layout they arrive in: the sconv's
    channel-major output (stride 1 along T, attn_prefill.py:162-168) or
    token-major rows; only layouts neither kernel reads (channel-major with
    T % 8 != 0, misaligned views) are copied first.

    caches / lens (optional, not in the reference signature): the B rows'
    cache objects (PagedKV- or RingKV-shaped, empty: a whole-prompt
    prefill) and live lengths (default T) whose population the engine does
    just before this call (model.py:507-512). The adapter then appends the
    rows itself, in one launch, from the same in-place K/V; the attention
    reads the K/V tensors in place either way (reading them back from the
    pages just written measured slower)."""
    B, H, T, D = q.shape
    HK = k.shape[1]
    E = rel.shape[3]
    assert k.shape == (B, HK, T, D) and v.shape == (B, HK, T, D)
    assert rel.shape == (B, H, T, E) and rel.stride(3) == 1
    assert q_positions.shape == (T,) and kv_positions.shape == (T,)
    assert q_positions.dtype == torch.int64
    assert kv_positions.dtype == torch.int64
    assert H % HK == 0
    if window is not None:
        assert E == window, (E, window)
    dev = q.device
    # The kernel derives positions from indices, i.e. it computes with
    # q_positions == kv_positions == p0 + arange(T) for any common p0 (the
    # mask and the bias depend on q - k only); that is what the engine
    # passes (model.py:526-528). Anything else is rejected: on the device
    # the check feeds the kernel's reject flag (NaN output, no host sync),
    # on the host (CPU positions, or TMOPT_CHECK set) it raises.
    if (q_positions.device.type == "cpu" or
            kv_positions.device != q_positions.device or
            os.environ.get("TMOPT_CHECK")):
        pos = torch.stack([q_positions, kv_positions.to(q_positions.device)])
        ar = torch.arange(T, device=pos.device)
        assert not bool(((pos - q_positions[:1]) != ar).any()), \
            "q_positions and kv_positions must be the same p0 + arange(T)"
        reject = None
    else:
        reject = attn.prefill_check_positions(q_positions.contiguous(),
                                              kv_positions.contiguous())
    qp = _packed(q, B, T, H, D)
    rt = rel.transpose(1, 2)                     # [B, T, H, E]
    if not (B == 1 or rt.stride(0) == T * rt.stride(1)):
        rt = rt.contiguous()
    relp = rt.as_strided((B * T, H, E), (rt.stride(1), rt.stride(2), 1))
    out = torch.empty((B, T, H, D), dtype=q.dtype, device=dev)
    cu = _uniform_cu(B, T, dev)
    w = 0 if window is None else int(window)
    kr, vr = _kv_rows(k), _kv_rows(v)            # [B, T, HK, D]
    if caches is not None:
        assert len(caches) == B
        assert all(int(c.n) == 0 for c in caches), \
            "caches must be empty (chunked prefill: prefill_chunk_state)"
        lens = [T] * B if lens is None else [int(x) for x in lens]
        _append_rows(kr, vr, caches, lens)
    attn.prefill_varlen(qp, kr, vr, cu, 1.0 / D, window=w, max_seqlen=T,
                        rel=relp, out=out.view(B * T, H, D),
                        return_lse=False, reject=reject)
    return out


# --------------------------------------------------------------------------
# chunked prefill over the engine's KV storage
# --------------------------------------------------------------------------
# The reference prefills whole prompts and leaves chunked prefill at
# Engine.prefill (engine/pyengine/scheduler.py:22-23). These adapters are
# that seam over its own storage: a chunk's queries attend to the
# sequence's cached prior context (GlobalPool pages / SwaPool ring rows,
# kv.py:215-268) plus the chunk's own keys, then the chunk is appended as
# PagedKV.append / RingKV.append would (kv.py:193-205, :89-103). The prior
# keys are read in place from the pool (the ring through a ring block
# table), the chunk's own keys from the packed rows, so the append can come
# after the attention, which a ring requires (it overwrites positions the
# chunk's first queries still see).

def _chunk_cu(q, cu_seqlens, max_seqlen):
    """(cu_seqlens, max_seqlen) of a chunk batch: one sequence of
    q.shape[0] tokens when cu_seqlens is None (no device read); otherwise
    max_seqlen as given, or read back once (a host synchronisation, which a
    graph capture must avoid by passing it) for both launches."""
    if cu_seqlens is None:
        cu = torch.full((2,), q.shape[0], dtype=torch.int32,
                        device=q.device)
        cu[0] = 0
        return cu, q.shape[0]
    assert cu_seqlens.dtype == torch.int32
    if max_seqlen is None:
        max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max())
    return cu_seqlens, max_seqlen


def attn_prefill_chunk_swa(q, k, v, rel, pool_k, pool_v, slots, prior,
                           cu_seqlens=None, max_seqlen=None):
    """Chunked prefill of a sliding-window layer over SwaPool ring rows.

    q [total, H, D], k/v [total, HK, D] bf16: the chunks of B sequences
    packed by cu_seqlens [B+1] int32 (None: one sequence); rel [total, H, W]
    bf16 or None; pool_k/pool_v [S+1, W, HK, D] (SwaPool; window = W, rel
    extent = W as attn_swa asserts); slots [B] i64 ring rows; prior [B]
    i64 tokens each ring has seen (RingKV.n). Scale 1/D. Attends, then
    appends the chunks to the rings (only the last W positions survive).
    max_seqlen: the longest chunk; with several sequences pass it to keep
    the call free of host synchronisation (graph capture).
    Returns out [total, H, D] bf16."""
    total, H, D = q.shape
    S1, W, HK, _ = pool_k.shape
    assert pool_k.is_contiguous() and pool_v.is_contiguous()
    assert pool_v.shape == pool_k.shape and W % PAGE == 0
    assert slots.dtype == torch.int64 and prior.dtype == torch.int64
    if rel is not None:
        assert rel.shape == (total, H, W), (rel.shape, (total, H, W))
    cu, max_seqlen = _chunk_cu(q, cu_seqlens, max_seqlen)
    per = W // PAGE
    kp = pool_k.view(S1 * per, PAGE, HK, D)
    vp = pool_v.view(S1 * per, PAGE, HK, D)
    table = (slots[:, None] * per + torch.arange(
        per, device=q.device, dtype=torch.int64)[None]).to(torch.int32)
    start = prior.to(torch.int32)
    out, _ = attn.prefill_varlen(q, k, v, cu, 1.0 / D, window=W,
                                 max_seqlen=max_seqlen, prior_lens=start,
                                 k_pool=kp, v_pool=vp, block_table=table,
                                 table_wrap=per, rel=rel, return_lse=False)
    attn.kv_write_paged(k, v, table, start, kp, vp, cu_seqlens=cu,
                        max_seqlen=max_seqlen, table_wrap=per)
    return out


def attn_prefill_chunk_global(q, k, v, rel, pool_kp, pool_vp, table_dev,
                              slots, prior, cu_seqlens=None,
                              max_seqlen=None):
    """Chunked prefill of a global layer over GlobalPool pages.

    q [total, H, D], k/v [total, HK, D] bf16 packed by cu_seqlens [B+1]
    int32 (None: one sequence); rel [total, H, E] bf16 or None;
    pool_kp/pool_vp [(P+1), 16, HK, D]; table_dev [S+1, num_pages] i64
    (GlobalPool's device page table, already covering each sequence's
    prior + chunk positions: PagedKV.ensure_pages, kv.py:170-191); slots
    [B] i64; prior [B] i64 (PagedKV.n). Scale 1/D, causal. Attends, then
    appends the chunks through the page table. max_seqlen: the longest
    chunk; with several sequences pass it to keep the call free of host
    synchronisation (graph capture). Returns out [total, H, D]."""
    total, H, D = q.shape
    assert pool_kp.is_contiguous() and pool_vp.is_contiguous()
    assert pool_kp.shape[1] == PAGE
    assert table_dev.dtype == torch.int64 and table_dev.dim() == 2
    assert slots.dtype == torch.int64 and prior.dtype == torch.int64
    if rel is not None:
        assert rel.shape[:2] == (total, H)
    cu, max_seqlen = _chunk_cu(q, cu_seqlens, max_seqlen)
    table = table_dev[slots].to(torch.int32)
    start = prior.to(torch.int32)
    out, _ = attn.prefill_varlen(q, k, v, cu, 1.0 / D, window=0,
                                 max_seqlen=max_seqlen, prior_lens=start,
                                 k_pool=pool_kp, v_pool=pool_vp,
                                 block_table=table, rel=rel,
                                 return_lse=False)
    attn.kv_write_paged(k, v, table, start, pool_kp, pool_vp, cu_seqlens=cu,
                        max_seqlen=max_seqlen)
    return out


def prefill_chunk_state(q, k, v, rel, cache):
    """One sequence's chunk against its own cache object, shaped like the
    reference's PagedKV (kp, vp [P, 16, HK, D], table_dev_row [num_pages]
    i64, n, page_size, ensure_pages(last_page)) or RingKV (k, v [W, HK, D],
    n): the cache's pages are allocated for the chunk on the host as
    PagedKV.append does (kv.py:196-198), the chunk attends to the n cached
    tokens plus itself (window = W on a ring, causal on pages; scale 1/D)
    and is appended, and cache.n advances by the chunk length.
    q [T, H, D], k/v [T, HK, D] bf16, rel [T, H, E] or None.
    Returns out [T, H, D] bf16."""
    T, H, D = q.shape
    dev = q.device
    n = int(cache.n)
    meta = _to_device([n, 0, T], dev)            # prior, cu_seqlens
    prior, cu = meta[0:1], meta[1:3]
    if hasattr(cache, "kp"):
        ps = cache.page_size
        assert ps == PAGE
        cache.ensure_pages((n + T - 1) // ps)
        if getattr(cache, "table_dev_row", None) is not None:
            table = cache.table_dev_row.to(torch.int32)[None].contiguous()
        else:                                    # a PagedKV with its own pool
            table = _to_device([cache.table], dev)
        kp, vp, wrap, window = cache.kp, cache.vp, 0, 0
    else:
        W = cache.k.shape[0]
        assert W % PAGE == 0 and cache.k.is_contiguous()
        per = W // PAGE
        kp = cache.k.view(per, PAGE, *cache.k.shape[1:])
        vp = cache.v.view(per, PAGE, *cache.v.shape[1:])
        table = torch.arange(per, dtype=torch.int32, device=dev)[None]
        wrap, window = per, W
    out, _ = attn.prefill_varlen(q, k, v, cu, 1.0 / D, window=window,
                                 max_seqlen=T, prior_lens=prior, k_pool=kp,
                                 v_pool=vp, block_table=table,
                                 table_wrap=wrap, rel=rel, return_lse=False)
    attn.kv_write_paged(k, v, table, prior, kp, vp, cu_seqlens=cu,
                        max_seqlen=T, table_wrap=wrap)
    cache.n = n + T
    return out
