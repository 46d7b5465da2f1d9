"""The reference-signature adapters (attn_swa, attn_global,
attn_prefill_fused) against the oracle's restatement of the model
semantics: scale 1/head_dim, fused relative bias, ring SWA pool, per-token
`flat` rows built exactly like model.py:938-945, padded [B,H,T,D] prefill
with channel-major K/V. Geometry edges of the reference's own arm
(t_fused_attn.py:119-122): 0, 3, 200, 511, 512, 513, 800, 1500 and a dead
row at position 0 on the scratch slot."""
import pytest
import torch

from helpers import assert_out_close
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def test_attn_swa_ring_pool(tm, dev):
    g = torch.Generator().manual_seed(13)
    W, HK, D, HQ = 512, 16, 128, 64
    pos = torch.tensor([0, 3, 200, 511, 512, 513, 800, 0])
    MB = pos.shape[0]
    # stale random bytes everywhere (dead slots must be excluded by the
    # window, never read as zeros); shuffled slot map, scratch row last
    pool_k = (torch.randn((MB + 1, W, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    pool_v = (torch.randn((MB + 1, W, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    slots = torch.cat([torch.randperm(MB - 1, generator=g),
                       torch.tensor([MB])])
    q = torch.randn((MB, HQ, D), generator=g).to(torch.bfloat16)
    rel = (torch.randn((MB, HQ, W), generator=g) * 0.5).to(torch.bfloat16)
    ref, _ = attn_ref.decode_reference_semantics(q, pool_k, pool_v, slots,
                                                 pos, rel, W)
    out = tm.attn_swa(q.to(dev), pool_k.to(dev), pool_v.to(dev),
                      slots.to(dev), pos.to(dev), rel.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (MB, HQ, D) and out.dtype == torch.bfloat16
    assert_out_close(out, ref, "attn_swa")


def test_attn_global_flat_rows(tm, dev):
    g = torch.Generator().manual_seed(14)
    HK, D, HQ, E = 8, 128, 64, 1024
    pos_host = [0, 3, 200, 511, 512, 513, 800, 1500, 0]
    MB = len(pos_host)
    num_pages = (max(pos_host) + 16) // 16 + 2
    total = MB * num_pages
    kp = (torch.randn((total + 1, 16, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    vp = (torch.randn((total + 1, 16, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    table_dev = torch.zeros((MB + 1, num_pages), dtype=torch.int64)
    table_dev[:MB] = torch.randperm(total, generator=g).view(MB, num_pages)
    table_dev[MB] = total                                  # scratch page
    slots = torch.cat([torch.randperm(MB - 1, generator=g),
                       torch.tensor([MB])])
    pos = torch.tensor(pos_host)
    # model.py:938-945 + decode_batch_ctx #2 (model.py:849-857)
    Lg = max(pos_host) + 1
    j = torch.arange(Lg)
    table = table_dev[slots]
    flat = table[:, j // 16] * 16 + (j % 16)[None, :]
    flat = torch.where(j[None, :] < (pos + 1)[:, None], flat,
                       torch.zeros_like(flat))
    q = torch.randn((MB, HQ, D), generator=g).to(torch.bfloat16)
    rel = (torch.randn((MB, HQ, E), generator=g) * 0.5).to(torch.bfloat16)
    ref, _ = attn_ref.decode_paged(q, kp, vp, table, pos + 1, 1.0 / D,
                                   rel=rel)
    out = tm.attn_global(q.to(dev), kp.to(dev), vp.to(dev),
                         flat.contiguous().to(dev), pos.to(dev), rel.to(dev),
                         Lg)
    torch.cuda.synchronize()
    assert_out_close(out, ref, "attn_global")


@pytest.mark.parametrize("window,E", [(None, 1024), (64, 64)])
@pytest.mark.parametrize("hq,hk", [(32, 4), (64, 16), (48, 4)])
@pytest.mark.parametrize("T", [200, 77])
def test_attn_prefill_fused_padded_batch(tm, dev, window, E, hq, hk, T):
    """T = 200: the kernel reads the channel-major K/V in place (runs of
    200 keys at the batch stride, last tile partial); T = 77 (not a
    multiple of 8, so dim rows are not 16-byte aligned): the copy path."""
    g = torch.Generator().manual_seed(15)
    B, D = 3, 128
    q = torch.randn((B, T, hq, D), generator=g).to(torch.bfloat16).transpose(
        1, 2)                                              # [B,H,T,D] view
    # K/V channel-major, as the eager sconv hands them over
    kc = torch.randn((B, hk, D, T), generator=g).to(torch.bfloat16)
    vc = torch.randn((B, hk, D, T), generator=g).to(torch.bfloat16)
    k, v = kc.transpose(2, 3), vc.transpose(2, 3)          # stride 1 along T
    rel = (torch.randn((B, T, hq, E), generator=g) * 0.5).to(
        torch.bfloat16).transpose(1, 2)                    # [B,H,T,E]
    positions = torch.arange(T)
    ref = attn_ref.prefill_reference_semantics(q, k, v, rel, positions,
                                               window)
    out = tm.attn_prefill_fused(q.to(dev), k.to(dev), v.to(dev), rel.to(dev),
                                positions.to(dev), positions.to(dev), window)
    torch.cuda.synchronize()
    assert out.shape == (B, T, hq, D)
    assert_out_close(out, ref, f"prefill_fused w={window} {hq}/{hk}")


def test_attn_prefill_fused_positions(tm, dev):
    """Positions: any common offset p0 + arange(T) gives the arange result
    (the mask and bias depend on q - k only); anything else is rejected on
    the device (NaN output, no host synchronisation) and on the host for
    CPU position tensors."""
    g = torch.Generator().manual_seed(16)
    B, T, D, hq, hk, E = 2, 100, 128, 32, 4, 64
    q = torch.randn((B, hq, T, D), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((B, hk, T, D), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((B, hk, T, D), generator=g).to(torch.bfloat16).to(dev)
    rel = torch.randn((B, hq, T, E), generator=g).to(torch.bfloat16).to(dev)
    ar = torch.arange(T, device=dev)
    base = tm.attn_prefill_fused(q, k, v, rel, ar, ar, E)
    off = tm.attn_prefill_fused(q, k, v, rel, ar + 4096, ar + 4096, E)
    torch.cuda.synchronize()
    assert torch.isfinite(base.float()).all()
    assert torch.equal(base, off)
    bad_q = ar.clone()
    bad_q[50] += 1
    # the device-side check itself (one work-group, flag always written)
    flags = [int(tm.prefill_check_positions(qp, kp)) for qp, kp in
             ((ar, ar), (ar + 4096, ar + 4096), (bad_q, ar), (ar, ar + 1),
              (ar.flip(0), ar.flip(0)))]
    assert flags == [0, 0, 1, 1, 1]
    for qp, kp in ((bad_q, ar), (ar, ar + 1), (ar.flip(0), ar.flip(0))):
        out = tm.attn_prefill_fused(q, k, v, rel, qp, kp, E)
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all()
    with pytest.raises(AssertionError):
        tm.attn_prefill_fused(q, k, v, rel, bad_q.cpu(), ar.cpu(), E)


def test_positions_check_lengths(tm, dev):
    """The one-work-group position check strides over T: a mismatch at the
    last index is found for T below, at and past the work-group size, and
    T = 1 (only the offset) passes."""
    for T in (1, 1024, 1025, 5000):
        ar = torch.arange(T, device=dev) + 7
        assert int(tm.prefill_check_positions(ar, ar)) == 0
        if T > 1:
            for which in ("q", "kv"):
                q, k = ar.clone(), ar.clone()
                (q if which == "q" else k)[-1] += 1
                assert int(tm.prefill_check_positions(q, k)) == 1, (T, which)


@pytest.mark.parametrize("T,lens", [(200, [200, 150, 77]), (77, [77, 60, 5])])
@pytest.mark.parametrize("kind", ["global", "swa", "swa_pooled"])
def test_attn_prefill_fused_populates_caches(tm, dev, kind, T, lens):
    """attn_prefill_fused given the rows' caches (the engine's
    st.cache.append(kn[i, :lens[i]], vv[i, :lens[i]]) at model.py:507-512)
    appends the channel-major K/V itself (pages of a shared pool, separate
    rings, or rings that are rows of one SwaPool in a permuted slot order,
    kv.py:231-245) and reads the K/V tensors for the attention. The live
    rows equal the cache-less path's bitwise, every cache holds its row's
    tokens bit-exact, n advances, pool rows no cache owns stay untouched.
    T = 77: channel-major dim rows that are not 16-byte aligned, which
    neither kernel reads in place: the adapter copies them before it
    touches any cache."""
    import numpy as np
    from helpers import PagedCache, RingCache
    from oracle import kv_ref
    g = torch.Generator().manual_seed(17)
    B, D = 3, 128
    if kind == "global":
        hq, hk, E, window = 64, 8, 1024, None
    else:
        hq, hk, E, window = 64, 16, 512, 512
    bf = torch.bfloat16
    q = torch.randn((B, T, hq, D), generator=g).to(bf).to(dev).transpose(1, 2)
    kc = torch.randn((B, hk * D, T), generator=g).to(bf).to(dev)
    vc = torch.randn((B, hk * D, T), generator=g).to(bf).to(dev)
    k = kc.transpose(1, 2).view(B, T, hk, D).transpose(1, 2)   # sconv layout
    v = vc.transpose(1, 2).view(B, T, hk, D).transpose(1, 2)
    rel = (torch.randn((B, T, hq, E), generator=g) * 0.5).to(bf).to(
        dev).transpose(1, 2)
    ar = torch.arange(T, device=dev)
    base = tm.attn_prefill_fused(q, k, v, rel, ar, ar, window)
    if kind == "global":
        P = 64
        free = torch.randperm(P, generator=g).tolist()
        kp = torch.zeros((P, 16, hk, D), dtype=bf, device=dev)
        vp = torch.zeros_like(kp)
        caches = [PagedCache(kp, vp, free, torch.zeros(
            P // 2, dtype=torch.int64, device=dev)) for _ in range(B)]
    elif kind == "swa":
        caches = [RingCache(torch.zeros((E, hk, D), dtype=bf, device=dev),
                            torch.zeros((E, hk, D), dtype=bf, device=dev))
                  for _ in range(B)]
    else:
        pk = torch.zeros((B + 2, E, hk, D), dtype=bf, device=dev)
        pv = torch.zeros_like(pk)
        slots = [3, 0, 2]
        caches = [RingCache(pk[s], pv[s]) for s in slots]
    out = tm.attn_prefill_fused(q, k, v, rel, ar, ar, window, caches=caches,
                                lens=lens)
    torch.cuda.synchronize()
    if kind == "swa_pooled":
        for s in (1, 4):
            assert not bool(pk[s].any()) and not bool(pv[s].any()), s
    for i, n in enumerate(lens):
        assert torch.equal(out[i, :n], base[i, :n]), f"row {i}"
        c = caches[i]
        assert c.n == n
        for x, pool, ring in ((k, "kp", "k"), (v, "vp", "v")):
            rows = x[i].transpose(0, 1)[:n].contiguous()         # [n, hk, D]
            if kind == "global":
                got = kv_ref.gather(kv_ref.as_u16(getattr(c, pool)), c.table,
                                    n)
            else:
                got = kv_ref.gather(
                    kv_ref.as_u16(getattr(c, ring)).reshape(E // 16, 16, hk, D),
                    list(range(E // 16)), n, table_wrap=E // 16,
                    lo=max(0, n - E))
                rows = rows[max(0, n - E):]
            assert np.array_equal(got, kv_ref.as_u16(rows)), \
                f"cache row {i} ({ring})"


def test_attn_swa_model_shape_ring_grid(tm, dev):
    """attn_swa at the model's SWA shape (B = 64, W = E = 512, 64Q/16KV):
    full rings and short ones (positions 0..30000), so the ring-aligned
    work split (whole rings per work-group) meets rows of every length;
    every row against the oracle's model semantics."""
    g = torch.Generator().manual_seed(18)
    B, W, HK, D, HQ = 64, 512, 16, 128, 64
    pos = torch.randint(0, 30000, (B,), generator=g)
    pos[:8] = torch.tensor([0, 1, 15, 16, 255, 510, 511, 512])
    slots = torch.randperm(B, generator=g)
    pool_k = (torch.randn((B + 1, W, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    pool_v = (torch.randn((B + 1, W, HK, D), generator=g) * 0.5).to(
        torch.bfloat16)
    q = torch.randn((B, HQ, D), generator=g).to(torch.bfloat16)
    rel = (torch.randn((B, HQ, W), generator=g) * 0.5).to(torch.bfloat16)
    ref, _ = attn_ref.decode_reference_semantics(q, pool_k, pool_v, slots,
                                                 pos, rel, W)
    out = tm.attn_swa(q.to(dev), pool_k.to(dev), pool_v.to(dev),
                      slots.to(dev), pos.to(dev), rel.to(dev))
    torch.cuda.synchronize()
    assert_out_close(out, ref, "attn_swa model shape")


def _edge_rows(T, extra, g):
    """Query rows for sampled checks: the run's ends, the band edges of
    the model's extents (511-513, 1023-1025) and random ones."""
    fixed = [0, 1, 2, 63, 64, 65, 255, 256, 511, 512, 513, 1023, 1024,
             1025, T - 2, T - 1]
    rnd = torch.randint(0, T, (extra,), generator=g).tolist()
    return sorted({r for r in fixed + rnd if 0 <= r < T})


@pytest.mark.parametrize("with_caches", [False, True])
@pytest.mark.parametrize("kind", ["swa", "global"])
def test_attn_prefill_fused_model_shape(tm, dev, kind, with_caches):
    """attn_prefill_fused at the shape the bench's adapter lines time
    (B = 6, T = 1536; SWA 64Q/16KV, W = E = 512; global 64Q/8KV, E =
    1024), K/V channel-major as the sconv hands them over (read in place),
    with and without the rows' caches (rings / shared page pool with a
    shuffled free list), on sampled rows of every batch row against the
    oracle's model semantics."""
    from helpers import PagedCache, RingCache
    g = torch.Generator().manual_seed(19)
    gd = torch.Generator(device=dev).manual_seed(19)
    B, T, D = 6, 1536, 128
    if kind == "global":
        hq, hk, E, window = 64, 8, 1024, None
    else:
        hq, hk, E, window = 64, 16, 512, 512
    bf = torch.bfloat16

    def rnd(*shape, s=1.0):
        return (torch.randn(shape, generator=gd, device=dev) * s).to(bf)
    q = rnd(B, T, hq, D).transpose(1, 2)                       # [B,H,T,D]
    k = rnd(B, hk * D, T).transpose(1, 2).view(B, T, hk, D).transpose(1, 2)
    v = rnd(B, hk * D, T).transpose(1, 2).view(B, T, hk, D).transpose(1, 2)
    assert k.stride(2) == 1 and k.stride(3) == T            # channel-major
    rel = rnd(B, T, hq, E, s=0.5).transpose(1, 2)              # [B,H,T,E]
    ar = torch.arange(T, device=dev)
    caches = None
    if with_caches and kind == "global":
        P = B * T // 16 + 64
        free = torch.randperm(P, generator=g).tolist()
        kp = torch.zeros((P, 16, hk, D), dtype=bf, device=dev)
        vp = torch.zeros_like(kp)
        caches = [PagedCache(kp, vp, free, torch.zeros(
            T // 16 + 8, dtype=torch.int64, device=dev)) for _ in range(B)]
    elif with_caches:
        # rows of one SwaPool in a permuted slot order (the engine's pooled
        # rings): one append launch for the six rows, T > W, so only each
        # row's last W tokens survive (RingKV's drop rule)
        pk = torch.zeros((B + 1, E, hk, D), dtype=bf, device=dev)
        pv = torch.zeros_like(pk)
        slots = torch.randperm(B + 1, generator=g)[:B].tolist()
        caches = [RingCache(pk[s], pv[s]) for s in slots]
    out = tm.attn_prefill_fused(q, k, v, rel, ar, ar, window, caches=caches)
    torch.cuda.synchronize()
    assert out.shape == (B, T, hq, D)
    if with_caches and kind == "swa":
        pos = torch.arange(T - E, T)
        for b, s in enumerate(slots):
            for x, pool in ((k, pk), (v, pv)):
                want = x[b].transpose(0, 1)[T - E:]           # [E, hk, D]
                assert torch.equal(pool[s][pos % E], want), (b, s)
    rows = _edge_rows(T, 24, g)
    ref = attn_ref.prefill_reference_semantics(
        q.cpu(), k.cpu(), v.cpu(), rel.cpu(), ar.cpu(), window, rows=rows)
    assert_out_close(out[:, rows], ref,
                     f"prefill_fused {kind} B6 T1536 caches={with_caches}")
