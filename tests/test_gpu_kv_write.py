"""Bit-exact parity of the HIP KV-cache write against the numpy oracle.

Covers the flat slot-mapping form (index_put_ semantics, model.py:941-948),
the block-table form for prefill runs, decode steps and ring pools, strided
inputs, skipped rows, and the reference's structural pins restated from
engine/pyengine/tests/t_b3.py:81-130.
"""
import numpy as np
import pytest
import torch

from oracle import kv_ref

pytestmark = pytest.mark.gpu


def _bf16(shape, g):
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def test_write_slots_matches_index_put(tm, dev):
    g = torch.Generator().manual_seed(11)
    T, H, D, P = 37, 4, 128, 40
    k = _bf16((T, H, D), g)
    v = _bf16((T, H, D), g)
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    slots = torch.randperm(P * 16, generator=g)[:T].to(torch.int64)
    slots[::7] = -1                       # skipped rows
    slots[3] = P * 16 + 5                 # beyond the pool: skipped
    want_k = kv_ref.write_slots(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                slots.numpy())
    want_v = kv_ref.write_slots(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                slots.numpy())
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_slots(k.to(dev), v.to(dev), slots.to(dev), kd, vd)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_write_slots_strided_input(tm, dev):
    g = torch.Generator().manual_seed(12)
    T, H, D, P = 20, 4, 128, 8
    big = _bf16((T, H, 2 * D), g)
    k = big[:, :, :D]                      # head stride 256, token 1024
    v = big[:, :, D:]
    assert not k.is_contiguous()
    kp = torch.zeros((P, 16, H, D), dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    slots = torch.randperm(P * 16, generator=g)[:T].to(torch.int64)
    want_k = kv_ref.write_slots(kv_ref.as_u16(kp).copy(),
                                kv_ref.as_u16(k.contiguous()), slots.numpy())
    want_v = kv_ref.write_slots(kv_ref.as_u16(vp).copy(),
                                kv_ref.as_u16(v.contiguous()), slots.numpy())
    bd = big.to(dev)
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_slots(bd[:, :, :D], bd[:, :, D:], slots.to(dev), kd, vd)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


@pytest.mark.parametrize("wrap", [0, 3])
def test_write_paged_varlen(tm, dev, wrap):
    g = torch.Generator().manual_seed(13 + wrap)
    H, D = 4, 128
    lens = [5, 33, 16, 1, 70]
    start = [0, 7, 100, 3, 20]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    k = _bf16((T, H, D), g)
    v = _bf16((T, H, D), g)
    need = 10 if not wrap else wrap
    P = 64
    perm = torch.randperm(P, generator=g)
    table = perm[:len(lens) * need].view(len(lens), need).to(torch.int32)
    table[0, 0] = P + 3                    # invalid entry: never written
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu, start, table.numpy(), 16, wrap)
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                cu, start, table.numpy(), 16, wrap)
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev),
                      torch.tensor(start, dtype=torch.int32, device=dev), kd,
                      vd, cu_seqlens=torch.from_numpy(cu).to(dev),
                      table_wrap=wrap)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_write_paged_decode_step(tm, dev):
    """One token per sequence at position ctx-1 (model.py:938-948)."""
    g = torch.Generator().manual_seed(21)
    B, H, D, P, npg = 9, 4, 128, 128, 8
    k = _bf16((B, H, D), g)
    v = _bf16((B, H, D), g)
    table = torch.randperm(P, generator=g)[:B * npg].view(B, npg).to(
        torch.int32)
    pos = torch.tensor([0, 3, 15, 16, 17, 63, 64, 100, 127], dtype=torch.int32)
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                None, pos.numpy(), table.numpy())
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                None, pos.numpy(), table.numpy())
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev), pos.to(dev), kd, vd)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_t_b3_paged_pin(tm, dev):
    """t_b3.py:119-130: page size 4, shuffled free order of 8 pages, appends
    of 5 then 8 tokens; gather reproduces logical order through a table
    that equals order[:4]."""
    g = torch.Generator().manual_seed(1)
    H, D = 2, 8
    ks = _bf16((13, H, D), g)
    vs = _bf16((13, H, D), g)
    order = torch.randperm(8, generator=g)
    table = order[:4].to(torch.int32)[None].contiguous()
    kp = torch.zeros((8, 4, H, D), dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    for s0, s1 in ((0, 5), (5, 13)):
        tm.kv_write_paged(
            ks[s0:s1].to(dev), vs[s0:s1].to(dev), table.to(dev),
            torch.tensor([s0], dtype=torch.int32, device=dev), kp, vp,
            cu_seqlens=torch.tensor([0, s1 - s0], dtype=torch.int32,
                                    device=dev))
    torch.cuda.synchronize()
    got_k = kv_ref.gather(kv_ref.as_u16(kp), table[0].numpy(), 13, page=4)
    got_v = kv_ref.gather(kv_ref.as_u16(vp), table[0].numpy(), 13, page=4)
    assert np.array_equal(got_k, kv_ref.as_u16(ks))
    assert np.array_equal(got_v, kv_ref.as_u16(vs))


def test_t_b3_ring_pin(tm, dev):
    """t_b3.py:100-117: ring capacity 8 (2 pages of 4), 13 tokens appended
    as 3 then 10 (oversized mid-stream) or 13 at once: the live window is
    tokens 5..12 in either case."""
    g = torch.Generator().manual_seed(2)
    H, D = 2, 8
    ks = _bf16((13, H, D), g)
    vs = _bf16((13, H, D), g)
    table = torch.tensor([[6, 2]], dtype=torch.int32, device=dev)
    for chunks in (((0, 3), (3, 13)), ((0, 13),)):
        kp = torch.zeros((8, 4, H, D), dtype=torch.bfloat16, device=dev)
        vp = torch.zeros_like(kp)
        for s0, s1 in chunks:
            tm.kv_write_paged(
                ks[s0:s1].to(dev), vs[s0:s1].to(dev), table,
                torch.tensor([s0], dtype=torch.int32, device=dev), kp, vp,
                cu_seqlens=torch.tensor([0, s1 - s0], dtype=torch.int32,
                                        device=dev), table_wrap=2)
        torch.cuda.synchronize()
        got = kv_ref.gather(kv_ref.as_u16(kp), [6, 2], 13, page=4,
                            table_wrap=2, lo=5)
        assert np.array_equal(got, kv_ref.as_u16(ks[5:]))
        got = kv_ref.gather(kv_ref.as_u16(vp), [6, 2], 13, page=4,
                            table_wrap=2, lo=5)
        assert np.array_equal(got, kv_ref.as_u16(vs[5:]))


@pytest.mark.parametrize("wrap", [0, 9])
def test_write_paged_long_runs_and_single_tokens(tm, dev, wrap):
    """A mixed step: two long runs beside a hundred one-token rows, so the
    launch packs several 16-byte chunks per lane (a grid sized by the
    longest run would otherwise be mostly empty work-groups)."""
    g = torch.Generator().manual_seed(29 + wrap)
    H, D = 4, 128
    lens = [2000] + [1] * 100 + [777]
    S = len(lens)
    start = torch.randint(0, 300, (S,), generator=g).tolist()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    k = _bf16((T, H, D), g)
    v = _bf16((T, H, D), g)
    # every row gets distinct pages for the positions it writes; the rest
    # of its table row points outside the pool
    per = [wrap if wrap else (s + n + 15) // 16 for s, n in zip(start, lens)]
    width = max(per)
    P = sum(per) + 8
    perm = torch.randperm(P, generator=g).to(torch.int32)
    table = torch.full((S, width), P + 5, dtype=torch.int32)
    off = 0
    for i, n in enumerate(per):
        table[i, :n] = perm[off:off + n]
        off += n
    table[3, start[3] // 16 % (wrap or 10**9)] = P + 11   # skipped write
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu, start, table.numpy(), 16, wrap)
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                cu, start, table.numpy(), 16, wrap)
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev),
                      torch.tensor(start, dtype=torch.int32, device=dev), kd,
                      vd, cu_seqlens=torch.from_numpy(cu).to(dev),
                      table_wrap=wrap)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def _chunks_per_lane(max_len, num_seqs, HKV=4, D=128):
    """The launch's chunks-per-lane rule (kv_write.hip): the smallest power
    of two up to 16 that keeps (max_len * HKV * D / 8) / (256 R) x num_seqs
    within 32768 work-groups."""
    work = max_len * HKV * D // 8
    R = 1
    while True:
        bx = -(-work // (256 * R))
        if R == 16 or bx == 1 or bx * num_seqs <= 32768:
            return R
        R *= 2


@pytest.mark.parametrize("n_single,want_r", [(99, 4), (199, 8), (399, 16)])
@pytest.mark.parametrize("wrap", [0, 200])
def test_write_paged_many_chunks_per_lane(tm, dev, n_single, want_r, wrap):
    """A 4096-token run beside hundreds of one-token rows (a mixed step at
    real batch sizes): the launch packs 4, 8 or 16 chunks per lane; every
    token must land bit-exact, with and without a ring table (a ring of 200
    pages = 3200 positions, so the long run's first 896 tokens are dropped
    as RingKV.append drops them)."""
    assert _chunks_per_lane(4096, n_single + 1) == want_r
    g = torch.Generator().manual_seed(40 + n_single + wrap)
    H, D = 4, 128
    lens = [4096] + [1] * n_single
    S = len(lens)
    start = [int(x) for x in torch.randint(0, 5000, (S,), generator=g)]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    k = _bf16((T, H, D), g)
    v = _bf16((T, H, D), g)
    # distinct pages for the table entries a run writes, -1 elsewhere
    used = []
    for s0, n in zip(start, lens):
        keep = max(s0, s0 + n - wrap * 16) if wrap else s0
        lps = {p // 16 for p in range(keep, s0 + n)}
        used.append(sorted({lp % wrap for lp in lps} if wrap else lps))
    width = wrap if wrap else max(u[-1] + 1 for u in used)
    P = sum(len(u) for u in used) + 3
    perm = torch.randperm(P, generator=g).to(torch.int32)
    table = torch.full((S, width), -1, dtype=torch.int32)
    off = 0
    for i, u in enumerate(used):
        table[i, u] = perm[off:off + len(u)]
        off += len(u)
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu, start, table.numpy(), 16, wrap)
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                cu, start, table.numpy(), 16, wrap)
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev),
                      torch.tensor(start, dtype=torch.int32, device=dev), kd,
                      vd, cu_seqlens=torch.from_numpy(cu).to(dev),
                      table_wrap=wrap)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_config4_full_append(tm, dev):
    """BASELINE config 4's KV-cache write at full size (8 runs, 21,970
    tokens from position 0 through a shuffled table, pool = 2x the pages),
    as bench.py times it; the whole pool compared bit-exact."""
    from importlib import import_module
    wl = import_module("tm-opt_amd.workloads")
    c = wl.config4(window=0)
    T, H, D = c.k.shape
    assert T == sum(c.lens) and len(c.lens) == 8
    g = torch.Generator().manual_seed(c.meta["seed"])
    table, P = wl.paged_layout(c.lens, g)
    kp = torch.zeros((P, 16, H, D), dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    cu = c.cu_seqlens.numpy()
    start = np.zeros(len(c.lens), dtype=np.int32)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(c.k),
                                cu, start, table.numpy())
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(c.v),
                                cu, start, table.numpy())
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(c.k.to(dev), c.v.to(dev), table.to(dev),
                      torch.from_numpy(start).to(dev), kd, vd,
                      cu_seqlens=c.cu_seqlens.to(dev),
                      max_seqlen=max(c.lens))
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_write_paged_row_width_bound(tm, dev):
    """A run whose positions reach past its table row: the tokens of pages
    beyond the row's width are skipped, and the next row's pages (which a
    read past the row would find) stay untouched."""
    g = torch.Generator().manual_seed(51)
    H, D, P = 4, 128, 16
    k = _bf16((40, H, D), g)
    v = _bf16((40, H, D), g)
    table = torch.tensor([[3, 9], [5, 12]], dtype=torch.int32)  # 2 pages/row
    cu = np.array([0, 40], dtype=np.int32)      # run 0: positions 0..39
    start = np.array([0], dtype=np.int32)
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu, start, table.numpy())
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                cu, start, table.numpy())
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(k.to(dev), v.to(dev), table.to(dev),
                      torch.from_numpy(start).to(dev), kd, vd,
                      cu_seqlens=torch.from_numpy(cu).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)
    # positions 32..39 (logical page 2) were skipped: pages 5 and 12 intact
    assert torch.equal(kd[5].cpu(), kp[5]) and torch.equal(kd[12].cpu(),
                                                          kp[12])


def _channel_major(rows, T_pad=None):
    """A [T, H, D] tensor with the same values laid out channel-major:
    tokens contiguous, head_dim strided (T_pad >= T tokens per dim row)."""
    T, H, D = rows.shape
    T_pad = T_pad or T
    buf = torch.zeros((H, D, T_pad), dtype=rows.dtype, device=rows.device)
    buf[:, :, :T] = rows.permute(1, 2, 0)
    return buf.permute(2, 0, 1)[:T]            # [T, H, D], strides (1, D*Tp, Tp)


@pytest.mark.parametrize("wrap", [0, 5])
def test_write_paged_channel_major_packed(tm, dev, wrap):
    """Channel-major K/V (tokens contiguous, head_dim strided) read in place:
    runs starting off the 8-token grid, a run ending at the tensor's last
    row, a ring table with RingKV's drop rule; bit-exact against the
    token-major rows' append."""
    g = torch.Generator().manual_seed(55 + wrap)
    H, D = 4, 128
    lens = [5, 133, 64, 1, 70, 199]           # 472 tokens: a multiple of 8
    start = [0, 7, 100, 3, 20, 61]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    k = _bf16((T, H, D), g)
    v = _bf16((T, H, D), g)
    per = [wrap if wrap else (s + n + 15) // 16 for s, n in zip(start, lens)]
    width = max(per)
    P = sum(per) + 2
    perm = torch.randperm(P, generator=g).to(torch.int32)
    table = torch.full((len(lens), width), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(per):
        table[i, :n] = perm[off:off + n]
        off += n
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(k),
                                cu, start, table.numpy(), 16, wrap)
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(v),
                                cu, start, table.numpy(), 16, wrap)
    # K tight (the last run ends at the tensor's last element), V with dim
    # rows padded past the tokens
    kc = _channel_major(k.to(dev))
    vc = _channel_major(v.to(dev), T_pad=T + 24)
    assert kc.stride() == (1, D * T, T) and vc.stride(0) == 1
    kd, vd = kp.to(dev), vp.to(dev)
    tm.kv_write_paged(kc, vc, table.to(dev),
                      torch.tensor(start, dtype=torch.int32, device=dev), kd,
                      vd, cu_seqlens=torch.from_numpy(cu).to(dev),
                      table_wrap=wrap)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


def test_write_paged_channel_major_engine_views(tm, dev):
    """The reference prefill's own append (model.py:507-512): the sconv
    hands K/V over channel-major, [B, T, C] with stride 1 along T, viewed
    as [B, T, HK, D]; each sequence appends kn[i, :len_i] (a strided view)
    through its own table. Every call reads the view in place."""
    g = torch.Generator().manual_seed(57)
    B, T, HK, D = 3, 96, 8, 128
    lens = [96, 37, 1]
    C = HK * D
    kc = _bf16((B, C, T), g)                   # channel-major storage
    vc = _bf16((B, C, T), g)
    kn = kc.transpose(1, 2).view(B, T, HK, D)  # strides (C*T, 1, D*T, T)
    vn = vc.transpose(1, 2).view(B, T, HK, D)
    P = 40
    perm = torch.randperm(P, generator=g).to(torch.int32)
    tables = perm[:B * 8].view(B, 8)
    kp = _bf16((P, 16, HK, D), g)
    vp = _bf16((P, 16, HK, D), g)
    want_k = kv_ref.as_u16(kp).copy()
    want_v = kv_ref.as_u16(vp).copy()
    kd, vd = kp.to(dev), vp.to(dev)
    knd = kc.to(dev).transpose(1, 2).view(B, T, HK, D)
    vnd = vc.to(dev).transpose(1, 2).view(B, T, HK, D)
    for i, n in enumerate(lens):
        kv_ref.write_paged(want_k, kv_ref.as_u16(kn[i, :n].contiguous()),
                           [0, n], [0], tables[i:i + 1].numpy())
        kv_ref.write_paged(want_v, kv_ref.as_u16(vn[i, :n].contiguous()),
                           [0, n], [0], tables[i:i + 1].numpy())
        assert knd[i, :n].stride() == (1, D * T, T)
        tm.kv_write_paged(knd[i, :n], vnd[i, :n],
                          tables[i:i + 1].to(dev).contiguous(),
                          torch.zeros(1, dtype=torch.int32, device=dev), kd,
                          vd, cu_seqlens=torch.tensor([0, n],
                                                      dtype=torch.int32,
                                                      device=dev))
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kd), want_k)
    assert np.array_equal(kv_ref.as_u16(vd), want_v)


@pytest.mark.parametrize("layout", ["token", "channel"])
@pytest.mark.parametrize("wrap", [0, 5])
def test_append_rows_batch(tm, dev, layout, wrap):
    """tmopt_kv_append_rows: B rows of a padded [B, T, H, D] batch (the
    prefill's st.cache.append(kn[i, :lens[i]], ...) loop, model.py:507-512)
    in one launch: ragged lengths including 0 and the full T, starts off the
    page grid, token-major and channel-major sources, a ring table with
    RingKV's drop rule; bit-exact against the oracle's per-row appends."""
    g = torch.Generator().manual_seed(61 + wrap)
    B, T, H, D = 5, 136, 4, 128
    lens = [136, 0, 57, 1, 100]
    start = [0, 5, 19, 200, 33]
    k = _bf16((B, T, H, D), g)
    v = _bf16((B, T, H, D), g)
    per = [wrap if wrap else (s + n + 15) // 16 + 1 for s, n in zip(start, lens)]
    width = max(per)
    P = sum(per) + 2
    perm = torch.randperm(P, generator=g).to(torch.int32)
    table = torch.full((B, width), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(per):
        table[i, :n] = perm[off:off + n]
        off += n
    kp = _bf16((P, 16, H, D), g)
    vp = _bf16((P, 16, H, D), g)
    # the oracle: the rows' first lens[i] tokens as packed runs
    rows_k = torch.cat([k[i, :lens[i]] for i in range(B)])
    rows_v = torch.cat([v[i, :lens[i]] for i in range(B)])
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want_k = kv_ref.write_paged(kv_ref.as_u16(kp).copy(), kv_ref.as_u16(rows_k),
                                cu, start, table.numpy(), 16, wrap)
    want_v = kv_ref.write_paged(kv_ref.as_u16(vp).copy(), kv_ref.as_u16(rows_v),
                                cu, start, table.numpy(), 16, wrap)
    if layout == "token":
        kd, vd = k.to(dev), v.to(dev)
    else:
        # channel-major per row: [B, H, D, T] storage viewed as [B, T, H, D]
        kd = k.permute(0, 2, 3, 1).contiguous().to(dev).permute(0, 3, 1, 2)
        vd = v.permute(0, 2, 3, 1).contiguous().to(dev).permute(0, 3, 1, 2)
        assert kd.stride(1) == 1 and kd.stride(3) == T
    kpd, vpd = kp.to(dev), vp.to(dev)
    tm.kv_append_rows(kd, vd, torch.tensor(lens, dtype=torch.int32,
                                           device=dev),
                      torch.tensor(start, dtype=torch.int32, device=dev),
                      table.to(dev), kpd, vpd, table_wrap=wrap)
    torch.cuda.synchronize()
    assert np.array_equal(kv_ref.as_u16(kpd), want_k)
    assert np.array_equal(kv_ref.as_u16(vpd), want_v)
