"""numpy oracle of the KV-cache write and block-table gather (TEST
INFRASTRUCTURE ONLY — see oracle/__init__.py).

Pure index arithmetic and byte copies on uint16 views of bf16 data, so every
comparison is bit-exact.
"""
import numpy as np

PAGE = 16


def as_u16(t):
    """bf16 torch tensor -> uint16 numpy array with the same bits."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(
        np.uint16)


def write_slots(pool, rows, slots):
    """pool.view(-1, H, D)[slots] = rows for slots >= 0 and < pool rows, in
    token order (engine/pyengine/model.py:941-942; kv.py:203-204). pool is
    any [..., H, D] array; it is modified in place and returned."""
    H, D = rows.shape[1], rows.shape[2]
    flat = pool.reshape(-1, H, D)
    for t, s in enumerate(np.asarray(slots).tolist()):
        if 0 <= s < flat.shape[0]:
            flat[s] = rows[t]
    return pool


def flat_slots(table_row, positions, page=PAGE, table_wrap=0):
    """Logical positions -> flat pool rows through one table row:
    table[p // page] * page + p % page (PagedKV._flat_slots,
    engine/pyengine/kv.py:161-168); with a ring of table_wrap pages the
    logical page is taken modulo table_wrap (RingKV slot p % W,
    kv.py:99-100)."""
    positions = np.asarray(positions, dtype=np.int64)
    lp = positions // page
    if table_wrap:
        lp = lp % table_wrap
    return np.asarray(table_row, dtype=np.int64)[lp] * page + positions % page


def write_paged(pool, rows, cu_seqlens, start_pos, block_table, page=PAGE,
                table_wrap=0):
    """Append runs through a block table. Run i's token t sits at position
    start_pos[i] + t. With a ring table only the last table_wrap * page
    positions of a run can survive; earlier ones are dropped as
    RingKV.append drops them (engine/pyengine/kv.py:94-98). Entries outside
    the pool are skipped, and so are tokens whose logical page lies past the
    table row's width (the reference's tables always cover the appended
    positions, PagedKV.ensure_pages kv.py:170-191; the native write treats
    a too-short row as absent entries). cu_seqlens None = one token per
    run."""
    H, D = rows.shape[1], rows.shape[2]
    flat = pool.reshape(-1, H, D)
    n_pages = flat.shape[0] // page
    S = len(start_pos)
    for i in range(S):
        if cu_seqlens is None:
            t0, t1 = i, i + 1
        else:
            t0, t1 = int(cu_seqlens[i]), int(cu_seqlens[i + 1])
        T = t1 - t0
        p0 = int(start_pos[i])
        keep_from = p0 + T - table_wrap * page if table_wrap else p0
        for t in range(T):
            p = p0 + t
            if p < keep_from or p < 0:
                continue
            lp = p // page
            if table_wrap:
                lp %= table_wrap
            if lp >= len(block_table[i]):
                continue
            pg = int(block_table[i][lp])
            if not 0 <= pg < n_pages:
                continue
            flat[pg * page + p % page] = rows[t0 + t]
    return pool


def gather(pool, table_row, n, page=PAGE, table_wrap=0, lo=0):
    """Rows of positions lo..n-1 in logical order (PagedKV.gather,
    kv.py:207-212; RingKV.gather keeps the last W, kv.py:105-114)."""
    H, D = pool.shape[-2], pool.shape[-1]
    flat = pool.reshape(-1, H, D)
    return flat[flat_slots(table_row, np.arange(lo, n), page, table_wrap)]
