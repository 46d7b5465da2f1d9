"""Generate tests/golden/attn_small.json: tiny paged-decode, varlen-prefill
and KV-write cases with expected outputs computed by plain Python loops
(math.exp, no torch, no numpy, no code shared with oracle/).

Inputs are multiples of 1/8 in [-2, 2], exactly representable in bf16, so a
bf16 implementation sees the same values the fp64 brute force uses. They are
stored as base64 int8 (value * 8) with their shape; outputs as base64 fp32.
The reference has no numeric fixtures for this path (its activation dump is
absent), so these vectors pin the restated algorithm, not reference bits:
decode follows engine/pyengine/kernels/attn_swa.py:57-117, prefill
attn_prefill.py:80-141, the KV write model.py:938-948 / kv.py:193-205.

Run: python tests/golden/make_golden.py  (rewrites the JSON)
"""
import base64
import json
import math
import os
import random
import struct

PAGE = 16
HERE = os.path.dirname(os.path.abspath(__file__))


def q8(rng):
    return rng.randint(-16, 16) / 8.0


def tensor(rng, *shape):
    if len(shape) == 1:
        return [q8(rng) for _ in range(shape[0])]
    return [tensor(rng, *shape[1:]) for _ in range(shape[0])]


def attend(qv, keys, vals, scale, bias=None):
    """softmax(scale * q.k + bias) . V in fp64; returns (out, lse)."""
    s = []
    for j, kv in enumerate(keys):
        x = scale * sum(a * b for a, b in zip(qv, kv))
        if bias is not None:
            x += bias[j]
        s.append(x)
    m = max(s)
    e = [math.exp(x - m) for x in s]
    tot = sum(e)
    out = [sum(e[j] * vals[j][d] for j in range(len(vals))) / tot
           for d in range(len(vals[0]))]
    return out, m + math.log(tot)


def decode_case(rng, name, ctx, HQ, HKV, D, window, wrap=0, rel_extent=0):
    B = len(ctx)
    rep = HQ // HKV
    n_log = [(n + PAGE - 1) // PAGE for n in ctx]
    width = wrap if wrap else max(n_log)
    P = sum(wrap if wrap else n for n in n_log) + 3
    ids = list(range(P))
    rng.shuffle(ids)
    table, off = [], 0
    for b in range(B):
        cnt = wrap if wrap else n_log[b]
        row = ids[off:off + cnt] + [-1] * (width - cnt)
        off += cnt
        table.append(row)
    k_pool = tensor(rng, P, PAGE, HKV, D)
    v_pool = tensor(rng, P, PAGE, HKV, D)
    q = tensor(rng, B, HQ, D)
    rel = tensor(rng, B, HQ, rel_extent) if rel_extent else None
    scale = 1.0 / math.sqrt(D)
    out, lse = [], []
    for b in range(B):
        n = ctx[b]
        lo = max(0, n - window) if window else 0
        ob, lb = [], []
        for h in range(HQ):
            kh = h // rep
            keys, vals, bias = [], [], []
            for p in range(lo, n):
                lp = p // PAGE
                if wrap:
                    lp %= wrap
                pg = table[b][lp]
                keys.append(k_pool[pg][p % PAGE][kh])
                vals.append(v_pool[pg][p % PAGE][kh])
                dist = n - 1 - p
                bias.append(rel[b][h][dist] if rel and dist < rel_extent
                            else 0.0)
            o, l = attend(q[b][h], keys, vals, scale, bias if rel else None)
            ob.append(o)
            lb.append(l)
        out.append(ob)
        lse.append(lb)
    return {"name": name, "kind": "decode", "ctx": ctx, "HQ": HQ,
            "HKV": HKV, "D": D, "window": window, "table_wrap": wrap,
            "scale": scale, "block_table": table, "k_pool": k_pool,
            "v_pool": v_pool, "q": q, "rel": rel, "out": out, "lse": lse}


def prefill_case(rng, name, lens, HQ, HKV, D, window):
    rep = HQ // HKV
    total = sum(lens)
    q = tensor(rng, total, HQ, D)
    k = tensor(rng, total, HKV, D)
    v = tensor(rng, total, HKV, D)
    cu = [0]
    for t in lens:
        cu.append(cu[-1] + t)
    scale = 0.25
    out = [[None] * HQ for _ in range(total)]
    lse = [[None] * total for _ in range(HQ)]
    for i, T in enumerate(lens):
        t0 = cu[i]
        for j in range(T):
            lo = max(0, j - window + 1) if window else 0
            for h in range(HQ):
                kh = h // rep
                keys = [k[t0 + x][kh] for x in range(lo, j + 1)]
                vals = [v[t0 + x][kh] for x in range(lo, j + 1)]
                o, l = attend(q[t0 + j][h], keys, vals, scale)
                out[t0 + j][h] = o
                lse[h][t0 + j] = l
    return {"name": name, "kind": "prefill", "lens": lens, "cu": cu,
            "HQ": HQ, "HKV": HKV, "D": D, "window": window, "scale": scale,
            "q": q, "k": k, "v": v, "out": out, "lse": lse}


def prefill_paged_case(rng, name, prior, lens, HQ, HKV, D, window, wrap=0):
    """Chunked prefill: run i's queries sit at positions prior[i] + j and
    see keys 0 .. prior[i] + j. Keys before prior[i] live in a shuffled
    page pool through a block table (a ring of `wrap` pages holding the
    last 16 * wrap positions when wrap > 0, as RingKV keeps them); the
    run's own keys are the packed k / v rows. Without a ring the pool also
    holds the run's own keys (the same values), so the case serves the
    all-paged source as well."""
    rep = HQ // HKV
    total = sum(lens)
    cu = [0]
    for t in lens:
        cu.append(cu[-1] + t)
    q = tensor(rng, total, HQ, D)
    k = tensor(rng, total, HKV, D)
    v = tensor(rng, total, HKV, D)
    S = len(lens)
    n_pages = [wrap if wrap else (prior[i] + lens[i] + PAGE - 1) // PAGE
               for i in range(S)]
    width = max(n_pages)
    P = sum(n_pages) + 2
    ids = list(range(P))
    rng.shuffle(ids)
    table, off = [], 0
    for i in range(S):
        row = ids[off:off + n_pages[i]] + [-1] * (width - n_pages[i])
        off += n_pages[i]
        table.append(row)
    k_pool = tensor(rng, P, PAGE, HKV, D)
    v_pool = tensor(rng, P, PAGE, HKV, D)

    def row_of(i, p):
        lp = p // PAGE
        if wrap:
            lp %= wrap
        return table[i][lp], p % PAGE

    # the pool's content: prior keys (random), plus the run's own keys when
    # the table is not a ring (then the paged source reads them there)
    pk = {}
    for i in range(S):
        last = prior[i] if wrap else prior[i] + lens[i]
        first = max(0, prior[i] - wrap * PAGE) if wrap else 0
        for p in range(first, last):
            pg, o = row_of(i, p)
            if p >= prior[i]:
                kv = (k[cu[i] + p - prior[i]], v[cu[i] + p - prior[i]])
            else:
                kv = (tensor(rng, HKV, D), tensor(rng, HKV, D))
            k_pool[pg][o], v_pool[pg][o] = kv
            pk[(i, p)] = kv
    scale = 0.125
    out = [[None] * HQ for _ in range(total)]
    lse = [[None] * total for _ in range(HQ)]
    for i, T in enumerate(lens):
        for j in range(T):
            pos = prior[i] + j
            lo = max(0, pos - window + 1) if window else 0
            for h in range(HQ):
                kh = h // rep
                keys, vals = [], []
                for p in range(lo, pos + 1):
                    if p < prior[i]:
                        kv = pk[(i, p)]
                    else:
                        kv = (k[cu[i] + p - prior[i]], v[cu[i] + p - prior[i]])
                    keys.append(kv[0][kh])
                    vals.append(kv[1][kh])
                o, l = attend(q[cu[i] + j][h], keys, vals, scale)
                out[cu[i] + j][h] = o
                lse[h][cu[i] + j] = l
    return {"name": name, "kind": "prefill_paged", "lens": lens,
            "prior": prior, "cu": cu, "HQ": HQ, "HKV": HKV, "D": D,
            "window": window, "table_wrap": wrap, "scale": scale,
            "block_table": table, "k_pool": k_pool, "v_pool": v_pool,
            "q": q, "k": k, "v": v, "out": out, "lse": lse}


def kv_write_case(rng, name):
    """Paged append of three runs (start positions 0, 5, 30; lengths 7, 20,
    3) through a shuffled table; expected pool after the write."""
    H, D, P = 2, 8, 12
    lens, start = [7, 20, 3], [0, 5, 30]
    cu = [0, 7, 27, 30]
    ids = list(range(P))
    rng.shuffle(ids)
    table = [ids[0:2] + [-1, -1], ids[2:4] + [-1, -1], ids[4:7] + [-1]]
    k = tensor(rng, 30, H, D)
    pool = tensor(rng, P, PAGE, H, D)
    want = json.loads(json.dumps(pool))
    for i in range(3):
        for t in range(lens[i]):
            p = start[i] + t
            pg = table[i][p // PAGE]
            want[pg][p % PAGE] = k[cu[i] + t]
    return {"name": name, "kind": "kv_write", "cu": cu, "start": start,
            "block_table": table, "k": k, "pool": pool, "want": want}


def _flat(x):
    if isinstance(x, list):
        out = []
        for e in x:
            out.extend(_flat(e))
        return out
    return [x]


def _shape(x):
    sh = []
    while isinstance(x, list):
        sh.append(len(x))
        x = x[0] if x else None
    return sh


def pack(x):
    """nested list of multiples of 1/8 -> {"shape", "q8"} (base64 int8)."""
    vals = bytes((int(round(v * 8)) & 0xff) for v in _flat(x))
    return {"shape": _shape(x), "q8": base64.b64encode(vals).decode()}


def pack_f32(x):
    """nested list of floats -> {"shape", "f32"} (base64 little-endian)."""
    vals = _flat(x)
    return {"shape": _shape(x),
            "f32": base64.b64encode(struct.pack(f"<{len(vals)}f",
                                                *vals)).decode()}


INPUTS = ("q", "k", "v", "k_pool", "v_pool", "rel", "pool", "want")
OUTPUTS = ("out", "lse")


def main():
    rng = random.Random(20261201)
    cases = [
        decode_case(rng, "decode_global_gqa8", [1, 5, 16, 17, 40], 16, 2,
                    128, 0),
        decode_case(rng, "decode_window7", [3, 7, 8, 30, 47], 8, 2, 128, 7),
        decode_case(rng, "decode_ring_rel", [1, 20, 33, 50], 4, 1, 128, 32,
                    wrap=2, rel_extent=32),
        prefill_case(rng, "prefill_causal", [1, 4, 9, 40], 8, 1, 128, 0),
        prefill_case(rng, "prefill_window3", [6, 10], 4, 1, 128, 3),
        kv_write_case(rng, "kv_write_paged"),
    ]
    # a generator of its own, so the cases above keep their values
    rng2 = random.Random(20261202)
    cases += [
        prefill_paged_case(rng2, "prefill_paged_prior", [0, 5, 16, 40],
                           [3, 17, 1, 33], 8, 2, 128, 0),
        prefill_paged_case(rng2, "prefill_ring_window20", [10, 50, 33],
                           [5, 40, 2], 8, 2, 128, 20, wrap=2),
    ]
    for c in cases:
        for key in INPUTS:
            if c.get(key) is not None:
                c[key] = pack(c[key])
        for key in OUTPUTS:
            if c.get(key) is not None:
                c[key] = pack_f32(c[key])
    path = os.path.join(HERE, "attn_small.json")
    with open(path, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py",
                   "page_size": PAGE, "cases": cases}, f)
    print(path)


if __name__ == "__main__":
    main()
