"""Seeded synthetic inputs for the five configurations of BASELINE.json,
plus the algorithmic-work counters the roofline figures divide by.

Seeds: one torch.Generator per configuration, seeded 20261201 + index
(C1..C5 -> 1..5). Draw order: lengths, then the block-table permutation,
then Q, K, V, each N(0, 1) in fp32 rounded to bf16.

Pool layout is the reference's GlobalPool page pool [P, 16, HKV, D]
(engine/pyengine/kv.py:248-268): a shuffled pool of twice the needed pages,
so physical placement is scattered like a long-running server's free list
(kv.py:139-142, t_b3.py:119-130). Pages that no sequence owns are filled
with NaN in correctness runs ("poison"), so any read of them poisons the
output; timing runs fill them with zeros.
"""
import math
from dataclasses import dataclass, field

import torch

PAGE = 16
HQ, HKV, D = 32, 4, 128
SCALE = 1.0 / math.sqrt(D)
SEED0 = 20261201


def generator(index, device="cpu"):
    g = torch.Generator(device=device)
    g.manual_seed(SEED0 + index)
    return g


def _randn_bf16(shape, g, device):
    return torch.randn(shape, generator=g, dtype=torch.float32,
                       device=device).to(torch.bfloat16)


@dataclass
class DecodeCase:
    name: str
    q: torch.Tensor            # [B, HQ, D] bf16
    k_pool: torch.Tensor       # [P, 16, HKV, D] bf16
    v_pool: torch.Tensor
    block_table: torch.Tensor  # [B, max_pages] int32 (-1 = unassigned)
    ctx_lens: torch.Tensor     # [B] int32
    window: int = 0
    scale: float = SCALE
    meta: dict = field(default_factory=dict)

    @property
    def B(self):
        return self.q.shape[0]

    def visible(self):
        n = self.ctx_lens.to(torch.int64).cpu()
        return torch.minimum(n, torch.tensor(self.window)) if self.window \
            else n

    def algorithmic_bytes(self):
        """Decode bytes as the roofline counts them: visible K+V rows, Q, O,
        LSE, the block-table entries of visible pages and ctx_lens. Split
        partials and partial-page over-read are overhead, not counted."""
        B, hq, d = self.q.shape
        hkv = self.k_pool.shape[2]
        nv = self.visible()
        kv = int(nv.sum()) * hkv * d * 2 * 2
        qo = B * hq * d * 2 * 2
        lse = B * hq * 4
        table = int(((nv + PAGE - 1) // PAGE).sum()) * 4
        return kv + qo + lse + table + B * 4

    def to(self, device):
        return DecodeCase(self.name, self.q.to(device),
                          self.k_pool.to(device), self.v_pool.to(device),
                          self.block_table.to(device),
                          self.ctx_lens.to(device), self.window, self.scale,
                          dict(self.meta))


def decode_lens(index, B, lo, hi, g=None):
    """The context lengths of a seeded decode config: the first draw of its
    generator, U{lo..hi} (make_decode's order: lengths, table, Q, K, V)."""
    g = generator(index, "cpu") if g is None else g
    return torch.randint(lo, hi + 1, (B,), generator=g)


def make_decode(name, index, B, lo, hi, window=0, device="cpu",
                poison=True, hq=HQ, hkv=HKV, ctx=None, pool_factor=2):
    """Paged decode batch: ctx ~ U{lo..hi} (or the given list), pages of the
    visible range backed by distinct random pages of a shuffled pool of
    pool_factor x the backed pages; logical pages before a window's first
    page point at one NaN poison page (never to be read)."""
    g = generator(index, "cpu")
    if ctx is None:
        ctx = decode_lens(index, B, lo, hi, g)
    else:
        ctx = torch.as_tensor(ctx, dtype=torch.int64)
    n_log = (ctx + PAGE - 1) // PAGE                 # logical pages
    if window:
        first = torch.clamp(ctx - window, min=0) // PAGE
    else:
        first = torch.zeros_like(ctx)
    n_back = n_log - first                           # backed pages
    need = int(n_back.sum())
    P = pool_factor * need + 1                       # + poison page
    perm = torch.randperm(P - 1, generator=g)
    poison_page = P - 1
    max_pages = int(n_log.max())
    table = torch.full((B, max_pages), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        nb = int(n_back[b])
        f = int(first[b])
        table[b, :f] = poison_page
        table[b, f:f + nb] = perm[off:off + nb].to(torch.int32)
        off += nb
    gd = generator(index, device) if device != "cpu" else g
    q = _randn_bf16((B, hq, D), gd, device)
    fill = float("nan") if poison else 0.0
    k_pool = torch.full((P, PAGE, hkv, D), fill, dtype=torch.bfloat16,
                        device=device)
    v_pool = torch.full_like(k_pool, fill)
    used = perm[:need].to(device)
    k_pool[used] = _randn_bf16((need, PAGE, hkv, D), gd, device)
    v_pool[used] = _randn_bf16((need, PAGE, hkv, D), gd, device)
    return DecodeCase(name, q, k_pool, v_pool, table.to(device),
                      ctx.to(torch.int32).to(device), window, SCALE,
                      {"seed": SEED0 + index, "pool_pages": P,
                       "backed_pages": need})


def config1(device="cpu", poison=True):
    """C1: global decode, B=4, ctx U[128,1024] (CPU-runnable)."""
    return make_decode("C1_global_decode_b4", 1, 4, 128, 1024, 0, device,
                       poison)


def config2(device="cpu", poison=True):
    """C2: global decode, B=64, ctx U[1024,8192]."""
    return make_decode("C2_global_decode_b64", 2, 64, 1024, 8192, 0, device,
                       poison)


def config3(device="cpu", poison=True):
    """C3: window-4096 decode, B=128, ctx U[2048,32768]."""
    return make_decode("C3_swa4096_decode_b128", 3, 128, 2048, 32768, 4096,
                       device, poison)


# --------------------------------------------------------------------------
# prefill
# --------------------------------------------------------------------------

@dataclass
class PrefillCase:
    name: str
    q: torch.Tensor           # [total, HQ, D]
    k: torch.Tensor           # [total, HKV, D]
    v: torch.Tensor
    cu_seqlens: torch.Tensor  # [S+1] int32
    window: int = 0
    scale: float = SCALE
    meta: dict = field(default_factory=dict)

    @property
    def lens(self):
        c = self.cu_seqlens.to(torch.int64).cpu()
        return (c[1:] - c[:-1]).tolist()

    def visible_pairs(self, window=None, prior=None):
        w = self.window if window is None else window
        return visible_pairs(self.lens, w, prior)

    def algorithmic_flops(self):
        hq, d = self.q.shape[1], self.q.shape[2]
        return 4 * d * hq * self.visible_pairs()


def visible_pairs(lens, window=0, prior=None):
    """Exact count of (query, key) pairs that the causal/window mask keeps:
    query j of a run with p prior tokens sits at p + j and sees
    min(p + j + 1, W) keys (all p + j + 1 when W == 0)."""
    tot = 0
    for i, T in enumerate(lens):
        p = 0 if prior is None else int(prior[i])
        a, b = p + 1, p + T   # visible counts without window: a..b
        if window and b > window:
            full_from = max(a, window)
            n_full = b - full_from + 1
            tri_hi = min(b, window - 1)
            tri = (tri_hi * (tri_hi + 1) // 2 - (a - 1) * a // 2) \
                if tri_hi >= a else 0
            tot += tri + n_full * window
        else:
            tot += b * (b + 1) // 2 - (a - 1) * a // 2
    return tot


def make_prefill(name, index, lens=None, n_seqs=8, lo=512, hi=8192,
                 window=0, device="cpu", hq=HQ, hkv=HKV):
    g = generator(index, "cpu")
    if lens is None:
        lens = torch.randint(lo, hi + 1, (n_seqs,), generator=g).tolist()
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(
        torch.int32)
    total = int(cu[-1])
    _ = torch.randperm(8, generator=g)   # keeps the draw order of the plan
    gd = generator(index, device) if device != "cpu" else g
    q = _randn_bf16((total, hq, D), gd, device)
    k = _randn_bf16((total, hkv, D), gd, device)
    v = _randn_bf16((total, hkv, D), gd, device)
    return PrefillCase(name, q, k, v, cu.to(device), window, SCALE,
                       {"seed": SEED0 + index, "lens": list(lens)})


def config4(window=0, device="cpu"):
    """C4: varlen causal prefill, 8 seqs, T ~ U[512, 8192]."""
    nm = "C4_prefill_global" if not window else f"C4_prefill_swa{window}"
    return make_prefill(nm, 4, window=window, device=device)


def config4_long(window=0, device="cpu"):
    """C4's head config on 4 runs of 8192 tokens: with window 4096, half of
    every run's queries see a full window (C4's own draws peak at 4,645
    tokens, so its window line differs from the global one by 0.4%)."""
    nm = "C4_long_global" if not window else f"C4_long_swa{window}"
    return make_prefill(nm, 4, lens=[8192] * 4, window=window, device=device)


def paged_layout(lens, g, pool_factor=2, prior=None):
    """Shuffled block table for runs of the given lengths (+prior tokens):
    returns (block_table [S, max_pages] int32, num_pages)."""
    tot = [int(t) + (0 if prior is None else int(prior[i]))
           for i, t in enumerate(lens)]
    npg = [(t + PAGE - 1) // PAGE for t in tot]
    need = sum(npg)
    P = pool_factor * need
    perm = torch.randperm(P, generator=g)
    table = torch.full((len(lens), max(npg)), -1, dtype=torch.int32)
    off = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    return table, P


# --------------------------------------------------------------------------
# config 5: mixed continuous-batching step over 66 layers
# --------------------------------------------------------------------------

@dataclass
class MixedStep:
    """One step of config 5 for every layer. Rows 0..n_chunks-1 of each
    layer's block table are the chunked-prefill runs, the rest the decode
    rows. Every layer has a pool set of its own (K and V pages of a global
    layer: every page of every row; of a window layer: the pages a query of
    the row can see) and a shuffled table over it, so no layer reads pages
    another layer has just brought into the 256 MB Infinity Cache: ~88 GB
    of pools in all."""
    n_layers: int
    window: int
    is_global: list             # per layer
    tables: list                # per layer [R, width] int32
    pools: list                 # per layer (k, v) [P_l, 16, HKV, D]
    chunk_lens: list
    chunk_prior: list
    dec_ctx: torch.Tensor       # [96] int32 (after this step's append)
    q_prefill: torch.Tensor     # [sum chunks, HQ, D]
    q_decode: torch.Tensor      # [96, HQ, D]
    k_new: torch.Tensor         # [sum chunks + 96, HKV, D]
    v_new: torch.Tensor
    cu_all: torch.Tensor        # [R + 1] int32 (chunks, then 1 per row)
    start_all: torch.Tensor     # [R] int32
    cu_chunks: torch.Tensor     # [n_chunks + 1] int32
    prior: torch.Tensor         # [n_chunks] int32
    scale: float = SCALE
    meta: dict = field(default_factory=dict)

    def pool(self, layer):
        """(k, v) page pools of one layer."""
        return self.pools[layer]

    def decode_bytes(self, layer):
        n = self.dec_ctx.to(torch.int64).cpu()
        if not self.is_global[layer]:
            n = torch.minimum(n, torch.tensor(self.window))
        B, hq, d = self.q_decode.shape
        hkv = self.pools[0][0].shape[2]
        return int(n.sum()) * hkv * d * 4 + B * hq * d * 4 + B * hq * 4 + \
            int(((n + PAGE - 1) // PAGE).sum()) * 4 + B * 4

    def prefill_flops(self, layer):
        w = 0 if self.is_global[layer] else self.window
        hq, d = self.q_prefill.shape[1], self.q_prefill.shape[2]
        return 4 * d * hq * visible_pairs(self.chunk_lens, w,
                                          self.chunk_prior)

    def kv_write_bytes(self):
        T = self.k_new.shape[0]
        hkv, d = self.k_new.shape[1], self.k_new.shape[2]
        return 2 * 2 * T * hkv * d * 2 + T * 8


def config5(device="cuda", n_layers=66, window=4096, n_decode=96,
            chunk=2048, prior=4096, n_chunks=2, lo=1024, hi=65536):
    g = generator(5, "cpu")
    u = torch.rand(n_decode, generator=g, dtype=torch.float64)
    ctx = torch.floor(torch.exp(math.log(lo) + u * (math.log(hi) -
                                                    math.log(lo)))).long()
    ctx = torch.clamp(ctx, lo, hi)
    chunk_tot = prior + chunk
    R = n_chunks + n_decode
    log_pages = [(chunk_tot + PAGE - 1) // PAGE] * n_chunks + \
        [int((c + PAGE - 1) // PAGE) for c in ctx]
    width = max(log_pages)
    # backed logical pages per row: global = all; window = pages that hold
    # a key some query of the row can see
    first_s = [0] * n_chunks + [int(max(0, int(c) - window) // PAGE)
                                for c in ctx]
    Pg = sum(log_pages) + 1
    Ps = sum(lp - f for lp, f in zip(log_pages, first_s)) + 1
    gd = generator(5, device) if device != "cpu" else g
    hkv = HKV

    def pool(P):
        k = _randn_bf16((P, PAGE, hkv, D), gd, device)
        v = _randn_bf16((P, PAGE, hkv, D), gd, device)
        return k, v

    is_global = [i % 4 == 3 for i in range(n_layers)]
    pools = [pool(Pg if is_global[i] else Ps) for i in range(n_layers)]
    tables = []
    for i in range(n_layers):
        P = Pg if is_global[i] else Ps
        perm = torch.randperm(P - 1, generator=g).to(torch.int32)
        t = torch.full((R, width), P - 1, dtype=torch.int32)  # poison page
        off = 0
        for r in range(R):
            f = 0 if is_global[i] else first_s[r]
            n = log_pages[r] - f
            t[r, f:f + n] = perm[off:off + n]
            off += n
        tables.append(t.to(device))
    T_new = n_chunks * chunk + n_decode
    cu_all = [0]
    for r in range(R):
        cu_all.append(cu_all[-1] + (chunk if r < n_chunks else 1))
    start_all = [prior] * n_chunks + [int(c) - 1 for c in ctx]
    ic = lambda x: torch.tensor(x, dtype=torch.int32, device=device)
    return MixedStep(
        n_layers=n_layers, window=window, is_global=is_global, tables=tables,
        pools=pools, chunk_lens=[chunk] * n_chunks,
        chunk_prior=[prior] * n_chunks, dec_ctx=ctx.to(torch.int32).to(device),
        q_prefill=_randn_bf16((n_chunks * chunk, HQ, D), gd, device),
        q_decode=_randn_bf16((n_decode, HQ, D), gd, device),
        k_new=_randn_bf16((T_new, hkv, D), gd, device),
        v_new=_randn_bf16((T_new, hkv, D), gd, device),
        cu_all=ic(cu_all), start_all=ic(start_all),
        cu_chunks=ic([i * chunk for i in range(n_chunks + 1)]),
        prior=ic([prior] * n_chunks),
        meta={"seed": SEED0 + 5, "global_pages": Pg, "swa_pages": Ps,
              "decode_ctx": ctx.tolist()})
