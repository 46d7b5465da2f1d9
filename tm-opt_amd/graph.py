"""hipGraph capture of the decode step's attention work.

The reference captures its whole pooled decode step per device segment with
CUDA graphs (engine/pyengine/graphrun.py:76-380): static input buffers, the
batch padded to max_batch with a scratch slot, and one capture per 512-token
bucket of the padded key length (graphrun.py:339-343) because its gather
indices are shaped by that length.

Here the attention part of a step is, per layer, one KV-cache append
(tmopt_kv_write_paged: the new token of every row goes to page
ctx/16 of its block table) and one paged decode (tmopt_attn_decode_paged).
Both read positions and lengths from device memory and launch grids that do
not depend on them (the decode grid is the persistent one), so ONE capture
serves every step for the lifetime of the buffers: no buckets, no
recapture. Nothing inside the captured region allocates, synchronises, or
issues a memset (workspaces are allocated before capture).

StepGraph captures any callable that works on static buffers (warm-up
twice on a side stream, then capture, as graphrun.py:260-301 does);
DecodeStepGraph builds the multi-layer decode-attention step on top of it.
"""
import torch

from . import attn


class StepGraph:
    """Capture `fn` (a callable touching only static device buffers)."""

    def __init__(self, fn, device=None):
        self.fn = fn
        self.device = torch.device(device or "cuda")
        self.graph = None
        self.pool = None
        self.stream = None

    def capture(self, warmup=2):
        with torch.cuda.device(self.device):
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(warmup):
                    self.fn()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            self.pool = torch.cuda.graph_pool_handle()
            self.stream = torch.cuda.Stream()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self.pool, stream=self.stream):
                self.fn()
            self.graph = g
        return self

    def replay(self):
        assert self.graph is not None, "capture() first"
        self.graph.replay()


class DecodeStepGraph:
    """Decode-step attention for a stack of layers, captured once.

    layers: list of dicts with k_pool, v_pool ([P, 16, HKV, D] bf16),
    block_table ([MB, width] int32, static), window (0 = global) and
    table_wrap (ring tables for sliding-window pools, 0 otherwise).
    Static inputs the host fills before each replay (outside the graph):
      q      [L, MB, HQ, D]  bf16   query of every row, per layer
      k_new  [L, MB, HKV, D] bf16   the step's new key / value rows
      v_new  [L, MB, HKV, D] bf16
      ctx    [MB] int32             keys after this step's append (pos + 1)
    Outputs after replay: out [L, MB, HQ, D] bf16, lse [L, MB, HQ] fp32.
    Rows without a live sequence should point at a scratch slot / page with
    ctx = 1, as the reference's dead rows do (kv.py:223-228)."""

    def __init__(self, layers, max_batch, HQ, HKV, D=attn.HEAD_DIM,
                 scale=None, device="cuda", min_pages=8, num_workgroups=0):
        self.layers = layers
        self.L = len(layers)
        self.MB, self.HQ, self.HKV, self.D = max_batch, HQ, HKV, D
        self.scale = scale if scale is not None else D ** -0.5
        dev = torch.device(device)
        bf = torch.bfloat16
        self.q = torch.zeros((self.L, max_batch, HQ, D), dtype=bf, device=dev)
        self.k_new = torch.zeros((self.L, max_batch, HKV, D), dtype=bf,
                                 device=dev)
        self.v_new = torch.zeros_like(self.k_new)
        self.ctx = torch.ones(max_batch, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(max_batch, dtype=torch.int32, device=dev)
        self.out = torch.zeros((self.L, max_batch, HQ, D), dtype=bf,
                               device=dev)
        self.lse = torch.zeros((self.L, max_batch, HQ), dtype=torch.float32,
                               device=dev)
        # one workspace serves every layer: the layers run in stream order
        self.workspace = attn.decode_workspace(max_batch, HQ, HKV, dev,
                                               num_workgroups)
        self.min_pages = min_pages
        self.num_workgroups = num_workgroups
        self.graph = StepGraph(self._step, dev)

    def _step(self):
        torch.sub(self.ctx, 1, out=self.pos)
        for l, ly in enumerate(self.layers):
            attn.kv_write_paged(self.k_new[l], self.v_new[l],
                                ly["block_table"], self.pos, ly["k_pool"],
                                ly["v_pool"],
                                table_wrap=ly.get("table_wrap", 0))
            attn.decode_paged(self.q[l], ly["k_pool"], ly["v_pool"],
                              ly["block_table"], self.ctx, self.scale,
                              window=ly.get("window", 0),
                              table_wrap=ly.get("table_wrap", 0),
                              min_pages=self.min_pages,
                              num_workgroups=self.num_workgroups,
                              out=self.out[l], lse=self.lse[l],
                              workspace=self.workspace)

    def run_eager(self):
        self._step()

    def capture(self):
        self.graph.capture()
        return self

    def replay(self):
        self.graph.replay()


class MixedStepGraph:
    """Config-5 step: for every layer, append the step's tokens (chunked
    prefill runs + one token per decode row) through the layer's block
    table, then run the paged chunked prefill and the paged decode. All
    three kernels per layer are captured into ONE hipGraph for the whole
    step.

    With overlap=True the decode of a layer runs on a second stream, forked
    after the append and joined before the next layer: the HBM-bound decode
    and the MFMA-bound prefill then share the GPU instead of taking turns
    (in the graph they are two independent nodes between the append and
    the next layer). The decode's persistent work-groups hold their compute
    units for the whole decode, and a prefill work-group needs a whole
    compute unit's registers, so the decode's grid decides how the two
    share the chip. By default a global layer's decode (the longer one)
    takes two thirds of its stand-alone size (half the compute units) and a
    window layer's its stand-alone size (it is done in about half the time
    of that layer's prefill and then leaves the prefill every unit).
    Measured on config 5 (one box, four alternating runs each): 31.4-31.6
    ms per step, against 31.8-32.8 ms with two thirds for both kinds; with
    two thirds for both on another box 30.6 ms, against 31.4 ms with the
    stand-alone grid for both and 31.7 ms without the second stream.
    num_workgroups > 0 sets one grid for both kinds."""

    def __init__(self, step, min_pages=8, num_workgroups=0, overlap=True):
        self.s = step
        dev = step.q_decode.device
        B, HQ, D = step.q_decode.shape
        HKV = step.pools[0][0].shape[2]
        full = attn.decode_default_workgroups(HKV)
        if num_workgroups > 0:
            self.wgs = {True: num_workgroups, False: num_workgroups}
        elif overlap:
            self.wgs = {True: max(1, full * 2 // 3), False: full}
        else:
            self.wgs = {True: full, False: full}
        self.n_chunks = len(step.chunk_lens)
        self.max_chunk = max(step.chunk_lens)
        self.out_p = torch.empty_like(step.q_prefill)
        self.out_d = torch.empty_like(step.q_decode)
        self.lse_d = torch.empty((B, HQ), dtype=torch.float32, device=dev)
        self.ws = attn.decode_workspace(B, HQ, HKV, dev,
                                        max(self.wgs.values()))
        self.min_pages = min_pages
        self.overlap = overlap
        self.side = torch.cuda.Stream(device=dev) if overlap else None
        self.graph = StepGraph(self.run_eager, dev)

    def layer(self, l, parts=("kv", "prefill", "decode")):
        s = self.s
        kp, vp = s.pool(l)
        w = 0 if s.is_global[l] else s.window
        t = s.tables[l]
        if "kv" in parts:
            attn.kv_write_paged(s.k_new, s.v_new, t, s.start_all, kp, vp,
                                cu_seqlens=s.cu_all,
                                max_seqlen=self.max_chunk)
        if "prefill" in parts:
            attn.prefill_varlen(s.q_prefill, None, None, s.cu_chunks,
                                s.scale, window=w, max_seqlen=self.max_chunk,
                                prior_lens=s.prior, k_pool=kp, v_pool=vp,
                                block_table=t[:self.n_chunks],
                                out=self.out_p, return_lse=False)
        if "decode" in parts:
            attn.decode_paged(s.q_decode, kp, vp, t[self.n_chunks:],
                              s.dec_ctx, s.scale, window=w,
                              min_pages=self.min_pages,
                              num_workgroups=self.wgs[s.is_global[l]],
                              out=self.out_d, lse=self.lse_d,
                              workspace=self.ws)

    def run_eager(self):
        if not self.overlap:
            for l in range(self.s.n_layers):
                self.layer(l)
            return
        main = torch.cuda.current_stream()
        for l in range(self.s.n_layers):
            self.layer(l, ("kv",))
            fork = torch.cuda.Event()
            fork.record(main)
            self.side.wait_event(fork)
            with torch.cuda.stream(self.side):
                self.layer(l, ("decode",))
            self.layer(l, ("prefill",))
            join = torch.cuda.Event()
            join.record(self.side)
            main.wait_event(join)

    def capture(self):
        self.graph.capture()
        return self

    def replay(self):
        self.graph.replay()


BUCKET = 512   # the reference's padded-key-length bucket (graphrun.py)


class AttnGraphRunner:
    """The attention part of the reference's graphed decode step, captured
    with GraphRunner's semantics (engine/pyengine/graphrun.py:76-380) around
    the reference-signature adapters (compat.attn_global / attn_swa):

      * static row buffers padded to max_batch: the host stages the live
        rows' positions and slots, dead rows get position 0 and the scratch
        slot max_batch (SwaPool's scratch row, GlobalPool's scratch page
        behind table_dev[max_batch], kv.py:223-228, :262-268);
      * per layer, the step's own index math as model.py:926-950 computes
        it (page gather of the new token's flat row, ring slot pos % W), the
        append (tmopt_kv_write_slots, the index_put_ of model.py:941-948),
        the padded per-token flat rows of the global gather at the bucket
        length L_pad (decode_batch_ctx_static, model.py:860-887) and the
        attention call (model.py:970-976);
      * one captured program per L_pad = ceil((max pos + 1) / 512) * 512,
        a monotone high-water mark capped at the table's reach, captured
        on first sight after two warm-ups under the dead-row config (so
        warm-ups touch only scratch state) and replayed for every step of
        that bucket (graphrun.py:260-301, :338-361).

    layers: dicts with kind "global" (kp, vp [(P+1), 16, HK, D], table_dev
    [max_batch+1, num_pages] i64) or "swa" (k, v [max_batch+1, W, HK, D]).
    Before step(): fill q[l] [MB, HQ, D], k_new[l] / v_new[l] [MB, HK, D],
    rel[l] [MB, HQ, E] for the live rows (dead rows are don't-care).
    After step(): out[l] [MB, HQ, D] (dead rows are don't-care)."""

    def __init__(self, layers, max_batch, HQ, D=attn.HEAD_DIM,
                 device="cuda"):
        self.layers = layers
        self.MB = max_batch
        self.scratch = max_batch
        dev = torch.device(device)
        self.device = dev
        bf = torch.bfloat16
        self.pos_buf = torch.zeros(max_batch, dtype=torch.int64, device=dev)
        self.slots_buf = torch.full((max_batch,), self.scratch,
                                    dtype=torch.int64, device=dev)
        self.q, self.k_new, self.v_new, self.rel, self.out = [], [], [], [], []
        reach = None
        for ly in layers:
            if ly["kind"] == "global":
                HK = ly["kp"].shape[2]
                E = ly.get("rel_extent", 1024)
                r = ly["table_dev"].shape[1] * ly["kp"].shape[1]
                reach = r if reach is None else min(reach, r)
            else:
                HK = ly["k"].shape[2]
                E = ly["k"].shape[1]
            self.q.append(torch.zeros((max_batch, HQ, D), dtype=bf,
                                      device=dev))
            self.k_new.append(torch.zeros((max_batch, HK, D), dtype=bf,
                                          device=dev))
            self.v_new.append(torch.zeros((max_batch, HK, D), dtype=bf,
                                          device=dev))
            self.rel.append(torch.zeros((max_batch, HQ, E), dtype=bf,
                                        device=dev))
            self.out.append(torch.zeros((max_batch, HQ, D), dtype=bf,
                                        device=dev))
        self.reach = reach
        self.programs = {}
        self.hiwater = 0
        self.captures = 0

    def _run(self, L_pad):
        from . import compat
        pos, slots = self.pos_buf, self.slots_buf
        n = pos + 1
        for l, ly in enumerate(self.layers):
            q, k, v, rel = self.q[l], self.k_new[l], self.v_new[l], self.rel[l]
            if ly["kind"] == "global":
                kp, vp, td = ly["kp"], ly["vp"], ly["table_dev"]
                ps = kp.shape[1]
                HK, D = kp.shape[2], kp.shape[3]
                table = td[slots]                              # [MB, pages]
                flat_new = (table.gather(1, (pos // ps)[:, None])[:, 0] * ps
                            + pos % ps)
                attn.kv_write_slots(k, v, flat_new, kp.view(-1, HK, D),
                                    vp.view(-1, HK, D))
                j = torch.arange(L_pad, device=pos.device)
                flat = table[:, j // ps] * ps + (j % ps)[None, :]
                flat = flat.masked_fill(j[None, :] >= n[:, None], 0)
                self.out[l].copy_(compat.attn_global(q, kp, vp, flat, pos,
                                                     rel, L_pad))
            else:
                pk, pv = ly["k"], ly["v"]
                W, HK, D = pk.shape[1], pk.shape[2], pk.shape[3]
                rows = slots * W + pos % W                     # ring slot
                attn.kv_write_slots(k, v, rows, pk.view(-1, HK, D),
                                    pv.view(-1, HK, D))
                self.out[l].copy_(compat.attn_swa(q, pk, pv, slots, pos,
                                                  rel))

    def _capture(self, L_pad):
        # dead-row config in every static input: the executed warm-ups only
        # write the scratch slot / page (graphrun.py:267-277)
        self.pos_buf.zero_()
        self.slots_buf.fill_(self.scratch)
        g = StepGraph(lambda: self._run(L_pad), self.device).capture()
        self.programs[L_pad] = g
        self.captures += 1

    def bucket(self, pos):
        L = -(-(max(pos) + 1) // BUCKET) * BUCKET
        L = max(L, self.hiwater)
        return min(L, self.reach) if self.reach is not None else L

    def step(self, pos, slots):
        """One graphed step for the live rows: pos / slots host int lists in
        row order (len <= max_batch). Returns the L_pad bucket replayed."""
        B = len(pos)
        assert B == len(slots) and 0 < B <= self.MB
        L_pad = self.bucket(pos)
        if L_pad not in self.programs:
            self._capture(L_pad)
        self.hiwater = L_pad
        dead = self.MB - B
        # staged through pinned memory: queued on the stream, no host sync
        host = torch.tensor([list(pos) + [0] * dead,
                             list(slots) + [self.scratch] * dead],
                            dtype=torch.int64).pin_memory()
        self.pos_buf.copy_(host[0], non_blocking=True)
        self.slots_buf.copy_(host[1], non_blocking=True)
        self.programs[L_pad].replay()
        return L_pad
