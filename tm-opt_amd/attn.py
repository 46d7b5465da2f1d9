"""Native (block-table / varlen) entry points over the C ABI.

Every function here validates its tensors the way the reference wrappers do
(dtype, shape and contiguity asserts before launch, attn_swa.py:128-132,
attn_global.py:25-29, attn_prefill.py:169-180), then hands raw device
pointers, sizes and strides to libtmopt_attn.so on the current stream of the
tensors' device. Nothing here computes attention: if the library is absent
the call raises.
"""
import torch

from . import _lib

PAGE_SIZE = 16
HEAD_DIM = 128


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _check_rows(t, name):
    assert t.dtype == torch.bfloat16, f"{name} must be bf16, got {t.dtype}"
    assert t.stride(-1) == 1, f"{name}: last (head_dim) axis must be contiguous"


# --------------------------------------------------------------------------
# KV-cache write
# --------------------------------------------------------------------------

def kv_write_slots(k, v, slot_mapping, k_pool, v_pool):
    """pool.view(-1, HKV, D)[slot_mapping] = k (and v), bit-exact.

    k, v [T, HKV, D] bf16 (D contiguous); slot_mapping [T] int64 flat rows of
    the pools, negative = skip; k_pool/v_pool [..., HKV, D] bf16 contiguous
    (a [P, page, HKV, D] page pool or a [S, W, HKV, D] ring pool).
    Reference: engine/pyengine/model.py:941-942, :947-948; kv.py:203-204."""
    T, HKV, D = k.shape
    assert v.shape == k.shape, (v.shape, k.shape)
    _check_rows(k, "k")
    _check_rows(v, "v")
    assert slot_mapping.dtype == torch.int64 and slot_mapping.shape == (T,)
    assert k_pool.is_contiguous() and v_pool.is_contiguous()
    assert k_pool.shape == v_pool.shape and k_pool.dtype == torch.bfloat16
    assert tuple(k_pool.shape[-2:]) == (HKV, D), (k_pool.shape, HKV, D)
    rows = k_pool.numel() // (HKV * D)
    dev = k.device
    _lib.call("tmopt_kv_write_slots", _ptr(k), _ptr(v), k.stride(0),
              k.stride(1), v.stride(0), v.stride(1), _ptr(slot_mapping), T,
              HKV, D, _ptr(k_pool), _ptr(v_pool), rows, _stream(dev))


def _channel_major(x):
    """Rows [T, H, D] with contiguous tokens and a strided head_dim (the
    sconv output's layout) rather than contiguous head_dim rows."""
    return x.stride(-1) != 1 and x.stride(0) == 1


def kv_write_paged(k, v, block_table, start_pos, k_pool, v_pool,
                   cu_seqlens=None, max_seqlen=None, table_wrap=0):
    """Append token runs through a block table (positions computed in-kernel).

    k, v [T, HKV, D] bf16: token-major rows (head_dim contiguous) or
    channel-major ones (tokens contiguous, head_dim strided: the sconv
    output the reference's prefill appends, model.py:486-512), read in place
    either way; block_table [S, bt_stride] int32; start_pos [S] int32;
    cu_seqlens [S+1] int32 or None (one token per sequence: the decode
    step); pools [num_pages, page_size, HKV, D]. table_wrap > 0 makes each
    table row a ring of table_wrap pages (sliding-window pools).
    Reference: engine/pyengine/kv.py:89-103, :193-205; model.py:938-948."""
    T, HKV, D = k.shape
    assert v.shape == k.shape
    for x, name in ((k, "k"), (v, "v")):
        assert x.dtype == torch.bfloat16, f"{name} must be bf16"
        assert x.stride(-1) == 1 or _channel_major(x), \
            f"{name}: head_dim or tokens must be contiguous"
    assert block_table.dtype == torch.int32 and block_table.dim() == 2
    assert block_table.stride(1) == 1
    assert start_pos.dtype == torch.int32
    S = start_pos.shape[0]
    assert block_table.shape[0] >= S
    # the kernel bounds every row read by the stride: rows must be whole
    assert block_table.stride(0) == block_table.shape[1] or S <= 1, \
        "block-table rows must be whole (the row width is the stride)"
    if cu_seqlens is None:
        assert T == S, (T, S)
        max_seqlen = 1
    else:
        assert cu_seqlens.dtype == torch.int32 and cu_seqlens.shape == (S + 1,)
        if max_seqlen is None:
            max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max()) if S else 0
    assert k_pool.is_contiguous() and v_pool.is_contiguous()
    assert k_pool.shape == v_pool.shape and k_pool.dim() == 4
    P, page_size = k_pool.shape[0], k_pool.shape[1]
    assert tuple(k_pool.shape[2:]) == (HKV, D)
    _lib.call("tmopt_kv_write_paged", _ptr(k), _ptr(v), k.stride(0),
              k.stride(1), k.stride(2), v.stride(0), v.stride(1),
              v.stride(2), _ptr(cu_seqlens),
              _ptr(start_pos), S, int(max_seqlen), _ptr(block_table),
              block_table.stride(0), int(table_wrap), page_size, HKV, D,
              _ptr(k_pool), _ptr(v_pool), P, _stream(k.device))


def kv_append_rows(k, v, lens, start_pos, block_table, k_pool, v_pool,
                   max_len=None, table_wrap=0):
    """The prefill's cache population for a batch in one launch
    (model.py:507-512: st.cache.append(kn[i, :lens[i]], vv[i, :lens[i]])
    for every row i): k, v [B, T, HKV, D] bf16 views, token-major (head_dim
    contiguous) or channel-major (tokens contiguous), row stride a multiple
    of 8; lens / start_pos [B] int32 (device); block_table [B, width] int32
    with whole rows; pools [num_pages, page_size, HKV, D]. Row i's first
    lens[i] tokens land at positions start_pos[i].. through table row i, with
    every rule of kv_write_paged (kv.py:89-103, :193-205)."""
    B, T, HKV, D = k.shape
    assert v.shape == k.shape
    for x, name in ((k, "k"), (v, "v")):
        assert x.dtype == torch.bfloat16, f"{name} must be bf16"
        assert x.stride(-1) == 1 or x.stride(1) == 1, \
            f"{name}: head_dim or tokens must be contiguous"
    assert lens.dtype == torch.int32 and lens.shape == (B,)
    assert start_pos.dtype == torch.int32 and start_pos.shape == (B,)
    assert block_table.dtype == torch.int32 and block_table.dim() == 2
    assert block_table.shape[0] >= B and block_table.stride(1) == 1
    assert block_table.stride(0) == block_table.shape[1] or B <= 1, \
        "block-table rows must be whole (the row width is the stride)"
    assert k_pool.is_contiguous() and v_pool.is_contiguous()
    assert k_pool.shape == v_pool.shape and k_pool.dim() == 4
    P, page_size = k_pool.shape[0], k_pool.shape[1]
    assert tuple(k_pool.shape[2:]) == (HKV, D)
    _lib.call("tmopt_kv_append_rows", _ptr(k), _ptr(v), k.stride(0),
              k.stride(1), k.stride(2), k.stride(3), v.stride(0), v.stride(1),
              v.stride(2), v.stride(3), _ptr(lens), _ptr(start_pos), B,
              int(T if max_len is None else max_len), _ptr(block_table),
              block_table.stride(0), int(table_wrap), page_size, HKV, D,
              _ptr(k_pool), _ptr(v_pool), P, _stream(k.device))


# --------------------------------------------------------------------------
# Paged decode
# --------------------------------------------------------------------------

def decode_default_workgroups(HKV):
    """Grid size the library picks when num_workgroups == 0."""
    return int(_lib.load().tmopt_attn_decode_default_workgroups(HKV))


def decode_workspace_size(B, HQ, HKV, num_workgroups=0, D=HEAD_DIM):
    return int(_lib.load().tmopt_attn_decode_workspace_size(
        B, HQ, HKV, D, num_workgroups))


def decode_workspace(B, HQ, HKV, device, num_workgroups=0):
    """Scratch for decode_paged (per-piece partials + split geometry)."""
    n = decode_workspace_size(B, HQ, HKV, num_workgroups)
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def _decode_check(q, k_pool, v_pool, block_table, ctx_lens, window,
                  table_wrap, rel):
    B, HQ, D = q.shape
    assert q.dtype == torch.bfloat16 and q.is_contiguous()
    assert k_pool.is_contiguous() and v_pool.is_contiguous()
    assert k_pool.dtype == torch.bfloat16 and v_pool.dtype == torch.bfloat16
    assert k_pool.shape == v_pool.shape and k_pool.dim() == 4
    P, page_size, HKV, Dk = k_pool.shape
    assert Dk == D and HQ % HKV == 0, (k_pool.shape, q.shape)
    assert block_table.dtype == torch.int32 and block_table.dim() == 2
    assert block_table.stride(1) == 1 and block_table.shape[0] >= B
    # the kernel bounds every row read by the stride: rows must be whole
    assert block_table.stride(0) == block_table.shape[1] or B <= 1, \
        "block-table rows must be whole (the row width is the stride)"
    assert ctx_lens.dtype == torch.int32 and ctx_lens.shape == (B,)
    if rel is not None:
        assert rel.dtype == torch.bfloat16 and rel.is_contiguous()
        assert rel.shape[:2] == (B, HQ), (rel.shape, B, HQ)
    if table_wrap:
        assert 0 < window <= table_wrap * page_size, \
            "a ring table needs a window no wider than the ring"
    return B, HQ, D, P, page_size, HKV


def _decode_common_args(q, k_pool, v_pool, block_table, ctx_lens, scale,
                        window, table_wrap, rel, min_pages, num_workgroups,
                        dims):
    B, HQ, D, P, page_size, HKV = dims
    return (_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
            block_table.stride(0), int(table_wrap), _ptr(ctx_lens), B, HQ,
            HKV, D, page_size, P, int(window), float(scale), _ptr(rel),
            0 if rel is None else rel.shape[2], int(min_pages),
            int(num_workgroups))


def decode_paged(q, k_pool, v_pool, block_table, ctx_lens, scale, window=0,
                 table_wrap=0, rel=None, min_pages=8, num_workgroups=0,
                 out=None, lse=None, workspace=None, return_lse=True):
    """Split-KV paged decode attention (one launch, persistent grid).

    q [B, HQ, D] bf16 contiguous (query at position ctx_lens[b]-1);
    k_pool/v_pool [num_pages, 16, HKV, D] bf16 contiguous; block_table
    [B, bt_stride] int32; ctx_lens [B] int32; window 0 = global; table_wrap
    > 0 = each table row is a ring of that many pages (SWA ring pools).
    rel: optional [B, HQ, E] bf16 fused relative bias (attn_swa.py:97-102).
    min_pages / num_workgroups: work-split knobs (see the C header).
    workspace: from decode_workspace() (allocated if None; it needs no
    initialisation).
    Returns (out [B, HQ, D] bf16, lse [B, HQ] fp32).
    Reference: engine/pyengine/kernels/attn_swa.py:49-141,
    attn_global.py:15-38."""
    dims = _decode_check(q, k_pool, v_pool, block_table, ctx_lens, window,
                         table_wrap, rel)
    B, HQ, _, _, _, HKV = dims
    dev = q.device
    if out is None:
        out = torch.empty_like(q)
    if lse is None and return_lse:
        lse = torch.empty((B, HQ), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = decode_workspace(B, HQ, HKV, dev, num_workgroups)
    ws_bytes = workspace.numel() * workspace.element_size()
    _lib.call("tmopt_attn_decode_paged",
              *_decode_common_args(q, k_pool, v_pool, block_table, ctx_lens,
                                   scale, window, table_wrap, rel, min_pages,
                                   num_workgroups, dims),
              _ptr(out), _ptr(lse), _ptr(workspace), ws_bytes, _stream(dev))
    return out, lse


def decode_ring(q, pool_k, pool_v, slots, pos, scale, window, rel=None,
                min_pages=8, num_workgroups=0, seqs_per_workgroup=0,
                out=None, lse=None, workspace=None, return_lse=False):
    """Paged decode over a ring pool as the engine holds it: pool_k/pool_v
    [S, W, HKV, D] bf16 (SwaPool rows), slots [B] int64 ring rows, pos [B]
    int64 query positions, 0 < window <= W; the kernels read slots and pos
    in place (no block table or lengths built per call).
    seqs_per_workgroup > 0: each work-group takes that many whole rows (no
    row split, no merge launch; num_workgroups * seqs_per_workgroup >= B).
    Returns (out [B, HQ, D] bf16, lse [B, HQ] fp32 or None).
    Reference: engine/pyengine/kernels/attn_swa.py:120-141, kv.py:215-235."""
    B, HQ, D = q.shape
    assert q.dtype == torch.bfloat16 and q.is_contiguous()
    assert pool_k.is_contiguous() and pool_v.is_contiguous()
    assert pool_k.shape == pool_v.shape and pool_k.dim() == 4
    S, W, HKV, Dk = pool_k.shape
    assert W % PAGE_SIZE == 0 and Dk == D and HQ % HKV == 0
    assert 0 < window <= W
    assert slots.dtype == torch.int64 and slots.shape == (B,)
    assert pos.dtype == torch.int64 and pos.shape == (B,)
    assert slots.is_contiguous() and pos.is_contiguous()
    if rel is not None:
        assert rel.dtype == torch.bfloat16 and rel.is_contiguous()
        assert rel.shape[:2] == (B, HQ)
    per = W // PAGE_SIZE
    dev = q.device
    if out is None:
        out = torch.empty_like(q)
    if lse is None and return_lse:
        lse = torch.empty((B, HQ), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = decode_workspace(B, HQ, HKV, dev, num_workgroups)
    _lib.call("tmopt_attn_decode_ring", _ptr(q), _ptr(pool_k), _ptr(pool_v),
              _ptr(slots), per, _ptr(pos), B, HQ, HKV, D, S * per,
              int(window), float(scale), _ptr(rel),
              0 if rel is None else rel.shape[2], int(min_pages),
              int(num_workgroups), int(seqs_per_workgroup), _ptr(out),
              _ptr(lse), _ptr(workspace),
              workspace.numel() * workspace.element_size(), _stream(dev))
    return out, lse


def decode_table_from_flat(flat, pos, table=None, ctx_lens=None):
    """attn_global's per-token rows flat [B, Lg] int64 (model.py:938-945)
    and positions pos [B] int64 -> (block table [B, ceil(Lg/16)] int32 with
    table[b, i] = flat[b, 16 i] // 16, ctx_lens = pos + 1 int32), one
    launch. Reference: engine/pyengine/kernels/attn_global.py:15-38."""
    B, Lg = flat.shape
    assert flat.dtype == torch.int64 and flat.is_contiguous()
    assert pos.dtype == torch.int64 and pos.shape == (B,)
    assert pos.is_contiguous()
    npg = (Lg + PAGE_SIZE - 1) // PAGE_SIZE
    dev = flat.device
    if table is None:
        table = torch.empty((B, npg), dtype=torch.int32, device=dev)
    if ctx_lens is None:
        ctx_lens = torch.empty((B,), dtype=torch.int32, device=dev)
    assert table.dtype == torch.int32 and table.stride(1) == 1
    assert table.shape[0] >= B and table.shape[1] >= npg
    _lib.call("tmopt_decode_table_from_flat", _ptr(flat), Lg, _ptr(pos), B,
              _ptr(table), table.stride(0), _ptr(ctx_lens), _stream(dev))
    return table, ctx_lens


def decode_paged_noalloc(q, k_pool, v_pool, block_table, ctx_lens, scale,
                         out, lse=None, window=0, table_wrap=0, rel=None,
                         min_pages=8, num_workgroups=0):
    """decode_paged through the allocation-free entry point: the scratch is
    the library's static 16 MiB device buffer, so neither this call nor the
    library allocates (out, and lse if wanted, are the caller's). Calls
    that overlap on one GPU race on that buffer; launch shapes needing more
    scratch raise (TMOPT_EWORKSPACE). No counterpart in the reference: for
    callers that cannot allocate."""
    dims = _decode_check(q, k_pool, v_pool, block_table, ctx_lens, window,
                         table_wrap, rel)
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    assert out.is_contiguous()
    if lse is not None:
        assert lse.dtype == torch.float32 and lse.is_contiguous()
        assert lse.shape == q.shape[:2]
    _lib.call("tmopt_attn_decode_paged_noalloc",
              *_decode_common_args(q, k_pool, v_pool, block_table, ctx_lens,
                                   scale, window, table_wrap, rel, min_pages,
                                   num_workgroups, dims),
              _ptr(out), _ptr(lse), _stream(q.device))
    return out, lse


# --------------------------------------------------------------------------
# Varlen prefill
# --------------------------------------------------------------------------

def prefill_check_positions(q_positions, kv_positions, reject=None):
    """Device-side check of the fused prefill's position contract
    (attn_prefill.py:144-186): returns (or fills) an int32 [1] flag, 0 when
    q_positions and kv_positions are both q_positions[0] + arange(T), else
    1, for prefill_varlen's `reject`. No host synchronisation."""
    T = q_positions.shape[0]
    assert q_positions.shape == (T,) and kv_positions.shape == (T,)
    assert q_positions.dtype == torch.int64
    assert kv_positions.dtype == torch.int64
    assert q_positions.is_contiguous() and kv_positions.is_contiguous()
    assert q_positions.device == kv_positions.device
    if reject is None:
        reject = torch.empty(1, dtype=torch.int32, device=q_positions.device)
    _lib.call("tmopt_prefill_check_positions", _ptr(q_positions),
              _ptr(kv_positions), T, _ptr(reject),
              _stream(q_positions.device))
    return reject


def prefill_varlen(q, k, v, cu_seqlens, scale, window=0, max_seqlen=None,
                   prior_lens=None, k_pool=None, v_pool=None,
                   block_table=None, table_wrap=0, rel=None, out=None,
                   lse=None, return_lse=True, reject=None):
    """Varlen causal (optionally windowed) prefill attention on bf16 MFMA.

    q [total, HQ, D] bf16 (D contiguous, any token / head strides);
    cu_seqlens [S+1] int32. Query j of run i sits at position
    prior_lens[i] + j. Key sources:
      * block_table None: k/v hold each run's own keys (no prior context):
        [total, HKV, D] packed like q, or [S, T, HKV, D] with run i's keys
        in its first len_i rows (a padded batch read in place, T >=
        max_seqlen). Either token-major (head_dim contiguous) or
        channel-major (tokens contiguous, head_dim strided: the sconv
        output, attn_prefill.py:162-168), the latter in the [S, T, HKV, D]
        form only, T % 8 == 0;
      * block_table given, k/v None: every key, prior context included, is
        read from k_pool/v_pool [num_pages, 16, HKV, D] through block_table
        (int32 [S, bt_stride]); the run's own keys must already be there;
      * block_table and k/v given: prior keys from the pools, the run's own
        keys from k/v. table_wrap > 0 makes each table row a ring of that
        many pages (a sliding-window pool: 0 < window <= 16 * table_wrap,
        and the run must be appended to the ring after this call).
    rel: optional fused relative bias [total, HQ, E] (last axis contiguous,
    any token/head strides): pair (q, k) of head h adds rel[q_row, h,
    pos_q - pos_k] inside 0 <= dist < E (attn_prefill.py:115-120).
    reject: optional int32 device scalar; nonzero -> NaN outputs (device-side
    input rejection without a host sync).
    Returns (out [total, HQ, D] bf16, lse [HQ, total] fp32 or None).
    Reference: engine/pyengine/kernels/attn_prefill.py:71-194."""
    total, HQ, D = q.shape
    _check_rows(q, "q")
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.dim() == 1
    S = cu_seqlens.shape[0] - 1
    if max_seqlen is None:
        max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max()) if S else 0
    pooled = block_table is not None
    own = k is not None or v is not None
    if pooled:
        assert k_pool is not None and v_pool is not None
        assert k_pool.is_contiguous() and v_pool.is_contiguous()
        assert k_pool.shape == v_pool.shape and k_pool.dim() == 4
        P, page_size, HKV, Dk = k_pool.shape
        assert Dk == D
        assert block_table.dtype == torch.int32 and block_table.stride(1) == 1
        assert block_table.dim() == 2 and block_table.shape[0] >= S
        assert block_table.stride(0) == block_table.shape[1] or S <= 1, \
            "block-table rows must be whole (the row width is the stride)"
        if prior_lens is not None:
            assert prior_lens.dtype == torch.int32 and prior_lens.shape == (S,)
        if table_wrap:
            assert own, "a ring table needs the run's own k/v (mixed source)"
            assert 0 < window <= table_wrap * page_size, \
                "a ring table needs a window no wider than the ring"
    else:
        assert prior_lens is None, "prior context needs the paged source"
        assert own, "the packed source needs k and v"
        assert not table_wrap
        P, page_size = 0, PAGE_SIZE
    ks = vs = (0, 0, 0, 1)
    if own:
        assert k is not None and v is not None
        assert v.shape == k.shape and k.shape[-1] == D
        for x, name in ((k, "k"), (v, "v")):
            assert x.dtype == torch.bfloat16, f"{name} must be bf16"
        if k.dim() == 3:                       # packed by cu_seqlens
            _check_rows(k, "k")
            _check_rows(v, "v")
            assert k.shape[0] == total
            ks = (0, k.stride(0), k.stride(1), 1)
            vs = (0, v.stride(0), v.stride(1), 1)
        else:                                  # one padded row per run
            assert k.dim() == 4 and k.shape[0] >= S
            assert k.shape[1] >= max_seqlen, (k.shape, max_seqlen)
            for x, name in ((k, "k"), (v, "v")):
                assert x.stride(3) == 1 or x.stride(1) == 1, \
                    f"{name}: head_dim or tokens must be contiguous"
            ks = (k.stride(0), k.stride(1), k.stride(2), k.stride(3))
            vs = (v.stride(0), v.stride(1), v.stride(2), v.stride(3))
        if pooled:
            assert k.shape[-2] == HKV
            assert ks[3] == 1 and vs[3] == 1, \
                "the mixed source reads token-major k/v"
        HKV = k.shape[-2]
    assert HQ % HKV == 0
    if rel is not None:
        assert rel.dtype == torch.bfloat16 and rel.stride(2) == 1
        assert rel.shape[:2] == (total, HQ), (rel.shape, total, HQ)
    if reject is not None:
        assert reject.dtype == torch.int32 and reject.numel() >= 1
    dev = q.device
    if out is None:
        out = torch.empty((total, HQ, D), dtype=torch.bfloat16, device=dev)
    if lse is None and return_lse:
        lse = torch.empty((HQ, total), dtype=torch.float32, device=dev)
    _lib.call("tmopt_attn_prefill_varlen", _ptr(q), q.stride(0), q.stride(1),
              _ptr(k) if own else None, *ks,
              _ptr(v) if own else None, *vs, _ptr(cu_seqlens),
              _ptr(prior_lens), S, int(max_seqlen),
              _ptr(k_pool) if pooled else None,
              _ptr(v_pool) if pooled else None, _ptr(block_table),
              block_table.stride(0) if pooled else 0, int(table_wrap),
              page_size, P, HQ, HKV, D, int(window), float(scale), _ptr(rel),
              0 if rel is None else rel.stride(0),
              0 if rel is None else rel.stride(1),
              0 if rel is None else rel.shape[2], _ptr(out), out.stride(0),
              out.stride(1), _ptr(lse), _ptr(reject), _stream(dev))
    return out, lse
