/*
 * tmopt_attn.h — C ABI of the MI355X (gfx950) paged-attention library
 * libtmopt_attn.so.
 *
 * This is the drop-in boundary for tm-opt's paged attention path. Every entry
 * point takes plain device pointers, sizes and strides plus a hipStream_t; no
 * C++ or torch types cross the boundary. Conventions shared by all entry
 * points:
 *
 *   - Return value: 0 (TMOPT_OK) or a negative tmopt_status. Nothing aborts.
 *     tmopt_last_error() returns a thread-local description of the last
 *     failure on the calling thread.
 *   - Nothing allocates device memory. Scratch space is passed in through a
 *     `workspace` argument whose size the matching *_workspace_size query
 *     returns, so every call is legal inside hipGraph stream capture.
 *   - Every launch goes to the given stream; no host synchronisation.
 *   - Tensors are bf16 unless stated. Index tensors are int32 (block tables,
 *     lengths, cu_seqlens) or int64 (flat slot mappings).
 *   - KV pools are [num_pages, page_size, HKV, D] bf16, contiguous: one page
 *     holds page_size consecutive token rows, each row HKV*D elements. A pool
 *     row index is page * page_size + offset.
 *   - Results are deterministic: fixed reduction order, no atomics.
 *
 * Supported shapes: D == 128, page_size == 16, HQ % HKV == 0 with
 * any REP = HQ / HKV (the reference's H % HK == 0, attn_prefill.py:174).
 * Decode reads each KV head's pages once for up to 16 query heads; a
 * larger REP runs in groups of its largest divisor up to 16, each group
 * reading the pages once. Prefill stages keys once for up to 8 query heads;
 * a REP that 8, 4 or 2 does not divide runs in groups of the largest of
 * them (or 1) dividing it, each group loading the keys once.
 * Other shapes return TMOPT_EUNSUPPORTED.
 */
#ifndef TMOPT_ATTN_H
#define TMOPT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; declared here without HIP headers so
 * that host-only callers (ctypes, cgo, plain C) can include this file. */
typedef struct ihipStream_t* tmopt_stream_t;

typedef enum {
  TMOPT_OK = 0,
  TMOPT_EINVAL = -1,       /* bad pointer, size or stride */
  TMOPT_EUNSUPPORTED = -2, /* shape outside the supported set above */
  TMOPT_EWORKSPACE = -3,   /* workspace missing or too small */
  TMOPT_ELAUNCH = -4       /* hipLaunchKernel / hipGetLastError failure */
} tmopt_status;

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* tmopt_last_error(void);

/* Library version string, e.g. "tmopt_attn 0.1 gfx950". */
const char* tmopt_version(void);

/* ------------------------------------------------------------------------ */
/* KV-cache write                                                           */
/* ------------------------------------------------------------------------ */

/*
 * Scatter T token rows of K and V into the pools by flat row index.
 * Replaces the reference's torch index_put_ appends
 *   pool.kp.view(-1, HK, D)[flat_new] = k   (engine/pyengine/model.py:941-942)
 *   pool.k[slots, ring_slot] = k            (engine/pyengine/model.py:947-948)
 *   self.kp.view(-1, H, D)[slots] = k       (engine/pyengine/kv.py:203-204)
 * k, v:          [T, HKV, D] with element strides (k_stride_tok,
 *                k_stride_head); the D axis must be contiguous.
 * slot_mapping:  [T] int64 flat pool rows; a negative entry skips the token.
 *                Rows >= pool_rows are skipped as well (never written).
 * k_pool,v_pool: [pool_rows, HKV, D] contiguous.
 * Bit-exact copy. Duplicate rows in one call are written in unspecified
 * order (the same contract as index_put_ without accumulate).
 * T * HKV * D / 8 must stay below 2^31 (TMOPT_EINVAL otherwise).
 */
int tmopt_kv_write_slots(const void* k, const void* v, int64_t k_stride_tok,
                         int64_t k_stride_head, int64_t v_stride_tok,
                         int64_t v_stride_head, const int64_t* slot_mapping,
                         int64_t T, int HKV, int D, void* k_pool, void* v_pool,
                         int64_t pool_rows, tmopt_stream_t stream);

/*
 * Append varlen token runs through a block table, computing each row's page
 * in-kernel. Replaces PagedKV.append / RingKV.append
 * (engine/pyengine/kv.py:193-205, :89-103) and the decode-step append
 * (engine/pyengine/model.py:938-948) without the torch index math.
 * Token t of sequence i (cu_seqlens[i] <= t < cu_seqlens[i+1]) sits at
 * logical position start_pos[i] + (t - cu_seqlens[i]); its pool row is
 *   table[i][lp] * page_size + pos % page_size,  lp = pos / page_size,
 * with lp taken modulo table_wrap when table_wrap > 0 (ring pools: a
 * sequence owns table_wrap pages that are reused cyclically). With
 * table_wrap > 0 a token that a later token of the same call would
 * overwrite is dropped, as RingKV.append does (kv.py:97-98).
 * cu_seqlens may be NULL: then sequence i has exactly one token, k row i
 * (the decode step). max_seqlen bounds the per-sequence token count, and
 * max_seqlen * HKV * D / 8 must stay below 2^31 (TMOPT_EINVAL otherwise);
 * positions are int32.
 * Table entries outside [0, num_pages) are skipped, never dereferenced,
 * and so are tokens whose logical page lies past the row width (index >=
 * bt_stride).
 * Element strides: k[row, h, d] = k + row * k_stride_tok + h * k_stride_head
 * + d * k_stride_dim (v likewise). k_stride_dim == 1 (token-major rows,
 * 16-byte aligned) is the general form. Channel-major K / V -- tokens
 * contiguous (k_stride_tok == 1), head_dim strided, as the sconv hands the
 * prefill's K / V to the cache append (engine/pyengine/model.py:486-512,
 * experiments/DEADENDS.md:631-645) -- are read in place and transposed on
 * chip: D == 128, k_stride_dim, k_stride_head multiples of 8, 16-byte
 * aligned base (TMOPT_EUNSUPPORTED otherwise).
 */
int tmopt_kv_write_paged(const void* k, const void* v, int64_t k_stride_tok,
                         int64_t k_stride_head, int64_t k_stride_dim,
                         int64_t v_stride_tok, int64_t v_stride_head,
                         int64_t v_stride_dim, const int32_t* cu_seqlens,
                         const int32_t* start_pos, int num_seqs, int max_seqlen,
                         const int32_t* block_table, int64_t bt_stride,
                         int table_wrap, int page_size, int HKV, int D,
                         void* k_pool, void* v_pool, int64_t num_pages,
                         tmopt_stream_t stream);

/*
 * The prefill's cache population for a whole batch in one launch. Replaces
 * the engine's per-row loop (engine/pyengine/model.py:507-512:
 * st.cache.append(kn[i, :lens[i]], vv[i, :lens[i]]) for each row i, i.e.
 * PagedKV.append / RingKV.append, kv.py:193-205, :89-103): row r's tokens
 * t < lens[r] are k + r * k_stride_row + t * k_stride_tok + h *
 * k_stride_head + d * k_stride_dim (v likewise), written at logical
 * positions start_pos[r] + t through block-table row r, with every rule of
 * tmopt_kv_write_paged (page rule, ring wrap and drop, row-width bound,
 * skipped out-of-pool entries, token-major or channel-major rows). Row
 * strides are multiples of 8 elements; max_len >= every lens[r].
 */
int tmopt_kv_append_rows(const void* k, const void* v, int64_t k_stride_row,
                         int64_t k_stride_tok, int64_t k_stride_head,
                         int64_t k_stride_dim, int64_t v_stride_row,
                         int64_t v_stride_tok, int64_t v_stride_head,
                         int64_t v_stride_dim, const int32_t* lens,
                         const int32_t* start_pos, int num_rows, int max_len,
                         const int32_t* block_table, int64_t bt_stride,
                         int table_wrap, int page_size, int HKV, int D,
                         void* k_pool, void* v_pool, int64_t num_pages,
                         tmopt_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Paged decode attention (split-KV + LSE combine)                          */
/* ------------------------------------------------------------------------ */

/*
 * Work-groups tmopt_attn_decode_paged launches when num_workgroups == 0
 * (three per four compute units of the current device, divided among the
 * HKV / 4 head groups).
 */
int tmopt_attn_decode_default_workgroups(int HKV);

/*
 * Bytes of workspace tmopt_attn_decode_paged needs for a launch shape
 * (num_workgroups 0 = the default above): per-piece partial results of
 * sequences that several work-groups share, plus the split geometry the
 * merge kernel reads. No initialisation needed.
 */
size_t tmopt_attn_decode_workspace_size(int B, int HQ, int HKV, int D,
                                        int num_workgroups);

/*
 * One query token per sequence against its paged KV history. Replaces
 * _attn_decode_kernel (engine/pyengine/kernels/attn_swa.py:49-117) behind
 * attn_swa (attn_swa.py:120-141) and attn_global
 * (engine/pyengine/kernels/attn_global.py:15-38), and the unimplemented
 * native stub tmopt::kernels::decode_attention
 * (engine/include/tmopt/kernels.h:33-35).
 *
 * q:            [B, HQ, D] contiguous; query of sequence b sits at position
 *               ctx_lens[b] - 1.
 * k_pool,v_pool:[num_pages, page_size, HKV, D] contiguous.
 * block_table:  [B, bt_stride] int32 physical page ids; logical page lp of
 *               sequence b is block_table[b*bt_stride + (table_wrap ?
 *               lp % table_wrap : lp)]. Only pages holding visible keys are
 *               read; entries outside [0, num_pages) are never dereferenced
 *               and a logical page past the row width (index >= bt_stride)
 *               has no entry: the keys of both count as absent.
 * ctx_lens:     [B] int32 keys in the cache including the current token
 *               (0 = empty: output 0, LSE -inf).
 * window:       0 = global; W > 0 = sliding window, keys k with
 *               pos - k < W only (pages wholly outside are never read).
 *               With table_wrap > 0, 0 < window <= table_wrap * page_size
 *               (TMOPT_EINVAL otherwise: the ring no longer holds older
 *               keys).
 * scale:        softmax scale applied to q.k.
 * rel, rel_extent: optional fused relative bias (NULL = off): rel is
 *               [B, HQ, rel_extent] contiguous and the score of key k gets
 *               rel[b, h, dist] for 0 <= dist = pos - k < rel_extent, else 0
 *               (attn_swa.py:97-102).
 * min_pages:    lower bound of pages per work-group (> 0). The visible
 *               pages of the whole batch are dealt out in equal contiguous
 *               ranges of max(ceil(total / num_workgroups), min_pages).
 * num_workgroups: persistent grid size (0 = default). The grid does not
 *               depend on ctx_lens, so a captured hipGraph stays valid for
 *               any lengths.
 * out:          [B, HQ, D] bf16; lse: [B, HQ] fp32 natural-log sum-exp of
 *               the scaled scores (may be NULL).
 * workspace:    device scratch of tmopt_attn_decode_workspace_size bytes,
 *               16-byte aligned.
 * Two launches on `stream`: the persistent split kernel, then the merge of
 * sequences that were split across work-groups.
 * B <= 8192.
 */
int tmopt_attn_decode_paged(const void* q, const void* k_pool,
                            const void* v_pool, const int32_t* block_table,
                            int64_t bt_stride, int table_wrap,
                            const int32_t* ctx_lens, int B, int HQ, int HKV,
                            int D, int page_size, int64_t num_pages,
                            int window, float scale, const void* rel,
                            int rel_extent, int min_pages, int num_workgroups,
                            void* out, float* lse, void* workspace,
                            size_t workspace_bytes, tmopt_stream_t stream);

/*
 * Paged decode over a sliding-window layer's ring pool as the reference
 * engine hands it to attn_swa (engine/pyengine/kernels/attn_swa.py:
 * 120-141): the SwaPool rows (engine/pyengine/kv.py:215-235) k_pool /
 * v_pool [S+1, W, HKV, D] viewed as (S+1) * ring_pages pages of 16 tokens
 * (W = 16 * ring_pages), slots [B] int64 ring rows, pos [B] int64 query
 * positions. Row b attends keys max(0, pos[b] - window + 1) .. pos[b],
 * which sit at ring slot p % W of row slots[b] (RingKV, kv.py:75-76);
 * 0 < window <= W. No block table or lengths need building per call: the
 * kernels read slots and pos in place. Otherwise as
 * tmopt_attn_decode_paged (num_pages = (S+1) * ring_pages), with the same
 * results.
 * seqs_per_workgroup > 0 replaces the equal page split: work-group i takes
 * the whole rows [i * seqs_per_workgroup, (i + 1) * seqs_per_workgroup)
 * (num_workgroups * seqs_per_workgroup >= B, else TMOPT_EINVAL), so no row
 * is split and the merge launch is skipped (one launch). A row holds at most
 * ring_pages pages, so with full rings the work stays balanced.
 */
int tmopt_attn_decode_ring(const void* q, const void* k_pool,
                           const void* v_pool, const int64_t* slots,
                           int ring_pages, const int64_t* pos, int B, int HQ,
                           int HKV, int D, int64_t num_pages, int window,
                           float scale, const void* rel, int rel_extent,
                           int min_pages, int num_workgroups,
                           int seqs_per_workgroup, void* out, float* lse,
                           void* workspace, size_t workspace_bytes,
                           tmopt_stream_t stream);

/*
 * The int32 block table and lengths of attn_global's arguments
 * (engine/pyengine/kernels/attn_global.py:15-38): flat [B, Lg] int64
 * per-token pool rows as model.py:938-945 builds them (flat[b, j] =
 * table[b][j / 16] * 16 + j % 16 for j <= pos[b], 0 beyond) and pos [B]
 * int64. Writes block_table[b * bt_stride + i] = flat[b, 16 i] / 16 for
 * i < ceil(Lg / 16) (a page's rows are consecutive, so its first row names
 * it) and ctx_lens[b] = pos[b] + 1, in one launch: the inputs of
 * tmopt_attn_decode_paged. bt_stride >= ceil(Lg / 16).
 */
int tmopt_decode_table_from_flat(const int64_t* flat, int64_t Lg,
                                 const int64_t* pos, int B,
                                 int32_t* block_table, int64_t bt_stride,
                                 int32_t* ctx_lens, tmopt_stream_t stream);

/*
 * tmopt_attn_decode_paged without the workspace argument: the same kernels
 * and results, with the scratch taken from a static device array inside the
 * library (16 MiB per GPU, held until the process ends). This entry point
 * has no counterpart in the reference; it is for callers that cannot
 * allocate device memory: code under hipGraph stream capture, tight serving
 * loops, harnesses that forbid hipMalloc. It calls no hipMalloc / hipFree
 * and no allocating library routine.
 *   - Launch shapes whose workspace (tmopt_attn_decode_workspace_size)
 *     exceeds 16 MiB return TMOPT_EWORKSPACE (e.g. (B + num_workgroups) *
 *     HQ above ~32,000).
 *   - Every call on one GPU shares that GPU's array: calls that overlap on
 *     one GPU (concurrent streams, or graphs replayed concurrently) race.
 *     Calls in stream order do not: the scratch needs no clearing between
 *     calls (every slot a call reads, that call writes first).
 *   - The first call on a device resolves the array's device address
 *     (hipGetSymbolAddress); make it outside stream capture.
 */
int tmopt_attn_decode_paged_noalloc(const void* q, const void* k_pool,
                                    const void* v_pool,
                                    const int32_t* block_table,
                                    int64_t bt_stride, int table_wrap,
                                    const int32_t* ctx_lens, int B, int HQ,
                                    int HKV, int D, int page_size,
                                    int64_t num_pages, int window, float scale,
                                    const void* rel, int rel_extent,
                                    int min_pages, int num_workgroups,
                                    void* out, float* lse,
                                    tmopt_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Varlen causal prefill attention (bf16 MFMA)                              */
/* ------------------------------------------------------------------------ */

/*
 * Causal (optionally windowed) attention for packed variable-length query
 * runs. Replaces _attn_prefill_kernel
 * (engine/pyengine/kernels/attn_prefill.py:71-141) behind attn_prefill_fused
 * (attn_prefill.py:144-194); the padded [B,H,T,D] form becomes cu_seqlens
 * packing, and chunked prefill (the seam the reference leaves at
 * Engine.prefill, engine/pyengine/scheduler.py:22-23) reads prior context
 * from the paged cache or the sliding-window ring.
 *
 * q:      [total_q, HQ, D] with element strides (q_stride_tok,
 *         q_stride_head), D contiguous. Query j of sequence i (row
 *         cu_seqlens_q[i] + j) sits at position prior_lens[i] + j
 *         (prior_lens NULL = all zero).
 * Keys of sequence i are positions [0, prior_lens[i] + len_i). They come
 * from one of three sources:
 *   block_table == NULL (packed): k, v hold the run's own keys; prior_lens
 *         and table_wrap must be 0. Key j of run i, head h, dim d sits at
 *         element base_i + j * k_stride_tok + h * k_stride_head +
 *         d * k_stride_dim, where base_i = i * k_stride_run, or
 *         cu_seqlens_q[i] * k_stride_tok when k_stride_run is 0 (likewise
 *         v). Token-major rows: k_stride_dim == 1, k_stride_tok % 8 == 0.
 *         Channel-major rows (tokens contiguous, head_dim strided: the
 *         sconv output the reference hands to attn_prefill_fused,
 *         attn_prefill.py:162-168, experiments/DEADENDS.md:631-645):
 *         k_stride_tok == 1, k_stride_dim % 8 == 0 and >= max_seqlen_q,
 *         k_stride_run > 0; read in place. A channel-major row is read in
 *         16-byte pieces, so up to 7 elements past a run's last key (within
 *         the row) are read as well: they must be finite (they get zero
 *         weight). Run, head strides % 8 == 0 and 16-byte aligned k / v in
 *         both layouts.
 *   block_table != NULL, k == v == NULL (paged): every key is read from
 *         the paged pools (k_pool, v_pool, [num_pages, page_size, HKV, D])
 *         through block_table [num_seqs, bt_stride]; the run's new keys
 *         must already be written (tmopt_kv_write_paged). table_wrap = 0.
 *   block_table != NULL, k, v given (mixed): keys before prior_lens[i]
 *         from the pools, the run's own keys from packed, token-major
 *         k / v (addressed as above). The run's
 *         keys need not be in the pool yet: append them afterwards. With
 *         table_wrap > 0 each table row is a ring of table_wrap pages
 *         holding the last table_wrap * page_size positions (RingKV /
 *         SwaPool, engine/pyengine/kv.py:66-114, :215-235); then
 *         0 < window <= table_wrap * page_size, and the append must come
 *         after this call (it overwrites the ring).
 * Pool reads: logical page lp of sequence i is block_table[i * bt_stride +
 *         (table_wrap ? lp % table_wrap : lp)]; a page past the row width
 *         (index >= bt_stride) or with an entry outside [0, num_pages)
 *         reads as zeros. Rows before the first key a query block may see
 *         (window) are never read, so a windowed table may point pages
 *         wholly before the window at any page, poisoned or not.
 * window: 0 = causal; W > 0 adds pos_q - pos_k < W. Key tiles wholly
 *         outside the causal/window band are skipped.
 * scale:  softmax scale (> 0).
 * rel, rel_extent: optional fused relative bias (NULL = off): row r of q
 *         (token) and head h own rel[r * rel_stride_tok + h * rel_stride_head
 *         + dist] for 0 <= dist = pos_q - pos_k < rel_extent; pairs outside
 *         that band get 0 (attn_prefill.py:115-120). Rows must not overlap
 *         (rel_stride_tok >= rel_extent) and 32 rows must span less than
 *         2 GiB, else TMOPT_EUNSUPPORTED.
 * A run's q rows (and, with packed keys, its k / v rows) must span less
 * than 2 GiB (max_seqlen_q * stride): TMOPT_EUNSUPPORTED otherwise.
 * max_seqlen_q bounds every len_i (it sizes the grid).
 * out:    [total_q, HQ, D] with element strides (o_stride_tok,
 *         o_stride_head), D contiguous.
 * lse:    [HQ, total_q] fp32 natural-log sum-exp of the scaled scores, or
 *         NULL.
 * reject: optional device int32 (NULL = none). When it holds a nonzero
 *         value at launch, every output row and LSE entry the launch owns
 *         is written as NaN and no key is read: a caller that validated its
 *         inputs on the device (e.g. attn_prefill_fused's positions must
 *         be an arange) fails loudly without a host synchronisation.
 */
int tmopt_attn_prefill_varlen(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
    int64_t k_stride_run, int64_t k_stride_tok, int64_t k_stride_head,
    int64_t k_stride_dim, const void* v, int64_t v_stride_run,
    int64_t v_stride_tok, int64_t v_stride_head, int64_t v_stride_dim,
    const int32_t* cu_seqlens_q,
    const int32_t* prior_lens, int num_seqs, int max_seqlen_q,
    const void* k_pool, const void* v_pool, const int32_t* block_table,
    int64_t bt_stride, int table_wrap, int page_size, int64_t num_pages,
    int HQ, int HKV, int D, int window, float scale, const void* rel,
    int64_t rel_stride_tok, int64_t rel_stride_head, int rel_extent,
    void* out, int64_t o_stride_tok, int64_t o_stride_head, float* lse,
    const int32_t* reject, tmopt_stream_t stream);

/*
 * The position contract of the reference's fused prefill
 * (engine/pyengine/kernels/attn_prefill.py:144-186: q_positions and
 * kv_positions [T] int64, the arange the engine builds, model.py:526-528),
 * checked on the device without a host synchronisation: writes
 * *reject = 0 when q_positions[i] - q_positions[0] == i and
 * kv_positions[i] - q_positions[0] == i for every i < T, else 1 (the
 * flag tmopt_attn_prefill_varlen takes as `reject`). One work-group.
 */
int tmopt_prefill_check_positions(const int64_t* q_positions,
                                  const int64_t* kv_positions, int64_t T,
                                  int32_t* reject, tmopt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TMOPT_ATTN_H */
