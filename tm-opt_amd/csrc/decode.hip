// Persistent split-KV paged decode attention for gfx950 (CDNA4).
//
// Replaces _attn_decode_kernel (engine/pyengine/kernels/attn_swa.py:49-117):
// one query token per sequence against its paged K/V history, a GQA group
// of REP query heads per KV head, fp32 online softmax, probabilities rounded
// to bf16 for the P.V product (attn_swa.py:110-112), one bf16 rounding of
// the output. What is different, and why (MI355X):
//
//  * Balanced persistent grid. The visible pages of all sequences are laid
//    end to end (U pages in total) and work-group i of G processes the
//    contiguous range [i*C, (i+1)*C), C = max(ceil(U / G), min_pages). Every
//    work-group therefore streams the same number of bytes whatever the
//    length distribution, and the grid is fixed (G = 3/4 of the CUs by
//    default), so one launch shape serves every step of a captured
//    hipGraph.
//  * Only pages holding visible keys are touched: [lo/16, ceil(n/16)) where
//    lo = max(0, n - window) on sliding-window layers, 0 on global ones.
//  * A sequence cut by work-group boundaries leaves one normalised partial
//    (O, LSE) per piece, in slot b + i of the workspace (unique: work-groups
//    and sequences are both in order); decode_combine_kernel then merges
//    the pieces of each such sequence in work-group order. No atomics and no
//    cross-work-group fences (a device-scope release/acquire pair writes
//    back and invalidates a whole XCD L2 on MI355X), and a fixed merge
//    order, so repeated runs are bitwise identical. A sequence that one
//    work-group covers alone is written in place and skipped by the merge.
//  * One wave per KV head. The four waves of a work-group read the four
//    256-byte head slices of the same token rows, so together they stream
//    whole 16 KB pages. K and V arrive by 16-byte buffer loads whose
//    resource is one page: a missing page (past the range, or a table entry
//    outside the pool) has zero records, so its loads return zeros without
//    touching memory, and the next step's loads (query rows included, when
//    the step starts a new sequence) are always issued before the current
//    step's math (no branch around them, no vmcnt(0) drain).
//  * Coalesced loads: each group of 16 lanes reads one token's 256-byte
//    head slice (lanes 16 B apart); the rows are then staged through a
//    per-wave LDS tile (XOR-swizzled: conflict-free on 64 banks) from which
//    the MFMA fragments are read, V by transposed reads. Loading the MFMA
//    layout directly (16 tokens per instruction, lanes 1 KB apart) cost
//    12-15 % of the bandwidth.
//  * Scores and P.V run on MFMA (v_mfma_f32_16x16x32_bf16). S^T = K.Q^T puts
//    16 tokens on the M axis and the REP heads (padded to 16) on N, so each
//    lane owns 8 scores of one head: the running max needs two cross-lane
//    steps (xor 16, xor 32) and the running sum stays lane-local until the
//    end of a piece. P^T is then already in the B-operand layout of
//    O^T = V^T.P^T. Any GQA ratio up to 16 fills that many columns (one
//    read of the pages); a larger one runs as groups of its largest divisor
//    up to 16, each group a scheduled KV head of its own.
//
// Per step (two pages = 32 tokens, tile t = page t):
//  Load i of tile t brings tokens 16t + 4i + (lane >> 4), 16 bytes (dims
//  8 (lane & 15)..+7) per lane, into LDS rows of 256 B.
//  S^T: lane (r, g) reads row 16t + r, dims 32kk + 8g..+7 (one 16-byte read).
//  P.V: the A operand of lane (r, g) is dim 16 blk + r of tokens 4g..4g+3
//  and 16+4g..16+4g+3 (two transposed reads), matching the P^T lane layout
//  (element 4t + i <-> token 16t + 4g + i).
#include <mutex>

#include "common.h"

namespace tmopt {
namespace {

constexpr int kD = 128;
constexpr int kPS = 16;                      // tokens per page
constexpr int kRowB = 256;                   // one token's head slice
constexpr int kTileB = 2 * kPS * kRowB;      // 32 tokens: 8 KB
constexpr int kWaveLds = 2 * kTileB;         // K tile + V tile per wave
#ifndef TMOPT_DECODE_DEEP
#define TMOPT_DECODE_DEEP 2
#endif
constexpr int kDeep = TMOPT_DECODE_DEEP;     // step ring depth
constexpr int kMaxB = 8192;                  // prefix table lives in LDS
// cache policy of the K/V page loads: non-temporal (streamed once; the
// measured read rate of a plain stream rises from 6.2 to 6.9 TB/s with it)
constexpr int kStreamLoad = 2;

struct DecodeArgs {
  const __bf16* q;
  const __bf16* kpool;
  const __bf16* vpool;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_width;      // entries a row may be read at: min(bt_stride, 2^31-1)
  int table_wrap;
  const int32_t* ctx_lens;
  // the engine's own index tensors instead of a block table and lengths
  // (tmopt_attn_decode_ring): kind 2 = ring slots [B] int64 (page
  // slot * table_wrap + lp % table_wrap) and pos64 [B] int64 query
  // positions (keys = pos + 1)
  int bt_kind;
  const int64_t* rows64;
  const int64_t* pos64;
  int B, HQ;
  int HKV;           // KV heads as scheduled (HKV_stored * kv_div)
  int num_pages;     // clamped to INT32_MAX: page ids are int32
  int window;
  float scale_log2;  // scale * log2(e)
  const __bf16* rel;
  int rel_extent;
  int min_pages;     // lower bound of pages per work-group
  int seqs_per_wg;   // > 0: work-group i takes whole sequences
                     // [i * seqs_per_wg, (i + 1) * seqs_per_wg), no merge
  __bf16* out;
  float* lse;
  float* part_o;     // [B + G, HQ, D] fp32
  float* part_lse;   // [B + G, HQ]
  int* geo;          // [B + 2]: C, then the page-stream prefix pref[0..B]
  // read by the REP 0 kernels only (any other REP implies rep == REP,
  // kv_div == 1, HKV_stored == HKV)
  int rep;           // query heads per scheduled KV head (1..16)
  int kv_div;        // scheduled KV heads per stored one: 1 unless HQ/HKV
                     // is above 16 (then kv_div groups of `rep` query
                     // heads each read the stored head's pages)
  int HKV_stored;    // KV heads of a pool token row
};

__device__ __forceinline__ int vis_lo(int n, int window) {
  return (window > 0 && n > window) ? n - window : 0;
}

// visible pages of a sequence holding n tokens
__device__ __forceinline__ int vis_pages(int n, int window) {
  if (n <= 0) return 0;
  return (n + kPS - 1) / kPS - vis_lo(n, window) / kPS;
}

// keys of sequence b (its query sits at position n - 1)
template <int KIND>
__device__ __forceinline__ int seq_n(const DecodeArgs& a, int b) {
  if constexpr (KIND != 0) return (int)(as_const(a.pos64)[b] + 1);
  return as_const(a.ctx_lens)[b];
}

template <int KIND>
__device__ __forceinline__ int page_id(const DecodeArgs& a, int b, int lp) {
  const int idx = a.table_wrap > 0 ? lp % a.table_wrap : lp;
  int v;
  if constexpr (KIND == 2) {
    v = (int)as_const(a.rows64)[b] * a.table_wrap + idx;
  } else {
    // a logical page past the row's width has no entry: its keys are absent
    // (reading on would return the next row's page ids)
    if ((unsigned)idx >= (unsigned)a.bt_width) return -1;
    v = as_const(a.bt)[(int64_t)b * a.bt_stride + idx];
  }
  // one unsigned 32-bit compare: stays on the scalar unit (a 64-bit signed
  // compare would borrow VGPRs that in-flight loads may still own)
  return (unsigned)v < (unsigned)a.num_pages ? v : -1;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const __bf16* pool,
                                                            int phys,
                                                            int page_bytes) {
  const char* base = reinterpret_cast<const char*>(pool) +
                     (phys >= 0 ? (int64_t)phys * page_bytes : 0);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0,
                                           phys >= 0 ? page_bytes : 0,
                                           0x00020000);
}

// One 32-token step of the flattened page stream (wave-uniform).
struct Step {
  int b;       // sequence (-1: past the end of this work-group's range)
  int n;       // its context length
  int s0, s1;  // its first and one-past-last unit in the page stream
  int pg;      // first logical page
  int phys0, phys1;
  bool first;  // first step of this piece: the query rows come with it
  bool last;   // last step of this piece of sequence b
};

template <bool REL>
struct StepBuf {
  u32x4 q[4];     // query fragments (first step of a piece only)
  u32x4 k[2][4];  // [tile][load]: tokens 16 t + 4 i + (lane >> 4)
  u32x4 v[2][4];
  // raw bf16 bias bits of this lane's 8 scores, [4t + i] for token
  // 16t + 4g + i; converted only when used, so issuing never waits
  uint32_t rel[REL ? 8 : 1];
};

// Issue the loads of one 32-token step: the query fragments (from an
// empty resource, i.e. no memory traffic, unless the step starts a piece:
// a piece's query then never has to be waited for apart from its step),
// 16 K/V buffer loads and, with a relative bias, the 8 bias values this
// lane's scores need.
template <bool REL>
__device__ __forceinline__ void issue_step(StepBuf<REL>& buf,
                                           const DecodeArgs& a,
                                           const Step& st, int lane_off,
                                           int page_bytes, int hq, bool head_ok,
                                           int g) {
  {
    const bool want = st.first && st.b >= 0;
    const char* base = reinterpret_cast<const char*>(a.q) +
                       (want ? (int64_t)st.b * a.HQ * kD * 2 : 0);
    __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base), (short)0, want ? a.HQ * kD * 2 : 0,
        0x00020000);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      buf.q[kk] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rq, head_ok ? (hq * kD + 32 * kk + 8 * g) * 2 : 0x7ffffff0,
                     0, 0));
  }
  if constexpr (REL) {
    // rel row of sequence b: [HQ, E] bf16; out-of-band distances (and
    // padded heads) get an out-of-range offset, which reads as 0
    const char* base = reinterpret_cast<const char*>(a.rel) +
                       (st.b >= 0 ? (int64_t)st.b * a.HQ * a.rel_extent * 2 : 0);
    __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base), (short)0,
        st.b >= 0 ? a.HQ * a.rel_extent * 2 : 0, 0x00020000);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int dist = (st.n - 1) - ((st.pg + t) * kPS + 4 * g + i);
        const bool in = head_ok && dist >= 0 && dist < a.rel_extent;
        const int off = in ? (hq * a.rel_extent + dist) * 2 : 0x7ffffff0;
        buf.rel[4 * t + i] = __builtin_amdgcn_raw_buffer_load_b16(
            rr, off, 0, 0);
      }
  }
  // lane l of load i reads 16 bytes of token 4i + (l >> 4): each group of
  // 16 lanes reads one token's 256-byte head slice, so consecutive lanes
  // are contiguous and every instruction coalesces into 64-byte requests
  const int tok_b = page_bytes / kPS;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int phys = t == 0 ? st.phys0 : st.phys1;
    __amdgpu_buffer_rsrc_t rk = page_rsrc(a.kpool, phys, page_bytes);
    __amdgpu_buffer_rsrc_t rv = page_rsrc(a.vpool, phys, page_bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      buf.k[t][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rk, lane_off + 4 * i * tok_b, 0, kStreamLoad));
      buf.v[t][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rv, lane_off + 4 * i * tok_b, 0, kStreamLoad));
    }
  }
}

// DEPTH: steps whose loads are in flight or being consumed; DEPTH - 1 steps
// (16 KB each per wave) stream in while one is computed. One work-group per
// CU (one wave per SIMD, the whole register file per wave).
template <int REP, bool REL, int DEPTH, int KIND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void decode_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int r = lane & 15;  // MFMA row / column index
  const int g = lane >> 4;  // MFMA k-group
  const int wg = blockIdx.x;
  const int G = gridDim.x;
  const int kvh = blockIdx.y * nw + w;
  // the prefix table is only read before the walk; the per-wave K / V
  // tiles then reuse the same LDS (a barrier separates the two uses)
  int* pref = reinterpret_cast<int*>(smem);  // [B + 1]
  int* wsum = pref + a.B + 1;                // [4]

  // ---- 1. prefix sums of visible pages: pref[b] = first unit of seq b ----
  {
    int carry = 0;
    for (int b0 = 0; b0 < a.B; b0 += blockDim.x) {
      const int b = b0 + threadIdx.x;
      const int v = b < a.B ? vis_pages(seq_n<KIND>(a, b), a.window) : 0;
      // inclusive scan over the wave by DPP (VALU, no LDS round trips):
      // within each 16-lane row by shifts of 1, 2, 4, 8, then row 0's
      // total into row 1 and row 2's into row 3, then rows 0-1's total into
      // rows 2-3
      int x = v;
      x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // shr 1
      x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // shr 2
      x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // shr 4
      x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // shr 8
      x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false); // bcast 15
      x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false); // bcast 31
      if (lane == 63) wsum[w] = x;
      __syncthreads();
      int before = carry;
      for (int j = 0; j < w; ++j) before += wsum[j];
      if (b < a.B) pref[b + 1] = before + x;
      int tot = 0;
      for (int j = 0; j < nw; ++j) tot += wsum[j];
      carry += tot;
      __syncthreads();
    }
    if (threadIdx.x == 0) pref[0] = 0;
    __syncthreads();
  }
  const int U = __builtin_amdgcn_readfirstlane(pref[a.B]);
  int C = (U + G - 1) / G;
  if (C < a.min_pages) C = a.min_pages;
  // publish the split geometry for the combine kernel
  if (wg == 0 && blockIdx.y == 0) {
    for (int i = threadIdx.x; i <= a.B; i += blockDim.x) a.geo[1 + i] = pref[i];
    if (threadIdx.x == 0) a.geo[0] = C;
  }
  // this work-group's page range: an equal share of the page stream, or
  // (seqs_per_wg > 0) the pages of whole sequences, so that no sequence is
  // split and the merge has nothing to do
  int u0, u1;
  if (a.seqs_per_wg > 0) {
    const int b0 = min(wg * a.seqs_per_wg, a.B);
    const int b1 = min(b0 + a.seqs_per_wg, a.B);
    u0 = __builtin_amdgcn_readfirstlane(pref[b0]);
    u1 = __builtin_amdgcn_readfirstlane(pref[b1]);
  } else {
    u0 = min(wg * C, U);
    u1 = min(u0 + C, U);
  }
  // REP 1, 2, 4, 8, 16: that many query heads per KV head; REP 0: a.rep
  // of them (any count up to the 16 MFMA columns) and a.kv_div scheduled
  // heads per stored one
  const int rep = REP > 0 ? REP : a.rep;
  const int hq = kvh * rep + r;  // query head owned as MFMA column r
  const bool head_ok = r < rep;

  // ---- 2. sequences with no visible key: output 0, LSE -inf -------------
  for (int b = wg; b < a.B; b += G) {
    if (pref[b + 1] != pref[b] || !head_ok) continue;
    __bf16* o = a.out + ((int64_t)b * a.HQ + hq) * kD;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk)
      *reinterpret_cast<u32x2*>(o + 16 * blk + 4 * g) = u32x2{0, 0};
    if (a.lse && g == 0) a.lse[(int64_t)b * a.HQ + hq] = -INFINITY;
  }
  if (u0 >= u1) return;

  // ---- 3. the step stream of [u0, u1) -----------------------------------
  // Everything about the step stream is wave-uniform and lives in SGPRs:
  // the LDS prefix table is read only here, by the start-up binary search;
  // afterwards the running prefix advances from scalar loads of ctx_lens,
  // so no per-step LDS read needs a VGPR that an in-flight load still owns.
  int cb;  // first sequence with pref[cb + 1] > u0
  {
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (__builtin_amdgcn_readfirstlane(pref[mid + 1]) > u0) hi = mid;
      else lo = mid + 1;
    }
    cb = __builtin_amdgcn_readfirstlane(lo);
  }
  int seq_start = __builtin_amdgcn_readfirstlane(pref[cb]);
  int cur_n = seq_n<KIND>(a, cb);
  int seq_end = seq_start + vis_pages(cur_n, a.window);
  int cu = u0;
  int last_b = -1;  // sequence of the previous step handed out
  auto next_step = [&](Step& st) {
    if (cu >= u1) {
      st.b = -1; st.n = 0; st.pg = 0; st.phys0 = -1; st.phys1 = -1;
      st.s0 = 0; st.s1 = 0; st.first = false; st.last = false;
      return;
    }
    while (seq_end <= cu) {
      ++cb;
      seq_start = seq_end;
      cur_n = seq_n<KIND>(a, cb);
      seq_end = seq_start + vis_pages(cur_n, a.window);
    }
    const int piece_end = min(seq_end, u1);
    const int cnt = min(2, piece_end - cu);
    st.b = cb;
    st.n = cur_n;
    st.s0 = seq_start;
    st.s1 = seq_end;
    st.pg = vis_lo(cur_n, a.window) / kPS + (cu - seq_start);
    st.phys0 = page_id<KIND>(a, cb, st.pg);
    st.phys1 = cnt > 1 ? page_id<KIND>(a, cb, st.pg + 1) : -1;
    cu += cnt;
    st.last = cu == piece_end;
    st.first = cb != last_b;
    last_b = cb;
  };

  const int row_elems = (REP > 0 ? a.HKV : a.HKV_stored) * kD;
  const int page_bytes = kPS * row_elems * 2;
  const int kvs = REP > 0 ? kvh : kvh / a.kv_div;   // the stored KV head
  // byte offset of (token lane >> 4, head kvs, dims 8 (lane & 15)..) in a
  // page
  const int lane_off = ((lane >> 4) * row_elems + kvs * kD + 8 * (lane & 15)) * 2;
  // this wave's LDS tiles: 32 token rows of 256 B each for K, then for V.
  // K row x keeps 16-byte chunk c at slot c ^ (x & 15), V row x keeps
  // 32-byte unit u at slot u ^ (x & 7): conflict-free for the row writes,
  // for the K fragment reads (16 rows, one chunk) and for the transposed V
  // reads (8 rows, one unit, per 32 lanes).
  // The four lane-dependent bases below (multiples of 256 plus a swizzled
  // slot) give every access as base ^ (slot bits) + immediate.
  const uint32_t kt_l = (uint32_t)(uintptr_t)(
      (__attribute__((address_space(3))) char*)smem) + w * kWaveLds;
  const uint32_t vt_l = kt_l + kTileB;
  const int wtok = lane >> 4, wch = lane & 15;  // row / chunk of a write
  // write of load i, tile t: row x = 16t + 4i + wtok
  const uint32_t kw0 = kt_l + wtok * kRowB + 16 * (wch ^ wtok);
  const uint32_t vw0 = vt_l + wtok * kRowB + 32 * ((wch >> 1) ^ wtok) + 16 * (wch & 1);
  // K fragment (t, kk) of lane (r, g): row 16t + r, chunk 4kk + g
  const uint32_t kr0 = kt_l + r * kRowB + 16 * (g ^ r);
  // transposed V reads: rows 4g + (s >> 2) (+16), unit blk, dims 4 (s & 3)
  const int s16 = lane & 15;
  const int x0 = 4 * g + (s16 >> 2);
  const uint32_t vr0 = vt_l + x0 * kRowB + 32 * (x0 & 7) + 8 * (s16 & 3);

  // ---- per-piece state ----------------------------------------------------
  f32x4 o_acc[8];
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) o_acc[blk] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY;
  float l_part = 0.0f;
  bf16x8 qf[4];

  auto compute = [&](const StepBuf<REL>& buf, const Step& st) {
    const int n = st.n;
    const int lo = vis_lo(n, a.window);
    if (st.first) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, buf.q[kk]);
    }
    // ---- stage K and V rows in LDS -----------------------------------------
    // (V rows of invalid tokens are zeroed: masked probabilities are 0 and
    // must not meet a NaN in P.V)
    const int k0 = st.pg * kPS;
    wave_lds_sync();  // the previous step's fragment reads are done
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bool page_ok = (t == 0 ? st.phys0 : st.phys1) >= 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // row x = 16t + 4i + wtok: x & 15 = 4i ^ wtok, x & 7 = 4(i & 1) ^ wtok
        const int kpos = k0 + 16 * t + 4 * i + wtok;
        const bool vok = page_ok && kpos >= lo && kpos < n;
        const uint32_t rowo = (16 * t + 4 * i) * kRowB;
        lds_st128((kw0 ^ (64u * i)) + rowo, buf.k[t][i]);
        lds_st128((vw0 ^ (128u * (i & 1))) + rowo,
                  vok ? buf.v[t][i] : u32x4{0, 0, 0, 0});
      }
    }
    wave_lds_sync();
    // ---- S^T = K.Q^T for the two 16-token tiles -------------------------
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sc[t] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            lds_ld128((kr0 ^ (64u * kk)) + 16 * t * kRowB), qf[kk], sc[t], 0,
            0, 0);
    }
    // ---- mask, bias, running max ----------------------------------------
    float x[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bool page_ok = (t == 0 ? st.phys0 : st.phys1) >= 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kpos = (st.pg + t) * kPS + 4 * g + i;
        const bool ok = page_ok && kpos >= lo && kpos < n;
        float v = sc[t][i] * a.scale_log2;
        if constexpr (REL) v += bf16_bits_to_f32(buf.rel[4 * t + i]) * kLog2e;
        v = ok ? v : -INFINITY;
        x[t][i] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx = lane_pair(lane_pair(mx, 16, true), 32, true);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    // ---- probabilities: fp32 sum, bf16 operand --------------------------
    // B-operand element j = 4t + i  <->  token 16t + 4g + i
    float psum = 0.0f;
    float p[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[t][i] = fast_exp2(x[t][i] - m_use);
        psum += p[t][i];
      }
    l_part = l_part * alpha + psum;
    uint32_t pw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      pw[j] = pack_bf16x2(f32_to_bf16_bits(p[j >> 1][2 * (j & 1)]),
                          f32_to_bf16_bits(p[j >> 1][2 * (j & 1) + 1]));
    const bf16x8 pf =
        __builtin_bit_cast(bf16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
    // ---- O^T = O^T * alpha + V^T.P^T ------------------------------------
    // A operand (dims 16 blk + r, tokens 4g..4g+3 and 16+4g..16+4g+3) by two
    // transposed reads: source lane s of each 16-lane group names token
    // base + (s >> 2) and dims 16 blk + 4 (s & 3)..+3
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const uint32_t va = vr0 ^ (32u * blk);
      const bf16x4 lo4 = lds_tr16(va);
      const bf16x4 hi4 = lds_tr16(va + 16 * kRowB);
      const bf16x8 vf = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
      o_acc[blk] = o_acc[blk] * alpha;
      o_acc[blk] =
          __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o_acc[blk], 0, 0, 0);
    }
  };

  // End of a piece of sequence b: write the result (whole sequence) or a
  // normalised partial that decode_combine_kernel merges.
  auto finish_piece = [&](const Step& st) {
    const int b = st.b;
    float l_tot = l_part;
    l_tot = lane_pair(lane_pair(l_tot, 16, false), 32, false);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const float lse_nat =
        l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : -INFINITY;
    // Buffer stores with a per-row (wave-uniform) base: the lane offsets
    // stay 32-bit, and padded heads / the LSE of lanes g != 0 / a missing
    // LSE output get an out-of-range offset or an empty resource (dropped),
    // so there is no divergent branch and no 64-bit address to keep live.
    const int s0 = st.s0, s1 = st.s1;
    const int bad = 0x7ffffff0;
    if (s0 >= u0 && s1 <= u1) {
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<char*>(a.out + (int64_t)b * a.HQ * kD), (short)0,
          a.HQ * kD * 2, 0x00020000);
      const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<char*>(a.lse ? a.lse + (int64_t)b * a.HQ : nullptr),
          (short)0, a.lse ? a.HQ * 4 : 0, 0x00020000);
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const uint32_t w0 =
            pack_bf16x2(f32_to_bf16_bits(o_acc[blk][0] * inv),
                        f32_to_bf16_bits(o_acc[blk][1] * inv));
        const uint32_t w1 =
            pack_bf16x2(f32_to_bf16_bits(o_acc[blk][2] * inv),
                        f32_to_bf16_bits(o_acc[blk][3] * inv));
        __builtin_amdgcn_raw_buffer_store_b64(
            u32x2{w0, w1}, ro,
            head_ok ? (hq * kD + 16 * blk + 4 * g) * 2 : bad, 0, 0);
      }
      __builtin_amdgcn_raw_buffer_store_b32(
          __builtin_bit_cast(uint32_t, lse_nat), rl,
          head_ok && g == 0 ? hq * 4 : bad, 0, 0);
    } else {
      // one piece of a longer sequence: slot b + wg is unique because
      // work-groups and sequences are both laid out in order
      const int64_t slot0 = (int64_t)(b + wg) * a.HQ;
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<char*>(a.part_o + slot0 * kD), (short)0,
          a.HQ * kD * 4, 0x00020000);
      const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<char*>(a.part_lse + slot0), (short)0, a.HQ * 4,
          0x00020000);
#pragma unroll
      for (int blk = 0; blk < 8; ++blk)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, o_acc[blk] * inv), ro,
            head_ok ? (hq * kD + 16 * blk + 4 * g) * 4 : bad, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(
          __builtin_bit_cast(uint32_t, lse_nat), rl,
          head_ok && g == 0 ? hq * 4 : bad, 0, 0);
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) o_acc[blk] = f32x4{0, 0, 0, 0};
    m_run = -INFINITY;
    l_part = 0.0f;
  };

  __syncthreads();  // every wave is done with the prefix table

  // ---- 4. software-pipelined walk: next step's loads fly during math ----
  // A ring of DEPTH step buffers: before step s is computed, the loads of
  // step s + DEPTH - 1 go out into the buffer step s - 1 used. Steps past
  // the range have no pages (zero-record resources: no memory traffic).
  StepBuf<REL> buf[DEPTH];
  Step stp[DEPTH];
#pragma unroll
  for (int k = 0; k < DEPTH - 1; ++k) {
    next_step(stp[k]);
    issue_step<REL>(buf[k], a, stp[k], lane_off, page_bytes, hq, head_ok, g);
  }
  for (;;) {
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) {
      const int f = (k + DEPTH - 1) % DEPTH;
      next_step(stp[f]);
      issue_step<REL>(buf[f], a, stp[f], lane_off, page_bytes, hq, head_ok, g);
      if (stp[k].b < 0) return;
      compute(buf[k], stp[k]);
      if (stp[k].last) finish_piece(stp[k]);
    }
  }
}

// Merge the pieces of every sequence that several work-groups shared:
// grid (B, ceil(HQ / 8)), 8 heads x 32 lanes per work-group, 4 dims per
// lane; pieces are merged in work-group order (deterministic, no atomics),
// eight pieces' loads in flight at a time (one round for the pieces of most
// sequences: the load latency, not the bytes, is what this kernel waits on).
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
  const int b = blockIdx.x;
  const int C = as_const(a.geo)[0];
  const int s0 = as_const(a.geo)[1 + b];
  const int s1 = as_const(a.geo)[2 + b];
  if (s1 <= s0) return;                  // no visible key: written already
  const int wfirst = s0 / C;
  const int np = (s1 - 1) / C - wfirst + 1;
  if (np <= 1) return;                   // one piece: written in place
  const int h = blockIdx.y * 8 + (threadIdx.x >> 5);
  if (h >= a.HQ) return;
  const int d0 = 4 * (threadIdx.x & 31);
  const int64_t slot0 = (int64_t)(b + wfirst) * a.HQ + h;
  float m = -INFINITY, sum = 0.0f;
  f32x4 acc = f32x4{0, 0, 0, 0};
  constexpr int kBatch = 8;
  for (int k = 0; k < np; k += kBatch) {
    float l4[kBatch];
    f32x4 o4[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const bool in = k + j < np;
      const int64_t slot = slot0 + (int64_t)(in ? k + j : 0) * a.HQ;
      l4[j] = in ? a.part_lse[slot] : -INFINITY;
      o4[j] = *reinterpret_cast<const f32x4*>(a.part_o + slot * kD + d0);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const float m_new = fmaxf(m, l4[j]);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float keep = fast_exp2((m - m_use) * kLog2e);
      const float w = fast_exp2((l4[j] - m_use) * kLog2e);
      sum = sum * keep + w;
      acc = acc * keep + o4[j] * w;
      m = m_new;
    }
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  __bf16* o = a.out + ((int64_t)b * a.HQ + h) * kD + d0;
  *reinterpret_cast<u32x2*>(o) =
      u32x2{pack_bf16x2(f32_to_bf16_bits(acc[0] * inv),
                        f32_to_bf16_bits(acc[1] * inv)),
            pack_bf16x2(f32_to_bf16_bits(acc[2] * inv),
                        f32_to_bf16_bits(acc[3] * inv))};
  if (a.lse && d0 == 0)
    a.lse[(int64_t)b * a.HQ + h] =
        sum > 0.0f ? (m == -INFINITY ? 0.0f : m) + fast_log2(sum) * kLn2
                   : -INFINITY;
}

int waves_per_wg(int HKV) { return HKV % 4 == 0 ? 4 : (HKV % 2 == 0 ? 2 : 1); }

// Three work-groups per four CUs (one wave per SIMD where they run):
// measured on MI355X, C2 / C3 decode stream fastest between 0.75 and 0.85
// work-groups per CU, 3-8 % ahead of one per CU and 10-20 % ahead of two.
int default_wgs(int HKV) {
  const int ny = HKV / waves_per_wg(HKV);
  const int g = 3 * device_cus() / (4 * ny);
  return g > 0 ? g : 1;
}

size_t ws_layout(int B, int HQ, int G, size_t* off_lse, size_t* off_geo) {
  const size_t slots = (size_t)B + G;
  const size_t o_bytes = slots * HQ * kD * sizeof(float);
  const size_t l_bytes = (slots * HQ * sizeof(float) + 255) & ~(size_t)255;
  const size_t g_bytes = (((size_t)B + 2) * sizeof(int) + 255) & ~(size_t)255;
  if (off_lse) *off_lse = o_bytes;
  if (off_geo) *off_geo = o_bytes + l_bytes;
  return o_bytes + l_bytes + g_bytes;
}

template <int REP, int KIND>
void launch_kind(const DecodeArgs& a, dim3 grid, int nw, size_t lds,
                 hipStream_t st) {
  if (a.rel)
    hipLaunchKernelGGL((decode_kernel<REP, true, kDeep, KIND>), grid,
                       dim3(64 * nw), lds, st, a);
  else
    hipLaunchKernelGGL((decode_kernel<REP, false, kDeep, KIND>), grid,
                       dim3(64 * nw), lds, st, a);
}

template <int REP>
void launch(const DecodeArgs& a, int G, int nw, size_t lds, hipStream_t st) {
  const dim3 grid(G, a.HKV / nw);
  if (a.bt_kind == 2) launch_kind<REP, 2>(a, grid, nw, lds, st);
  else launch_kind<REP, 0>(a, grid, nw, lds, st);
}

// ---- static scratch of the allocation-free entry point -------------------
// Device memory for tmopt_attn_decode_paged_noalloc's workspace: a fixed
// array in the library's code object, so the call needs no allocation.
// Every GPU the library runs on holds its own copy until the process ends.
constexpr size_t kScratchBytes = size_t(16) << 20;   // 16 MiB per GPU
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`. The array's
// name is a host-side stand-in in host code, never a device address: it is
// resolved here, once per device with that device current, and only the
// resolved address is passed to kernels.
int scratch_address(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  TMOPT_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices,
                TMOPT_ELAUNCH, "decode_noalloc: no current device (%s)",
                hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    TMOPT_REQUIRE(e == hipSuccess && p != nullptr, TMOPT_ELAUNCH,
                  "decode_noalloc: hipGetSymbolAddress failed on device %d: "
                  "%s", dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return TMOPT_OK;
}

// The block table of attn_global's per-token rows (model.py:938-945: flat
// [b, j] = table[b][j / 16] * 16 + j % 16 for live j, 0 past the length):
// table[b][i] = flat[b][16 i] / 16, and ctx_lens[b] = pos[b] + 1. One thread
// per table entry (entries of pages past a row's length are 0, never read).
__global__ __launch_bounds__(256) void table_from_flat_kernel(
    const int64_t* __restrict__ flat, int64_t Lg, const int64_t* __restrict__ pos,
    int npages, int32_t* __restrict__ table, int64_t table_stride,
    int32_t* __restrict__ ctx_lens) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < npages)
    table[(int64_t)b * table_stride + i] =
        (int32_t)(flat[(int64_t)b * Lg + (int64_t)kPS * i] / kPS);
  if (i == 0) ctx_lens[b] = (int32_t)(pos[b] + 1);
}

}  // namespace
}  // namespace tmopt

using namespace tmopt;

extern "C" int tmopt_attn_decode_default_workgroups(int HKV) {
  if (HKV <= 0) return 0;
  return default_wgs(HKV);
}

extern "C" size_t tmopt_attn_decode_workspace_size(int B, int HQ, int HKV,
                                                   int D, int num_workgroups) {
  (void)D;
  if (B <= 0 || HQ <= 0 || HKV <= 0) return 0;
  const int G = num_workgroups > 0 ? num_workgroups : default_wgs(HKV);
  return ws_layout(B, HQ, G, nullptr, nullptr);
}

// The decode launch behind both entry points: `kind` 0 = int32 block table
// + int32 lengths (block_table, ctx_lens), 2 = ring slots + int64 positions
// (rows64, pos64). (Per-token flat rows read in place, one page id per
// 128 bytes, measured 17% slower than an int32 table at B = 64: every
// page lookup missed the scalar cache ahead of the step's loads.)
static int decode_impl(
    int kind, const void* q, const void* k_pool, const void* v_pool,
    const int32_t* block_table, const int64_t* rows64, int64_t bt_stride,
    int table_wrap, const int32_t* ctx_lens, const int64_t* pos64, int B,
    int HQ, int HKV, int D, int page_size, int64_t num_pages, int window,
    float scale, const void* rel, int rel_extent, int min_pages,
    int num_workgroups, int seqs_per_wg, void* out, float* lse,
    void* workspace, size_t workspace_bytes, tmopt_stream_t stream) {
  if (B == 0) return TMOPT_OK;
  TMOPT_REQUIRE(B > 0, TMOPT_EINVAL, "decode: B=%d", B);
  TMOPT_REQUIRE(B <= kMaxB, TMOPT_EUNSUPPORTED, "decode: B=%d above %d", B,
                kMaxB);
  TMOPT_REQUIRE(q && k_pool && v_pool && out &&
                    (kind == 0 ? block_table && ctx_lens : rows64 && pos64),
                TMOPT_EINVAL, "decode: null tensor pointer");
  TMOPT_REQUIRE(D == kD, TMOPT_EUNSUPPORTED, "decode: D=%d (only 128)", D);
  TMOPT_REQUIRE(page_size == kPS, TMOPT_EUNSUPPORTED,
                "decode: page_size=%d (only 16)", page_size);
  TMOPT_REQUIRE(HKV > 0 && HQ > 0 && HQ % HKV == 0, TMOPT_EINVAL,
                "decode: HQ=%d HKV=%d", HQ, HKV);
  // Query heads per scheduled KV head: the whole ratio up to 16 (the MFMA
  // columns), else its largest divisor up to 16, the stored head then
  // scheduled kv_div times (each reading its pages once per group).
  const int ratio = HQ / HKV;
  int rep = ratio;
  while (rep > 16 || ratio % rep != 0) --rep;
  const int kv_div = ratio / rep;
  TMOPT_REQUIRE((int64_t)HKV * kv_div <= 65535, TMOPT_EUNSUPPORTED,
                "decode: HKV=%d x %d query-head groups exceeds 65535", HKV,
                kv_div);
  TMOPT_REQUIRE((int64_t)kPS * HKV * kD * 2 < (1ll << 31), TMOPT_EUNSUPPORTED,
                "decode: page too large");
  TMOPT_REQUIRE(num_pages > 0 && bt_stride > 0 && table_wrap >= 0 &&
                    (table_wrap == 0 || table_wrap <= bt_stride),
                TMOPT_EINVAL,
                "decode: num_pages=%lld bt_stride=%lld table_wrap=%d",
                (long long)num_pages, (long long)bt_stride, table_wrap);
  TMOPT_REQUIRE(window >= 0, TMOPT_EINVAL, "decode: window=%d", window);
  // a ring table holds the last table_wrap * 16 positions: a wider (or no)
  // window would read rows the ring has already overwritten
  TMOPT_REQUIRE(table_wrap == 0 ||
                    (window > 0 && (int64_t)window <= (int64_t)table_wrap * kPS),
                TMOPT_EINVAL, "decode: window=%d outside a ring of %d pages",
                window, table_wrap);
  TMOPT_REQUIRE(min_pages > 0 && num_workgroups >= 0, TMOPT_EINVAL,
                "decode: min_pages=%d num_workgroups=%d", min_pages,
                num_workgroups);
  TMOPT_REQUIRE(rel == nullptr || rel_extent > 0, TMOPT_EINVAL,
                "decode: rel_extent=%d", rel_extent);
  TMOPT_REQUIRE(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool |
                 (uintptr_t)out) % 16 == 0,
                TMOPT_EINVAL, "decode: tensors must be 16-byte aligned");
  const int G = num_workgroups > 0 ? num_workgroups : default_wgs(HKV);
  TMOPT_REQUIRE(G <= 65535, TMOPT_EINVAL, "decode: num_workgroups=%d", G);
  TMOPT_REQUIRE(seqs_per_wg >= 0 &&
                    (seqs_per_wg == 0 || (int64_t)seqs_per_wg * G >= B),
                TMOPT_EINVAL,
                "decode: %d work-groups of %d whole sequences do not cover "
                "B=%d",
                G, seqs_per_wg, B);
  size_t off_lse = 0, off_geo = 0;
  const size_t need = ws_layout(B, HQ, G, &off_lse, &off_geo);
  TMOPT_REQUIRE(workspace && workspace_bytes >= need &&
                    (uintptr_t)workspace % 16 == 0,
                TMOPT_EWORKSPACE,
                "decode: workspace %zu bytes < %zu needed (or unaligned)",
                workspace_bytes, need);

  DecodeArgs a;
  a.q = (const __bf16*)q;
  a.kpool = (const __bf16*)k_pool;
  a.vpool = (const __bf16*)v_pool;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.bt_width = bt_stride > 0x7fffffff ? 0x7fffffff : (int)bt_stride;
  a.table_wrap = table_wrap;
  a.ctx_lens = ctx_lens;
  a.bt_kind = kind;
  a.rows64 = rows64;
  a.pos64 = pos64;
  a.B = B;
  a.HQ = HQ;
  a.HKV = HKV * kv_div;
  a.rep = rep;
  a.kv_div = kv_div;
  a.HKV_stored = HKV;
  a.num_pages = num_pages > 0x7fffffff ? 0x7fffffff : (int)num_pages;
  a.window = window;
  a.scale_log2 = scale * kLog2e;
  a.rel = (const __bf16*)rel;
  a.rel_extent = rel ? rel_extent : 0;
  a.min_pages = min_pages;
  a.seqs_per_wg = seqs_per_wg;
  a.out = (__bf16*)out;
  a.lse = lse;
  a.part_o = (float*)workspace;
  a.part_lse = (float*)((char*)workspace + off_lse);
  a.geo = (int*)((char*)workspace + off_geo);

  const int nw = waves_per_wg(a.HKV);
  const size_t tab = ((size_t)B + 1 + 4) * sizeof(int);
  const size_t tiles = (size_t)nw * kWaveLds;
  const size_t lds = tab > tiles ? tab : tiles;
  hipStream_t st = (hipStream_t)stream;
  switch (kv_div == 1 ? rep : 0) {
    case 1: launch<1>(a, G, nw, lds, st); break;
    case 2: launch<2>(a, G, nw, lds, st); break;
    case 4: launch<4>(a, G, nw, lds, st); break;
    case 8: launch<8>(a, G, nw, lds, st); break;
    case 16: launch<16>(a, G, nw, lds, st); break;
    default: launch<0>(a, G, nw, lds, st); break;
  }
  int rc = check_launch("decode");
  if (rc || seqs_per_wg > 0) return rc;   // whole sequences: nothing to merge
  hipLaunchKernelGGL(decode_combine_kernel, dim3(B, (HQ + 7) / 8), dim3(256),
                     0, st, a);
  return check_launch("decode_combine");
}

extern "C" int tmopt_attn_decode_paged(
    const void* q, const void* k_pool, const void* v_pool,
    const int32_t* block_table, int64_t bt_stride, int table_wrap,
    const int32_t* ctx_lens, int B, int HQ, int HKV, int D, int page_size,
    int64_t num_pages, int window, float scale, const void* rel,
    int rel_extent, int min_pages, int num_workgroups, void* out, float* lse,
    void* workspace, size_t workspace_bytes, tmopt_stream_t stream) {
  clear_error();
  return decode_impl(0, q, k_pool, v_pool, block_table, nullptr, bt_stride,
                     table_wrap, ctx_lens, nullptr, B, HQ, HKV, D, page_size,
                     num_pages, window, scale, rel, rel_extent, min_pages,
                     num_workgroups, 0, out, lse, workspace, workspace_bytes,
                     stream);
}

extern "C" int tmopt_attn_decode_ring(
    const void* q, const void* k_pool, const void* v_pool,
    const int64_t* slots, int ring_pages, const int64_t* pos, int B, int HQ,
    int HKV, int D, int64_t num_pages, int window, float scale,
    const void* rel, int rel_extent, int min_pages, int num_workgroups,
    int seqs_per_workgroup, void* out, float* lse, void* workspace,
    size_t workspace_bytes, tmopt_stream_t stream) {
  clear_error();
  TMOPT_REQUIRE(ring_pages > 0, TMOPT_EINVAL, "decode_ring: ring_pages=%d",
                ring_pages);
  return decode_impl(2, q, k_pool, v_pool, nullptr, slots, ring_pages,
                     ring_pages, nullptr, pos, B, HQ, HKV, D, kPS, num_pages,
                     window, scale, rel, rel_extent, min_pages,
                     num_workgroups, seqs_per_workgroup, out, lse, workspace,
                     workspace_bytes, stream);
}

extern "C" int tmopt_attn_decode_paged_noalloc(
    const void* q, const void* k_pool, const void* v_pool,
    const int32_t* block_table, int64_t bt_stride, int table_wrap,
    const int32_t* ctx_lens, int B, int HQ, int HKV, int D, int page_size,
    int64_t num_pages, int window, float scale, const void* rel,
    int rel_extent, int min_pages, int num_workgroups, void* out, float* lse,
    tmopt_stream_t stream) {
  clear_error();
  if (B == 0) return TMOPT_OK;
  // the workspace this launch shape needs (0 for arguments the full entry
  // point rejects: it reports them)
  const size_t need =
      tmopt_attn_decode_workspace_size(B, HQ, HKV, D, num_workgroups);
  TMOPT_REQUIRE(need <= kScratchBytes, TMOPT_EWORKSPACE,
                "decode_noalloc: the launch needs %zu bytes of scratch, above "
                "the %zu-byte static buffer (use tmopt_attn_decode_paged with "
                "a workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != TMOPT_OK) return rc;
  return tmopt_attn_decode_paged(q, k_pool, v_pool, block_table, bt_stride,
                                 table_wrap, ctx_lens, B, HQ, HKV, D,
                                 page_size, num_pages, window, scale, rel,
                                 rel_extent, min_pages, num_workgroups, out,
                                 lse, ws, kScratchBytes, stream);
}

extern "C" int tmopt_decode_table_from_flat(const int64_t* flat, int64_t Lg,
                                            const int64_t* pos, int B,
                                            int32_t* block_table,
                                            int64_t bt_stride,
                                            int32_t* ctx_lens,
                                            tmopt_stream_t stream) {
  clear_error();
  if (B == 0) return TMOPT_OK;
  TMOPT_REQUIRE(B > 0 && B <= 65535 && Lg > 0, TMOPT_EINVAL,
                "table_from_flat: B=%d Lg=%lld", B, (long long)Lg);
  TMOPT_REQUIRE(flat && pos && block_table && ctx_lens, TMOPT_EINVAL,
                "table_from_flat: null pointer");
  const int64_t npages = (Lg + kPS - 1) / kPS;
  TMOPT_REQUIRE(npages <= 0x7fffffff && bt_stride >= npages, TMOPT_EINVAL,
                "table_from_flat: bt_stride=%lld < %lld pages",
                (long long)bt_stride, (long long)npages);
  hipLaunchKernelGGL(table_from_flat_kernel,
                     dim3((unsigned)((npages + 255) / 256), B), dim3(256), 0,
                     (hipStream_t)stream, flat, Lg, pos, (int)npages,
                     block_table, bt_stride, ctx_lens);
  return check_launch("table_from_flat");
}
