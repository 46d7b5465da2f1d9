// Varlen causal (optionally windowed) prefill attention on bf16 MFMA, gfx950.
//
// Replaces _attn_prefill_kernel (engine/pyengine/kernels/attn_prefill.py:
// 71-141): per tile the math is the reference's — score = q.k * scale,
// masked by causality (and the window on SWA layers) as a selection, fp32
// online softmax, probabilities rounded to bf16 for the P.V product
// (attn_prefill.py:134-135), fp32 accumulation, one bf16 rounding on store.
// What is different, and why (MI355X):
//
//  * Packed varlen runs (cu_seqlens) instead of a right-padded [B,H,T,D]
//    batch, and chunked prefill: query j of run i sits at position
//    prior_i + j, and the keys may come from the paged cache through the
//    block table (prior context + the run's own, already written, keys).
//  * GQA grouping. A work-group owns (run, KV head, block of 256/REP
//    queries) for all REP query heads of that KV head, i.e. 256 score rows:
//    every K/V tile staged in LDS is used by REP heads. Each of the 8 waves
//    owns one 32-row MFMA block (one head x 32 queries), two waves per SIMD.
//  * Transposed scores. S^T = K.Q^T (v_mfma_f32_32x32x16_bf16, keys on M,
//    queries on N) leaves one query per lane, so the running max needs one
//    cross-lane step (a lane-half swap) and the running sum stays
//    lane-local; P^T is then already the B operand of O^T = V^T.P^T, and
//    the rescale factor of every O^T element a lane holds is that lane's own.
//  * K and V tiles (64 keys) go from global memory straight into LDS
//    (buffer_load ... lds, 1 KB per instruction, no registers), row-major
//    with 256-byte rows and XOR swizzles chosen for the 64 LDS banks of
//    gfx950: K 16-byte chunks by row & 15, V 64-byte blocks by row & 3. K
//    fragments are single 16-byte reads, V^T fragments two transposed
//    reads (ds_read_b64_tr_b16); none of them conflict. Four LDS stages,
//    tiles issued three ahead.
//  * Ping-pong: waves 0-3 and 4-7 alternate, half a tile apart, between an
//    MFMA phase (P.V of a tile and the next tile's scores) and a softmax
//    phase, so that each SIMD has one wave on the matrix core and one on
//    the vector ALU most of the time.
//  * Tiles wholly outside the causal/window band are never visited; only
//    tiles that straddle the diagonal, the window start or the run end pay
//    for per-element masking.
//  * A 1-D grid walks the (KV head, run, query block) items in "levels":
//    level z holds query block nqb_max-1-z of every run that has one, so the
//    heaviest blocks (most keys) are dispatched first and the light ones
//    fill the tail. Empty (run, block) pairs are compacted away and the
//    items are dealt to the 8 XCDs in turn (the dispatcher sends work-group
//    i to XCD i % 8), with each KV head kept on its own XCDs: every XCD gets
//    an equal share of every level and only one KV head's keys pass through
//    its L2. A plain (head, run, block) grid maps runs to XCDs by index and
//    left half of the XCDs idle for half the launch on mixed lengths.
#include <type_traits>

#include "common.h"

namespace tmopt {
namespace {

constexpr int kD = 128;
constexpr int kBN = 64;                   // keys per tile
constexpr int kRowB = 256;                // K / V tile row in LDS (one key)
constexpr int kTileB = kBN * kRowB;       // 16384
constexpr int kStage = 2 * kTileB;        // K tile then V tile
constexpr int kNStage = 4;                // 128 KB of LDS per work-group
constexpr int kBiasB = 32 * 128;          // fused bias: 32 window rows per wave
constexpr int kPage = 16;                 // paged source: tokens per page
constexpr float kLazy = 8.0f;             // lazy-rescale threshold (log2)
constexpr int kRing = 4;                  // MFMA-phase fragment ring
// a buffer offset past every resource this kernel builds (their ranges are
// checked below 2^31 - 16 on the host): the load returns zeros
constexpr int kOob = 0x7ffffff0;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// raw buffer resource: base, byte range, dword 3 as for every buffer access
// in this library
// (all fields are wave-uniform; readfirstlane keeps them in scalar
// registers, as the instruction needs, even where the compiler computed a
// field with vector instructions)
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
               __builtin_amdgcn_readfirstlane(
                   (int)((uint32_t)(p >> 32) & 0xffffu)),
               __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// 16 bytes per lane from global memory straight into LDS: lane l of the
// wave writes bytes lds + 16 l .. +15. Issued from inline assembly so that
// the compiler does not wait for it at every barrier or before LDS reads it
// cannot prove disjoint from it; the kernel waits for these loads itself
// (wait_vm). The compiler's own waits for ordinary loads (the fused bias)
// do not count these: they wait for every DMA issued between the load and
// its use, so the tile loop issues no DMA in that stretch.
__device__ __forceinline__ void dma(i32x4 rsrc, uint32_t lds, int voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc)
      : "memory", "m0");
}

// 4 bytes per lane into LDS: lane l of the wave writes bytes lds + 4 l ..
// +3 (the fused bias's window rows; the same rules as dma())
__device__ __forceinline__ void dma32(i32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc)
      : "memory", "m0");
}

// wait until at most N vector-memory loads of this wave are in flight
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) |
                             (15 << 8));
}

struct PrefillArgs {
  const __bf16* q;
  int64_t q_st, q_sh;
  const __bf16* k;
  int64_t k_st, k_sh;
  const __bf16* v;
  int64_t v_st, v_sh;
  int64_t k_sd, v_sd;   // head_dim strides (1: token-major rows)
  int64_t k_sr, v_sr;   // run strides (0: run s starts at row cu[s])
  const int32_t* cu;
  const int32_t* prior;
  const __bf16* kpool;
  const __bf16* vpool;
  const int32_t* bt;
  int64_t bt_stride;
  int bt_width;      // entries a row may be read at: min(bt_stride, 2^31-1)
  int table_wrap;    // > 0: each table row is a ring of that many pages
  int num_pages;
  int page_size;
  int HQ;
  int HKV;           // KV heads as scheduled (virtual, see kv_div)
  int kv_div;        // scheduled KV heads per stored one: 1 unless HQ/HKV
                     // is not 1, 2, 4 or 8 (then each stored head serves
                     // kv_div groups of up to 8 query heads)
  int HKV_stored;    // KV heads of the k/v rows and the pools
  int window;
  float scale;
  float scale_log2;
  __bf16* out;
  int64_t o_st, o_sh;
  float* lse;        // [HQ, cu[S]]
  int S;
  int nqb_max;       // query blocks of the longest run
  const __bf16* rel; // optional fused relative bias, rows like q
  int64_t r_st, r_sh;
  int rel_extent;
  const int32_t* reject;  // optional device flag: nonzero = write NaN
};

// Sum over the wave, wave-uniform: within each 16-lane row by DPP (xor 1,
// xor 2, half-row mirror, row mirror: a few cycles each), then the four row
// sums by lane reads. (The schedule below takes ~10 of these per
// work-group; as ds_bpermute shuffles, 6 LDS round trips each, they cost
// microseconds of every work-group's start.)
__device__ __forceinline__ int wave_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // xor 1
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // xor 2
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // 7 - i
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // 15 - i
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// query blocks of run s (lane-varying s)
__device__ __forceinline__ int run_blocks(const PrefillArgs& a, int s,
                                          int BQ) {
  const int len = a.cu[s + 1] - a.cu[s];
  return (len + BQ - 1) / BQ;
}

// items of one KV head in levels [0, z): a run with nb blocks has one item
// on each level z' >= nqb_max - nb. nb0: blocks of run `lane` (0 past S).
__device__ __forceinline__ int items_before(const PrefillArgs& a, int z,
                                            int BQ, int lane, int nb0) {
  int c = max(0, nb0 - a.nqb_max + z);
  for (int s = lane + 64; s < a.S; s += 64)
    c += max(0, run_blocks(a, s, BQ) - a.nqb_max + z);
  return __builtin_amdgcn_readfirstlane(wave_sum(c));
}

struct Work {
  int kvh, seq, qb;    // seq < 0: nothing to do
  int t0, len, prior;  // the run's first row, length and prior context
  int total;           // cu[S]: rows of the launch (the LSE row length)
};

// Work item of this work-group (computed by every wave, identically).
// Work-group L runs on XCD L % 8 as the L/8-th one there. KV heads are
// spread over the XCDs (8 % HKV == 0: 8/HKV XCDs per head; HKV % 8 == 0:
// HKV/8 heads per XCD; otherwise round robin), and each head's items, in
// level order, are dealt to its XCDs in turn.
__device__ __forceinline__ Work schedule(const PrefillArgs& a, int BQ,
                                         int lane) {
  const int L = blockIdx.x;
  int kvh, i;
  if (a.HKV <= 8 && 8 % a.HKV == 0) {
    const int R = 8 / a.HKV;
    kvh = (L & 7) / R;
    i = (L >> 3) * R + (L & 7) % R;
  } else if (a.HKV % 8 == 0) {
    const int R = a.HKV / 8;
    kvh = (L & 7) + 8 * ((L >> 3) % R);
    i = (L >> 3) / R;
  } else {
    kvh = L % a.HKV;
    i = L / a.HKV;
  }
  Work w{kvh, -1, 0, 0, 0, 0, 0};
  // row start, end and prior context of the first 64 runs, one per lane:
  // the item's own values are then lane reads, not a second round trip to
  // memory after the search
  const int c0 = lane < a.S ? a.cu[lane] : 0;
  const int c1 = lane < a.S ? a.cu[lane + 1] : 0;
  const int p0 = a.prior != nullptr && lane < a.S ? a.prior[lane] : 0;
  const int nb0 = (c1 - c0 + BQ - 1) / BQ;
  const int total = items_before(a, a.nqb_max, BQ, lane, nb0);
  if (i >= total) return w;
  // level z: the last one with items_before(z) <= i
  int lo = 0, hi = a.nqb_max;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (items_before(a, mid, BQ, lane, nb0) <= i) lo = mid; else hi = mid;
  }
  int rem = i - items_before(a, lo, BQ, lane, nb0);
  const int need = a.nqb_max - lo;  // runs with at least this many blocks
  for (int s0 = 0; s0 < a.S; s0 += 64) {
    const int s = s0 + lane;
    const bool act =
        s < a.S && (s0 == 0 ? nb0 : run_blocks(a, s, BQ)) >= need;
    const uint64_t m = __builtin_amdgcn_ballot_w64(act);
    const int pop = __builtin_popcountll(m);
    if (rem < pop) {
      const int rank = __builtin_amdgcn_mbcnt_hi(
          (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      const uint64_t hit = __builtin_amdgcn_ballot_w64(act && rank == rem);
      const int sl = __builtin_ctzll(hit);
      w.seq = s0 + sl;
      w.qb = a.nqb_max - 1 - lo;
      if (s0 == 0) {
        w.t0 = __builtin_amdgcn_readlane(c0, sl);
        w.len = __builtin_amdgcn_readlane(c1, sl) - w.t0;
        w.prior = __builtin_amdgcn_readlane(p0, sl);
      } else {
        w.t0 = as_const(a.cu)[w.seq];
        w.len = as_const(a.cu)[w.seq + 1] - w.t0;
        w.prior = a.prior != nullptr ? as_const(a.prior)[w.seq] : 0;
      }
      w.total = a.S <= 64 ? __builtin_amdgcn_readlane(c1, a.S - 1)
                          : as_const(a.cu)[a.S];
      return w;
    }
    rem -= pop;
  }
  return w;  // not reached for i < total
}

// Where the keys of a run come from.
enum Source : int {
  kPacked = 0,  // the run's own rows of packed k / v (no prior context)
  kPaged = 1,   // every key, prior and own, from the page pools
  kMixed = 2,   // keys before prior_lens[i] from the pools (or a ring of
                // pages), the run's own keys from packed k / v
  kPackedCM = 3,  // kPacked with channel-major k / v: tokens contiguous,
                  // head_dim strided (the sconv output), read in place
};

// Channel-major tiles in LDS are 128 dim rows of 64 keys (128 bytes, eight
// 16-byte chunks of 8 keys). Row r keeps logical chunk c in physical slot
// c ^ cm_sig(r). cm_sig is a bijection of (r >> 1) & 7 that flips bit 2
// between rows 4m and 4m + 2, so that
//  * 16 consecutive rows reading one chunk (V^T fragments: a 16-lane group)
//    hit 16 distinct 16-byte bank groups (8 slots x row parity), and
//  * 4 consecutive rows reading an aligned group of 4 chunks (K fragments
//    by transposed reads: a half wave) hit 16 distinct ones as well.
__device__ __forceinline__ int cm_sig(int r) {
  const int x = (r >> 1) & 7;
  return ((x & 1) << 2) | (x >> 1);
}

template <int REP, bool REL, int SRC>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
  constexpr bool CM = SRC == kPackedCM;   // channel-major k / v tiles
  constexpr bool POOL = SRC == kPaged || SRC == kMixed;  // keys from pools
  constexpr bool OWN = SRC != kPaged;     // the run's keys from packed k/v
  constexpr int BQ = 256 / REP;   // queries per work-group
  constexpr int QSUB = BQ / 32;   // 32-query sub-blocks per head
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // 8 waves, one 32-row block each (wave index kept in a scalar register)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int h2 = lane >> 5;       // lane half
  const Work wk = schedule(a, BQ, lane);
  if (wk.seq < 0) return;
  const int kvh = wk.kvh;
  const int kvs = kvh / a.kv_div;   // the stored KV head its keys come from
  const int seq = wk.seq;
  const int qb = wk.qb;

  const int t0 = wk.t0;
  const int len = wk.len;
  const int q0 = qb * BQ;
  const int prior = wk.prior;
  const int nk = prior + len;                 // keys of this run
  const int qn = min(BQ, len - q0);
  const int pos_lo = prior + q0;              // first query position
  const int pos_hi = prior + q0 + qn - 1;     // last valid query position
  // first key any query of the block may see; tiles start at a multiple of
  // the tile width below it
  const int kwin = a.window > 0 ? max(0, pos_lo - a.window + 1) : 0;
  const int k_lo = (kwin / kBN) * kBN;
  const int k_hi = pos_hi + 1;                // exclusive
  const int ntiles = (k_hi - k_lo + kBN - 1) / kBN;

  // ---- this wave's row block: head and 32-query sub-block ----------------
  const int head = kvh * REP + w / QSUB;
  const int qi = q0 + 32 * (w % QSUB) + l32;  // this lane's query (column)
  const bool qok = qi < len;
  const int qpos = prior + qi;

  // ---- Q fragments: B operand of S^T (column = query, k = dims) --------
  bf16x8 qf[8];   // loaded through LDS in the prologue below

  // ---- tile loads: global -> LDS directly (buffer_load ... lds) ----------
  // Wave w moves key rows 4w..4w+3 and 32+4w..32+4w+3 of the K and the V
  // tile: one 1 KB instruction per 4 rows, lane l writing LDS bytes
  // 16l..16l+15 of the 4-row block, i.e. row l>>4, physical 16-byte slot
  // l&15. The lane fetches the logical chunk that belongs in that slot:
  // K: slot c ^ (row & 15); V: 64-byte block b ^ (row & 3).
  // Rows past the run end (and pages outside the pool) fall outside the
  // buffer resource and arrive as zeros; tile offsets ride in the lane
  // offset, which is what the hardware range-checks.
  const int grp = lane >> 4, slot = lane & 15;
  const int kchunk = slot ^ ((4 * w + grp) & 15);
  const int vchunk = ((((slot >> 2) ^ grp) & 3) << 2) | (slot & 3);
  // LDS byte address of the dynamic shared block (0 here: the kernel has
  // no static LDS), a multiple of 256 as the fragment addressing assumes
  const uint32_t lds0 =
      (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)smem);
  // packed rows of the run (keys 0.. of the run itself)
  i32x4 rk = make_rsrc(nullptr, 0u), rv = make_rsrc(nullptr, 0u);
  int kst_b = 0, vst_b = 0, klane_p = 0, vlane_p = 0;
  [[maybe_unused]] int cm_key = 0;
  if constexpr (OWN) {
    // the run's first row: at row cu[s] of the packed rows, or at s times
    // the run stride (a padded batch read in place)
    const int64_t k0 = a.k_sr != 0 ? (int64_t)seq * a.k_sr
                                   : (int64_t)t0 * a.k_st;
    const int64_t v0 = a.v_sr != 0 ? (int64_t)seq * a.v_sr
                                   : (int64_t)t0 * a.v_st;
    if constexpr (CM) {
      // 128 dim rows of the run's keys, a.k_sd elements apart: wave w
      // moves dim rows 8w..8w+7 and 64+8w..64+8w+7 of the K and the V
      // tile, lane l row l >> 3, physical slot l & 7, i.e. logical chunk
      // (l & 7) ^ cm_sig(row) (the same for both blocks: their rows differ
      // by 64). Chunks starting at or past the run end take an offset
      // outside the resource and arrive as zeros.
      kst_b = (int)(a.k_sd * 2);
      vst_b = (int)(a.v_sd * 2);
      rk = make_rsrc(a.k + k0 + (int64_t)kvs * a.k_sh,
                        (uint32_t)(((int64_t)(kD - 1) * a.k_sd + len) * 2));
      rv = make_rsrc(a.v + v0 + (int64_t)kvs * a.v_sh,
                        (uint32_t)(((int64_t)(kD - 1) * a.v_sd + len) * 2));
      const int r = 8 * w + (lane >> 3);
      const int c = (lane & 7) ^ cm_sig(r);
      cm_key = 8 * c;
      klane_p = r * kst_b + 2 * cm_key;
      vlane_p = r * vst_b + 2 * cm_key;
    } else {
      kst_b = (int)(a.k_st * 2);
      vst_b = (int)(a.v_st * 2);
      rk = make_rsrc(a.k + k0 + (int64_t)kvs * a.k_sh,
                        (uint32_t)(((int64_t)(len - 1) * a.k_st + kD) * 2));
      rv = make_rsrc(a.v + v0 + (int64_t)kvs * a.v_sh,
                        (uint32_t)(((int64_t)(len - 1) * a.v_st + kD) * 2));
      klane_p = grp * kst_b + 16 * kchunk;
      vlane_p = grp * vst_b + 16 * vchunk;
    }
  }
  // pool rows: keys below `plim` (all keys on the paged source, the prior
  // context on the mixed one)
  [[maybe_unused]] const int row_b = a.HKV_stored * kD * 2;   // one token row
  [[maybe_unused]] const int64_t page_b = (int64_t)kPage * row_b;
  [[maybe_unused]] int klane = 0, vlane = 0;
  if constexpr (POOL) {
    klane = grp * row_b + kvs * (kD * 2) + 16 * kchunk;
    vlane = grp * row_b + kvs * (kD * 2) + 16 * vchunk;
  }
  [[maybe_unused]] const int32_t __attribute__((address_space(4)))* trow =
      POOL ? as_const(a.bt) + (int64_t)seq * a.bt_stride : nullptr;
  [[maybe_unused]] const int plim = SRC == kMixed ? prior : nk;

  // Four pool rows key0..key0+3 (one page: key0 % 4 == 0) into LDS. The
  // buffer resource covers only the page's rows in [kwin, plim): rows before
  // the first key a query of the block may see and rows past the pool's
  // part read as zeros and are never fetched (a ring page there holds an
  // overwritten position, a windowed table may point it at a poison page),
  // and so does a page whose table entry lies outside the pool or past the
  // row's width. The lane offset is relative to the resource base, so the
  // rows below it have negative offsets, i.e. out of range.
  // (live == false: the same instructions with an offset past every
  // resource, so nothing is fetched and the stage gets zeros)
  auto pool_dma = [&](int key0, uint32_t dk, uint32_t dv, bool live) {
    if constexpr (POOL) {
      const int lp = key0 >> 4;
      const int col = a.table_wrap > 0 ? lp % a.table_wrap : lp;
      const int pg = (unsigned)col < (unsigned)a.bt_width ? trow[col] : -1;
      const int r_lo = min(kPage, max(0, kwin - kPage * lp));
      const int r_hi = min(kPage, max(0, plim - kPage * lp));
      const bool valid = (unsigned)pg < (unsigned)a.num_pages && r_hi > r_lo;
      const uint32_t nrec = valid ? (uint32_t)((r_hi - r_lo) * row_b) : 0u;
      const int64_t pofs = valid ? (int64_t)pg * page_b + r_lo * row_b : 0;
      const int roff = ((key0 & (kPage - 1)) - r_lo) * row_b;
      dma(make_rsrc(reinterpret_cast<const char*>(a.kpool) + pofs,
                            nrec),
               dk, live ? klane + roff : kOob);
      dma(make_rsrc(reinterpret_cast<const char*>(a.vpool) + pofs,
                            nrec),
               dv, live ? vlane + roff : kOob);
    }
  };
  // four packed rows j..j+3 of the run's own keys into LDS (rows past the
  // run end are outside the resource: zeros)
  auto own_dma = [&](int j, uint32_t dk, uint32_t dv, bool live) {
    if constexpr (OWN) {
      dma(rk, dk, live ? klane_p + j * kst_b : kOob);
      dma(rv, dv, live ? vlane_p + j * vst_b : kOob);
    }
  };

  // issue tile `t` (index from k_lo) into LDS stage `st`: 4 instructions
  // per wave (2 with the source split inside a 4-row block: one per source,
  // each under the exec mask of the lanes whose row it holds). live ==
  // false issues the same instructions fetching nothing: the loops issue a
  // tile every iteration, past the last one too, so that the wave's count
  // of loads in flight is the same on every path and the waits at the end
  // of the odd slots are exact.
  auto issue_tile = [&](int t, int st, bool live = true) {
    const int kt = k_lo + t * kBN;
    const uint32_t sb = lds0 + st * kStage;
    if constexpr (CM) {
      // dim rows 8w.. and 64+8w.. of the channel-major tile (see above)
      const bool in = live && kt + cm_key < len;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t dk = sb + (w + 8 * i) * 1024, dv = dk + kTileB;
        dma(rk, dk, in ? klane_p + 64 * i * kst_b + 2 * kt : kOob);
        dma(rv, dv, in ? vlane_p + 64 * i * vst_b + 2 * kt : kOob);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r0 = 4 * w + 32 * i;          // first row of the block
        const uint32_t dk = sb + r0 * kRowB, dv = dk + kTileB;
        const int key0 = kt + r0;
        if constexpr (SRC == kPacked) {
          own_dma(key0, dk, dv, live);
        } else if constexpr (SRC == kPaged) {
          pool_dma(key0, dk, dv, live);
        } else {
          if (key0 + 4 <= plim) {
            pool_dma(key0, dk, dv, live);
          } else if (key0 >= plim) {
            own_dma(key0 - plim, dk, dv, live);
          } else {
            // lane group grp holds row key0 + grp
            if (key0 + grp < plim) pool_dma(key0, dk, dv, live);
            else own_dma(key0 - plim, dk, dv, live);
          }
        }
      }
    }
  };

  // ---- LDS fragment addresses -------------------------------------------
  // K fragment (kb, kk) of lane (l32, h2): row 32 kb + l32, logical chunk
  // 2 kk + h2 -> slot (2 kk + h2) ^ (l32 & 15) = (h2 ^ (l32 & 15)) ^ 2 kk.
  const uint32_t ka0 = (uint32_t)(l32 * kRowB + 16 * (h2 ^ (l32 & 15)));
  // V^T fragment (db, kb, kk) by two transposed reads: within each 16-lane
  // group, source lane s names key kbase + (s >> 2), dims 4 (s & 3)..+3 of
  // a 16-dim half; lane i of the group then holds dim dbase + i of keys
  // kbase..kbase+3. kbase = 32 kb + 16 kk + 4 h2 (+8 for the second read),
  // dbase = 32 db + 16 (l32 >> 4), which matches the order of this lane's
  // probabilities (keys 16 kk + 4 h2 + 0..3 and 16 kk + 8 + 4 h2 + 0..3).
  const int s16 = lane & 15;
  const uint32_t va0 = (uint32_t)((4 * h2 + (s16 >> 2)) * kRowB +
                                  64 * (s16 >> 2) + 32 * ((lane >> 4) & 1) +
                                  8 * (s16 & 3));

  // Channel-major tiles (dim rows of 64 keys, slots swizzled by cm_sig):
  // the K fragment (kb, kk) takes two transposed reads, each giving lane i
  // of a 16-lane group dims dbase..dbase+3 of key kbase + i: source lane s
  // names dim row dbase + (s >> 2) and keys kbase + 4 (s & 3)..+3, with
  // kbase = 32 kb + 16 (g & 1) and dbase = 16 kk + 8 (g >> 1) (+4 for the
  // second read), g = lane >> 4. Rows 16 kk + r share cm_sig(r), so kk and
  // kb only move the address by 2048 kk and flip the chunk bit 2 (64 kb).
  // The V^T fragment (db, kb, kk) is two 8-byte reads of dim row
  // 32 db + l32: keys 32 kb + 16 kk + 4 h2 + 0..3 (logical chunk 4 kb + 2 kk,
  // half h2) and the same 8 keys on (chunk 4 kb + 2 kk + 1), the order of
  // this lane's probabilities.
  [[maybe_unused]] uint32_t cka[2] = {0u, 0u};
  [[maybe_unused]] uint32_t cva = 0u;
  if constexpr (CM) {
    const int g = lane >> 4;
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
      const int r = 8 * (g >> 1) + 4 * rd + (s16 >> 2);
      const int c = 2 * (g & 1) + ((s16 & 3) >> 1);
      cka[rd] = (uint32_t)(r * 128 + 16 * (c ^ cm_sig(r)) + 8 * (s16 & 1));
    }
    cva = (uint32_t)(l32 * 128 + 16 * cm_sig(l32) + 8 * h2);
  }

  // K fragment (kb, kk) of the tile whose K rows start at LDS byte kt_b
  auto kfrag = [&](uint32_t kt_b, int kb, int kk) -> bf16x8 {
    if constexpr (CM) {
      const uint32_t p = kt_b + 2048u * kk;
      const bf16x4 lo = lds_tr16((p + cka[0]) ^ (64u * kb));
      const bf16x4 hi = lds_tr16((p + cka[1]) ^ (64u * kb));
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      return lds_ld128(((kt_b + ka0) ^ (32u * kk)) + 32 * kb * kRowB);
    }
  };

  // S^T = K.Q^T for the tile in `stage` (keys on M, queries on N)
  // (with the fused bias, s already holds the tile's bias / scale)
  auto scores = [&](int stage, f32x16 (&s)[2]) {
    const uint32_t kt_b = lds0 + stage * kStage;
    if constexpr (!REL) {
      s[0] = f32x16{};
      s[1] = f32x16{};
    }
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf = kfrag(kt_b, kb, kk);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0,
                                                        0, 0);
      }
  };

  // V^T fragment (db, kb, kk) of the tile whose V rows start at LDS byte
  // vt_b
  auto vfrag = [&](uint32_t vt_b, int db, int kb, int kk) -> bf16x8 {
    if constexpr (CM) {
      const uint32_t p = vt_b + cva + 4096u * db;
      const uint32_t c = 4 * kb + 2 * kk;
      const u32x2 lo = lds_ld64(p ^ (16u * c));
      const u32x2 hi = lds_ld64(p ^ (16u * (c + 1)));
      return __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
    } else {
      const uint32_t p =
          ((vt_b + va0) ^ (64u * db)) + (32 * kb + 16 * kk) * kRowB;
      const bf16x4 lo = lds_tr16(p);
      const bf16x4 hi = lds_tr16(p + 8 * kRowB);
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };

  // Fused bias rows of this wave's 32 queries: one buffer resource from
  // the first query's row (lane offsets: row l32, 32-bit), covering the
  // rows of the run only, so reads past them return zeros.
  // (The resource starts at the dword holding that row's first value and
  // ends at the dword holding the last row's last value, so that the dword
  // loads below are aligned whatever the strides and every dword holding a
  // value of the rows is in range.)
  const int rel_row0 = q0 + 32 * (w % QSUB);
  const int rel_nrow = REL ? min(32, len - rel_row0) : 0;
  const char* const rel_first =
      REL ? reinterpret_cast<const char*>(a.rel + (int64_t)(t0 + rel_row0) *
                                                      a.r_st +
                                          (int64_t)head * a.r_sh)
          : nullptr;
  const int rel_mis = (int)((uintptr_t)rel_first & 3);   // 0 or 2
  [[maybe_unused]] const __amdgpu_buffer_rsrc_t rrel =
      __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(rel_first - rel_mis), (short)0,
          rel_nrow > 0 ? ((int)(((int64_t)(rel_nrow - 1) * a.r_st +
                                 a.rel_extent) * 2) + rel_mis + 3) & ~3
                       : 0,
          0x00020000);
  [[maybe_unused]] const int rrow_b =
      REL ? rel_mis + l32 * (int)(a.r_st * 2) : 0;

  // The fused bias of a key tile enters as the initial value of its score
  // accumulators, bias / scale (zero outside the band), so that the tile's
  // softmax is the plain one. The lane's keys come in runs of four
  // (key0 .. key0+3, dist d0 .. d0-3), whose four bf16 values are adjacent
  // in the row: the three dwords from the one holding rel[d0-3], realigned
  // by the lane's byte shift rel_sh.
  // Every tile goes through LDS (the first one with the first K/V tiles,
  // a later one one MFMA phase ahead): each wave copies the 64-key window
  // of each of its 32 rows (dists q-kt-63 .. q-kt, 32 dwords from the one
  // holding rel[q-kt-63]; a row whose values start mid-dword takes the 32
  // dwords from q-kt-64 and so lacks rel[q-kt]) into its 4 KB of LDS, two
  // rows per 4-byte-per-lane DMA, and reads its runs back from there: 16
  // DMAs that touch the rows' own lines instead of 8 loads that each touch
  // 32 rows. Rows 2m and 2m+1 take the 256 bytes of DMA m, with dword j of
  // the window in slot j ^ 2m: the 32 rows' reads of one dword pair then
  // fall on 32 distinct bank pairs (plain rows, 128 bytes apart, would put
  // all 32 on two). A lane reads the first two dwords of each run (one
  // 8-byte read); the third is the first of another lane's run on the same
  // row (the low half's comes from the high half's previous run, the high
  // half's from the low half's same run), swapped across the lane halves.
  // The value a mid-dword row lacks, the third dword of the low half's
  // first run, is the first dword of the previous tile's window (`carry`,
  // the high half's last run; for the first tile, one load). The range
  // check is per dword and the resource ends at a dword boundary, so every
  // value of the rows arrives; dwords before a row or past the run read as
  // zeros or as a neighbouring row's values, which lie outside the band
  // and are dropped.
  typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
  [[maybe_unused]] uint32_t carry = 0;
  [[maybe_unused]] const uint32_t bb =
      lds0 + kNStage * kStage + (uint32_t)w * kBiasB;
  [[maybe_unused]] const i32x4 rrel_s = make_rsrc(
      rel_first - rel_mis,
      rel_nrow > 0 ? (uint32_t)(((((int64_t)(rel_nrow - 1) * a.r_st +
                                   a.rel_extent) * 2) + rel_mis + 3) & ~3)
                   : 0u);
  // DMA i (rows 2i and 2i+1 of the wave): lane l fills slot l & 31 of row
  // 2i + (l >> 5), i.e. dword (l & 31) ^ 2i of its window; its byte offset
  // is dma_b + i * dma_s + ((4 (l & 31)) ^ 8i) - 2 kt
  [[maybe_unused]] uint32_t dma_b = 0, dma_s = 0, dma_c = 0;
  // LDS byte address of the lane's row with its swizzle and lane half
  // folded in: dword j ^ 2 h2 of the window sits at bias_a ^ 4j
  [[maybe_unused]] uint32_t bias_a = 0;
  if constexpr (REL) {
    const int hl = lane >> 5;
    const int x0 = rel_mis + hl * (int)(a.r_st * 2) +
                   2 * (prior + rel_row0 + hl - 63);
    dma_b = (uint32_t)(x0 - (x0 & 2));
    dma_s = (uint32_t)(4 * a.r_st + 4);
    dma_c = 4u * (uint32_t)(lane & 31);
    bias_a = (bb + 256u * (uint32_t)(l32 >> 1) + 128u * (uint32_t)(l32 & 1)) |
             (8u * (uint32_t)((l32 >> 1) ^ h2));
  }
  // the first tile's carry: the dword after its window (the first of the
  // window one tile before), loaded with the first tiles
  [[maybe_unused]] auto bias_carry0 = [&] {
    if constexpr (REL) {
      const int x = rel_mis + l32 * (int)(a.r_st * 2) +
                    2 * (prior + rel_row0 + l32 - 63);
      int off = x - (x & 2) - 2 * k_lo + 128;
      asm volatile("" : "+v"(off));
      carry = __builtin_amdgcn_raw_buffer_load_b32(rrel, off, 0, 0);
    }
  };
  // a tile's windows, into LDS (always 16 DMAs; a tile neither in
  // the band nor just before it, or past the run, fetches nothing)
  [[maybe_unused]] auto bias_dma_base = [&](int kt) {
    const bool live = kt < k_hi && pos_lo - (kt + 2 * kBN - 1) < a.rel_extent;
    uint32_t b = live ? dma_b - 2u * (uint32_t)kt : (uint32_t)kOob;
    asm volatile("" : "+v"(b));
    return b;
  };
  [[maybe_unused]] auto bias_dma_one = [&](uint32_t b, int i) {
    dma32(rrel_s, bb + 256 * i, b + i * dma_s + (dma_c ^ (8u * i)));
  };
  [[maybe_unused]] auto bias_dma = [&](int kt) {
    if constexpr (REL) {
      const uint32_t b = bias_dma_base(kt);
#pragma unroll
      for (int i = 0; i < 16; ++i) bias_dma_one(b, i);
    }
  };
  // the runs of the tile whose windows are in LDS
  [[maybe_unused]] auto bias_read = [&](u32x3 (&x)[8]) {
    if constexpr (REL) {
      // run r = 4 kb + g: dword 30 - 4 r - 2 h2 of the row's window holds
      // rel[d0-3]
      u32x2 lo[8];
#pragma unroll
      for (int r = 0; r < 8; ++r)
        lo[r] = lds_ld64(bias_a ^ (4u * (uint32_t)(30 - 4 * r)));
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        // the low half takes the high half's lo[r-1][0] (dword 32 - 4 r,
        // for r = 0 the carry), the high half the low half's lo[r][0]
        const auto sw = __builtin_amdgcn_permlane32_swap(
            r == 0 ? carry : lo[r - 1][0], lo[r][0], false, false);
        x[r] = u32x3{lo[r][0], lo[r][1], (uint32_t)(h2 ? sw[0] : sw[1])};
      }
      carry = lo[7][0];
    }
  };
  // Byte shift that realigns a lane's runs: the same on every tile (tile
  // starts are multiples of 64 keys, so only the row's parity matters).
  [[maybe_unused]] const uint32_t rel_sh =
      REL ? (uint32_t)((rrow_b + 2 * (qpos - 3)) & 3) : 0u;
  // The score accumulators of a bias tile start at rel[q, h, dist] / scale
  // for 0 <= dist < E, zero outside (the softmax multiplies by scale).
  // FAST (no band test: a byte permute and a multiply per score) serves
  // every tile whose scores outside the band are all masked anyway: a
  // window no wider than the band (dist >= W is masked), or a tile whose
  // dists stay below E for every query (dist < 0 is masked by causality);
  // the value it leaves in a masked score is never used. The checked path
  // (a tile across dist = E without such a window) zeroes the bias outside
  // [0, E) per score.
  [[maybe_unused]] const float inv_scale = REL ? 1.0f / a.scale : 0.0f;
  [[maybe_unused]] const bool band_masked =
      a.window > 0 && a.window <= a.rel_extent;
  // the band's width for this lane's query (0 past the run end)
  [[maybe_unused]] const uint32_t e_q = qok ? (uint32_t)a.rel_extent : 0u;
  // byte selectors (v_perm) that turn a run's dwords y0, y1, y2 into fp32
  // values (bf16 in the high half, zeros below): with shift 0 the values
  // are y1.hi, y1.lo, y0.hi, y0.lo, with shift 2 y2.lo, y1.hi, y1.lo, y0.hi;
  // SEL_A picks the high half of the low dword of a pair (0) or the low
  // half of its high dword (2), SEL_B the low (0) or high (2) half of one
  [[maybe_unused]] const uint32_t sel_a = rel_sh ? 0x05040c0cu : 0x03020c0cu;
  [[maybe_unused]] const uint32_t sel_b = rel_sh ? 0x03020c0cu : 0x01000c0cu;
  [[maybe_unused]] auto bias_init = [&](f32x16 (&s)[2], int kt,
                                        const u32x3 (&x)[8], auto fast_c) {
    constexpr bool fast = decltype(fast_c)::value;
    if constexpr (REL) {
      // dist of the lane's first key for kb = g = 0 (opaque to the
      // compiler, so that the runs' dists derive from it here instead of
      // being hoisted out of the key loop as registers of their own)
      int dq = qpos - kt - 4 * h2;
      asm volatile("" : "+v"(dq));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = dq - 32 * kb - 8 * g;
          const uint32_t x0 = x[4 * kb + g][0], x1 = x[4 * kb + g][1],
                         x2 = x[4 * kb + g][2];
          const uint32_t y0 = x0, y1 = x1, y2 = x2;
          // element 4g + i is key0 + i, dist d0 - i
          const uint32_t hv[4] = {__builtin_amdgcn_perm(y2, y1, sel_a),
                                  __builtin_amdgcn_perm(y1, y1, sel_b),
                                  __builtin_amdgcn_perm(y1, y0, sel_a),
                                  __builtin_amdgcn_perm(y0, y0, sel_b)};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float bias = __builtin_bit_cast(float, hv[i]);
            if constexpr (!fast)   // 0 <= dist < E, one unsigned compare
              bias = (uint32_t)(d0 - i) < e_q ? bias : 0.0f;
            s[kb][4 * g + i] = bias * inv_scale;
          }
        }
    }
  };

  // per-element mask: causal, window, run end. Element j of block kb holds
  // key kt + 4 h2 + c with c = 32 kb + 8 (j >> 2) + (j & 3), a compile-time
  // constant, and the keys a query sees form one interval lo < c <= hi per
  // lane: two compares and a select per score.
  auto mask_tile = [&](f32x16 (&s)[2], int kt) {
    const int base = kt + 4 * h2;
    const int hi = qok ? min(qpos, nk - 1) - base : -1;
    const int lo = a.window > 0 ? qpos - a.window - base : -1;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int c = 32 * kb + 8 * (j >> 2) + (j & 3);
        s[kb][j] = (c <= hi && c > lo) ? s[kb][j] : -INFINITY;
      }
  };

  // ---- accumulators -----------------------------------------------------
  f32x16 o_acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o_acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_part = 0.0f;
  // The max runs on the raw scores (scale > 0 commutes with max; with the
  // fused bias they hold q.k + bias / scale) and each probability is one
  // fma + exp2: p = 2^(s*scale*log2e - m).

  // Lazy rescaling: the running max (log2 domain) only moves when the
  // tile's max exceeds it by more than kLazy, so probabilities stay below
  // 2^kLazy and O^T / l are rescaled on few tiles; O / l and the LSE are
  // exact for any reference point.
  auto new_max = [&](float mx, float sl2, bool& move, float& m_use) {
    const auto sw = __builtin_amdgcn_permlane32_swap(
        __builtin_bit_cast(uint32_t, mx), __builtin_bit_cast(uint32_t, mx),
        false, false);
    mx = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]),
               __builtin_bit_cast(float, (uint32_t)sw[1]));
    const float m_cand = mx * sl2;
    move = m_cand > m_run + kLazy;
    const float m_new = move ? m_cand : m_run;
    m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = move ? fast_exp2(m_run - m_use) : 1.0f;
    m_run = m_new;
    return alpha;
  };
  // probability pair q (kb = q >> 3, kk = (q >> 2) & 1, e = q & 3)
  auto prob_pair = [&](const f32x16 (&s)[2], int q, float sl2, float m_use,
                       float& psum) {
    const int kb = q >> 3, kk = (q >> 2) & 1, e = q & 3;
    const float p0 =
        fast_exp2(__builtin_fmaf(s[kb][8 * kk + 2 * e], sl2, -m_use));
    const float p1 =
        fast_exp2(__builtin_fmaf(s[kb][8 * kk + 2 * e + 1], sl2, -m_use));
    psum += p0 + p1;
    return pack_bf16x2_rn(p0, p1);
  };
  auto pack_p = [&](const uint32_t (&pw)[16], bf16x8 (&pf)[2][2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int q = 8 * kb + 4 * kk;
        pf[kb][kk] = __builtin_bit_cast(
            bf16x8, u32x4{pw[q], pw[q + 1], pw[q + 2], pw[q + 3]});
      }
  };

  // ---- two wave groups in ping-pong ---------------------------------------
  // Waves 0-3 and 4-7 (one of each per SIMD) alternate between an MFMA
  // phase (P.V of tile t and the scores of tile t+1: 32 MFMAs, fragment
  // reads, hardly any VALU) and a softmax phase (the online softmax of those
  // scores: VALU only), half a tile apart: while one wave of a SIMD keeps
  // the matrix core busy the other one uses the vector ALU. A work-group
  // barrier ends every odd slot (and, in the bias build, every phase);
  // group 1 runs one phase behind group 0 (its first softmax shares the
  // slot of group 0's first multiply), and both pass the same barriers in
  // the same order.
  const int grp_id = w >> 2;
  // A tile every valid query of the block sees whole. Query columns past
  // the run end (a partial last block) are left unmasked there: their Q
  // fragments are zero, so their scores are finite, and their rows are
  // never stored (masking them sent every tile of such a block down the
  // masked path, at about twice the cost per tile).
  auto full_tile = [&](int kt) {
    return (kt + kBN - 1 <= pos_lo) && (kt + kBN <= nk) &&
           (a.window == 0 || pos_hi - kt < a.window);
  };
  f32x16 sc[2];        // scores of the tile after the one being multiplied
  bf16x8 pf[2][2];     // probabilities of the tile being multiplied

  // The bias of the tile at kt into its score accumulators, from its
  // windows in LDS, whose DMAs were followed by 4 tile DMAs at most; the
  // windows are read before the next tile's DMAs into the same LDS go out
  // (the carry is the last read).
  [[maybe_unused]] auto bias_tile = [&](f32x16 (&s)[2], int kt)
      __attribute__((always_inline)) {
    if constexpr (REL) {
      constexpr std::true_type kT{};
      constexpr std::false_type kF{};
      // the bias band: some pair of the tile has dist = q - k < E (the
      // smallest dist is pos_lo - (kt + 63))
      const bool with_bias = pos_lo - (kt + kBN - 1) < a.rel_extent;
      const bool fast = band_masked || pos_hi - kt < a.rel_extent;
      wait_vm<4>();
      asm volatile("" ::: "memory");   // the LDS reads stay below the wait
      if (with_bias) {
        u32x3 x[8];
        bias_read(x);
        if (fast) bias_init(s, kt, x, kT);
        else bias_init(s, kt, x, kF);
      } else {
        s[0] = f32x16{};
        s[1] = f32x16{};
        carry = lds_ld64(bias_a ^ 8u)[0];
      }
      asm volatile("" : "+v"(carry));
    }
  };

  // softmax of scores `s` of the tile at kt (masking when needed): P^T
  // fragments, running max / sum update, O^T rescale when the max moved.
  // `hook` runs first (group 1 issues its tile DMA there).
  auto softmax_phase = [&](f32x16 (&s)[2], int kt, bool first, auto&& hook) {
    const bool full = full_tile(kt);
    hook();
    if (!full) mask_tile(s, kt);
    const float sl2 = a.scale_log2;
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; j += 2)
        mx = fmaxf(fmaxf(mx, s[kb][j]), s[kb][j + 1]);
    bool move;
    float m_use;
    const float alpha = new_max(mx, sl2, move, m_use);
    float psum = 0.0f;
    uint32_t pw[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) pw[q] = prob_pair(s, q, sl2, m_use, psum);
    pack_p(pw, pf);
    l_part = l_part * alpha + psum;
    // O^T holds the tiles before this one: rescale it to the new reference
    // (in place, each product tied to its accumulator register: a plain
    // multiply under the branch leaves the compiler a merge of two copies
    // of O^T, which it resolves with 32 register-pair moves on every tile)
    if (!first && __builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float x = o_acc[db][j];
          asm volatile("v_mul_f32 %0, %1, %0" : "+v"(x) : "v"(alpha));
          o_acc[db][j] = x;
        }
    }
  };

  // MFMA phase of tile t: O^T += V^T.P^T for tile t (four accumulators in
  // turn) interleaved with the scores of tile t+1 (two accumulators), the
  // V^T and K fragments read kRing - 1 MFMAs ahead (3: measured ~1% over 4
  // and 5 ahead on 4K-16K runs; 2 with the fused bias). With the fused
  // bias the phase first puts tile t+1's bias into its score accumulators,
  // then sends the 16 window DMAs of tile t+2 two per MFMA step over the
  // first eight steps (beside the MFMAs instead of in a row before them:
  // ~3% on the adapters' shapes). (Inlined: as a call, its captures would
  // travel through memory and the DMAs' scalar operands into vector
  // registers.)
  auto mfma_phase = [&](int t, auto with_s_c) __attribute__((always_inline)) {
    // (with_s as a type: one straight-line copy per case, no branch between
    // the MFMAs)
    constexpr bool with_s = decltype(with_s_c)::value;
    // the SIMD's issue port goes to this wave's MFMAs first; the softmax
    // wave fills the slots in between (measured ~2% over equal priority)
    __builtin_amdgcn_s_setprio(1);
    [[maybe_unused]] uint32_t b2 = 0;
    if constexpr (with_s && REL) {
      bias_tile(sc, k_lo + (t + 1) * kBN);
      b2 = bias_dma_base(k_lo + (t + 2) * kBN);
    }
    const uint32_t vt_b = lds0 + (t & 3) * kStage + kTileB;
    const uint32_t kt_b = lds0 + ((t + 1) & 3) * kStage;
    auto vf_n = [&](int n) {
      const int db = n & 3, kb = n >> 3, kk = (n >> 2) & 1;
      return vfrag(vt_b, db, kb, kk);
    };
    auto kf_n = [&](int n) { return kfrag(kt_b, n & 1, n >> 1); };
    // fragments read R - 1 MFMAs ahead; one fewer with the fused bias (a
    // fourth slot measured no faster there)
    constexpr int R = REL ? kRing - 1 : kRing;
    bf16x8 vf[R], kf[R];
#pragma unroll
    for (int i = 0; i < R - 1; ++i) {
      vf[i] = vf_n(i);
      if (with_s) kf[i] = kf_n(i);
    }
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      if (n + R - 1 < 16) vf[(n + R - 1) % R] = vf_n(n + R - 1);
      if (with_s && n + R - 1 < 16) kf[(n + R - 1) % R] = kf_n(n + R - 1);
      const int db = n & 3, kb = n >> 3, kk = (n >> 2) & 1;
      o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          vf[n % R], pf[kb][kk], o_acc[db], 0, 0, 0);
      if (with_s) {
        const int skb = n & 1, skk = n >> 1;
        sc[skb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            kf[n % R], qf[skk], (!REL && n < 2) ? f32x16{} : sc[skb], 0, 0,
            0);
      }
      if constexpr (with_s && REL) {
        if (n < 8) {
          bias_dma_one(b2, 2 * n);
          bias_dma_one(b2, 2 * n + 1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // A caller that found its inputs invalid on the device (without a host
  // sync) sets *reject: every output row and LSE entry of the launch is then
  // NaN and no key is read.
  const bool rejected = a.reject != nullptr && as_const(a.reject)[0] != 0;
  if (!rejected) {
  // ---- pipeline: 4 LDS stages, tiles issued three ahead -------------------
  // Slot 2t: group 0 multiplies tile t, group 1 does the softmax of tile t;
  // slot 2t+1: group 0 the softmax of tile t+1, group 1 multiplies tile t.
  // Tile t+3 goes out at the start of slot 2t into the stage of tile t-1
  // (last read in slot 2t-1) and must be in LDS before slot 2t+4; each
  // wave waits for its own part at the end of every odd slot, before the
  // barrier that publishes it (4 instructions per wave per tile).
  // The queries come first, by the same direct loads: the wave's 32 rows
  // (1 KB = 4 rows per instruction, 16-byte chunks swizzled by row & 15)
  // into stages 2 and 3, which hold no tile until tile 2 goes out after
  // every wave has its fragments; rows past the run end arrive as zeros.
  const uint32_t qlds = lds0 + 2 * kStage + (uint32_t)w * (32 * kRowB);
  {
    const int qrow0 = q0 + 32 * (w % QSUB);
    const int64_t qspan = ((int64_t)(len - qrow0 - 1) * a.q_st + kD) * 2;
    const auto rq = make_rsrc(
        a.q + (int64_t)(t0 + qrow0) * a.q_st + (int64_t)head * a.q_sh,
        qrow0 < len ? (uint32_t)qspan : 0u);
    const int qst_b = (int)(a.q_st * 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + grp;
      dma(rq, qlds + i * 1024, r * qst_b + 16 * (slot ^ (r & 15)));
    }
  }
  issue_tile(0, 0);
  if (ntiles > 1) issue_tile(1, 1);
  if constexpr (REL) {   // the first tile's bias windows and carry
    bias_dma(k_lo);
    bias_carry0();
  }
  wait_vm<0>();
  __syncthreads();
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    u32x4 x = __builtin_bit_cast(
        u32x4,
        lds_ld128(qlds + l32 * kRowB + 16 * ((2 * kk + h2) ^ (l32 & 15))));
    if (!qok) x = u32x4{0, 0, 0, 0};
    qf[kk] = __builtin_bit_cast(bf16x8, x);
  }
  __syncthreads();
  if (ntiles > 2) issue_tile(2, 2);
  // End of every odd slot: this wave's part of tile t+2 must be in LDS
  // before the barrier that publishes it. Loads issued after that tile's
  // may still fly: the DMA of tile t+3 and, with the fused bias, the 16
  // window DMAs of the tile after the next softmax (n in all).
  auto odd_end = [&](int n) {
    if (n == 20) wait_vm<20>();
    else if (n == 4) wait_vm<4>();
    else wait_vm<0>();
    __syncthreads();
  };
  constexpr int NB = REL ? 16 : 0;   // bias window DMAs per tile
  // Tile t+3's DMA goes out in slot 2t, where its stage is free: group 0
  // before its MFMA phase, group 1 at the start of its softmax. With the
  // fused bias, the MFMA phase's wait for its windows (4 DMAs at most
  // after them) also covers tile t+2.
  // The first and last tiles are peeled off the loops, so that the loops
  // hold one variant of the MFMA phase: O^T then keeps one set of
  // registers across iterations (variants merged inside the loop made the
  // compiler copy all 64 accumulator registers back and forth every tile).
  constexpr std::true_type kWithS{};
  constexpr std::false_type kNoS{};
  auto none = [] {};
  // No barrier between the two phases of a slot: a tile is published, and
  // its stage freed, at the odd slots' barriers alone; one there only kept
  // the groups in step (without it: ~2% faster on C4 and 4x8192, ~9% with
  // the fused bias at the adapters' shapes, outputs bitwise equal).
  // the first tile's bias (its windows came with the first tiles), then
  // the second tile's windows
  auto bias_first = [&] {
    if constexpr (REL) {
      bias_tile(sc, k_lo);
      bias_dma(k_lo + kBN);
    }
  };
  if (grp_id == 0) {
    bias_first();
    scores(0, sc);
    softmax_phase(sc, k_lo, true, none);
    for (int t = 0; t + 1 < ntiles; ++t) {
      issue_tile(t + 3, (t + 3) & 3, t + 3 < ntiles);
      mfma_phase(t, kWithS);
      softmax_phase(sc, k_lo + (t + 1) * kBN, false, none);
      odd_end(NB + 4);
    }
    mfma_phase(ntiles - 1, kNoS);
    odd_end(0);   // everything, before the output goes through LDS
  } else {
    bias_first();
    issue_tile(3, 3, 3 < ntiles);
    scores(0, sc);
    softmax_phase(sc, k_lo, true, none);
    if (ntiles > 1) mfma_phase(0, kWithS);
    else mfma_phase(0, kNoS);
    odd_end(ntiles > 1 ? NB + 4 : 0);
    for (int t = 1; t + 1 < ntiles; ++t) {
      softmax_phase(sc, k_lo + t * kBN, false,
                    [&] { issue_tile(t + 3, (t + 3) & 3, t + 3 < ntiles); });
      mfma_phase(t, kWithS);
      odd_end(NB + 4);
    }
    if (ntiles > 1) {
      const int t = ntiles - 1;
      softmax_phase(sc, k_lo + t * kBN, false, none);
      mfma_phase(t, kNoS);
      odd_end(0);   // the tile loads, before the output goes through LDS
    }
  }
  }  // !rejected

  // ---- finalise: l over both lane halves, normalise, store --------------
  const float l_tot = l_part + __shfl_xor(l_part, 32);
  const float inv = rejected ? __builtin_nanf("") :
                    l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (a.lse && h2 == 0 && qok)
    a.lse[(int64_t)head * wk.total + t0 + qi] =
        rejected ? __builtin_nanf("") :
        l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : -INFINITY;
  // O^T goes through LDS (free after the last barrier) so that the global
  // stores are whole rows: the wave writes its 32 x 128 block query-major
  // (256-byte rows, 16-byte chunks swizzled by row & 15, so neither the
  // 8-byte writes nor the 16-byte reads conflict), then each store
  // instruction covers 4 complete rows (16 lanes x 16 bytes per row)
  // instead of 16 bytes of 32 rows.
  const uint32_t ob = lds0 + (uint32_t)w * (32 * kRowB);
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const uint32_t w0 = pack_bf16x2(f32_to_bf16_bits(o_acc[db][4 * g4] * inv),
                                      f32_to_bf16_bits(o_acc[db][4 * g4 + 1] * inv));
      const uint32_t w1 = pack_bf16x2(f32_to_bf16_bits(o_acc[db][4 * g4 + 2] * inv),
                                      f32_to_bf16_bits(o_acc[db][4 * g4 + 3] * inv));
      const int c = 4 * db + g4;    // 16-byte chunk: dims 8c .. 8c+7
      lds_st64(ob + l32 * kRowB + 16 * (c ^ (l32 & 15)) + 8 * h2,
               u32x2{w0, w1});
    }
  wave_lds_sync();
  const int qrow0 = q0 + 32 * (w % QSUB);   // query of the block's row 0
  const int c16 = lane & 15;
  const bool al16 = ((a.o_st | a.o_sh) & 7) == 0 &&
                    ((uintptr_t)a.out & 15) == 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    const u32x4 x = __builtin_bit_cast(
        u32x4, lds_ld128(ob + r * kRowB + 16 * (c16 ^ (r & 15))));
    if (qrow0 + r < len) {
      __bf16* const dst = a.out + (int64_t)(t0 + qrow0 + r) * a.o_st +
                          (int64_t)head * a.o_sh + 8 * c16;
      if (al16) {
        *reinterpret_cast<u32x4*>(dst) = x;
      } else {
        reinterpret_cast<u32x2*>(dst)[0] = u32x2{x[0], x[1]};
        reinterpret_cast<u32x2*>(dst)[1] = u32x2{x[2], x[3]};
      }
    }
  }
}

template <int REP, bool REL>
void launch_src(const PrefillArgs& a, int src, dim3 grid, size_t lds,
                hipStream_t st) {
  if (src == kPacked)
    hipLaunchKernelGGL((prefill_kernel<REP, REL, kPacked>), grid, dim3(512),
                       lds, st, a);
  else if (src == kPaged)
    hipLaunchKernelGGL((prefill_kernel<REP, REL, kPaged>), grid, dim3(512),
                       lds, st, a);
  else if (src == kMixed)
    hipLaunchKernelGGL((prefill_kernel<REP, REL, kMixed>), grid, dim3(512),
                       lds, st, a);
  else
    hipLaunchKernelGGL((prefill_kernel<REP, REL, kPackedCM>), grid,
                       dim3(512), lds, st, a);
}

template <int REP>
void launch(PrefillArgs a, int src, int S, int max_seqlen, hipStream_t st) {
  constexpr int BQ = 256 / REP;
  a.nqb_max = (max_seqlen + BQ - 1) / BQ;
  // HKV * items-per-head work-groups, rounded up to whole XCD rounds
  const int64_t items = (int64_t)S * a.nqb_max;
  int64_t n = a.HKV * items;
  if (a.HKV <= 8 && 8 % a.HKV == 0) n = 8 * ((items + 8 / a.HKV - 1) / (8 / a.HKV));
  const dim3 grid((unsigned)n);
  const size_t lds = kNStage * kStage + (a.rel ? 8 * kBiasB : 0);
  if (a.rel)
    launch_src<REP, true>(a, src, grid, lds, st);
  else
    launch_src<REP, false>(a, src, grid, lds, st);
}

// One work-group: *reject = 1 unless q_pos[i] - q_pos[0] == i and
// kv_pos[i] - q_pos[0] == i for every i < T (always written, so the flag
// needs no clearing).
__global__ __launch_bounds__(1024) void positions_check_kernel(
    const int64_t* __restrict__ q_pos, const int64_t* __restrict__ kv_pos,
    int64_t T, int32_t* __restrict__ reject) {
  const int64_t p0 = q_pos[0];
  int bad = 0;
  for (int64_t i = threadIdx.x; i < T; i += blockDim.x)
    bad |= (q_pos[i] - p0 != i) | (kv_pos[i] - p0 != i);
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) reject[0] = bad ? 1 : 0;
}

}  // namespace
}  // namespace tmopt

using namespace tmopt;

extern "C" int tmopt_prefill_check_positions(const int64_t* q_positions,
                                             const int64_t* kv_positions,
                                             int64_t T, int32_t* reject,
                                             tmopt_stream_t stream) {
  clear_error();
  TMOPT_REQUIRE(q_positions && kv_positions && reject, TMOPT_EINVAL,
                "prefill_check_positions: null pointer");
  TMOPT_REQUIRE(T > 0, TMOPT_EINVAL,
                "prefill_check_positions: T must be positive (got %lld)",
                (long long)T);
  hipLaunchKernelGGL(positions_check_kernel, dim3(1), dim3(1024), 0,
                     (hipStream_t)stream, q_positions, kv_positions, T,
                     reject);
  return check_launch("prefill_check_positions");
}

extern "C" int tmopt_attn_prefill_varlen(
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
    const int32_t* reject, tmopt_stream_t stream) {
  clear_error();
  if (num_seqs == 0 || max_seqlen_q == 0) return TMOPT_OK;
  TMOPT_REQUIRE(num_seqs > 0 && num_seqs <= 65535 && max_seqlen_q > 0,
                TMOPT_EINVAL, "prefill: num_seqs=%d max_seqlen_q=%d", num_seqs,
                max_seqlen_q);
  TMOPT_REQUIRE(q && out && cu_seqlens_q, TMOPT_EINVAL,
                "prefill: null q/out/cu_seqlens");
  TMOPT_REQUIRE(D == kD, TMOPT_EUNSUPPORTED, "prefill: D=%d (only 128)", D);
  TMOPT_REQUIRE(HKV > 0 && HQ > 0 && HQ % HKV == 0 && HKV <= 65535,
                TMOPT_EINVAL, "prefill: HQ=%d HKV=%d", HQ, HKV);
  // Query heads per work-group: the largest of 8, 4, 2, 1 dividing HQ/HKV;
  // a ratio above it runs as kv_div scheduled heads per stored KV head
  // (its keys then load once per group of `rep` query heads).
  const int ratio = HQ / HKV;
  const int rep = ratio % 8 == 0 ? 8 : ratio % 4 == 0 ? 4 : ratio % 2 == 0 ? 2 : 1;
  const int kv_div = ratio / rep;
  TMOPT_REQUIRE((int64_t)HKV * kv_div <= 65535, TMOPT_EUNSUPPORTED,
                "prefill: HKV=%d x %d query-head groups exceeds 65535", HKV,
                kv_div);
  TMOPT_REQUIRE(window >= 0, TMOPT_EINVAL, "prefill: window=%d", window);
  TMOPT_REQUIRE(scale > 0.0f, TMOPT_EINVAL, "prefill: scale must be > 0");
  TMOPT_REQUIRE(rel == nullptr || rel_extent > 0, TMOPT_EINVAL,
                "prefill: rel_extent=%d", rel_extent);
  TMOPT_REQUIRE(rel == nullptr ||
                    (rel_stride_tok >= rel_extent && rel_stride_head >= 0 &&
                     (64 * rel_stride_tok + 2 * (int64_t)rel_extent) <
                         kOob),
                TMOPT_EUNSUPPORTED,
                "prefill: rel rows must not overlap, and 32 rows must span "
                "less than 2 GiB (stride_tok=%lld, extent=%d)",
                (long long)rel_stride_tok, rel_extent);
  {
    const int bq = 256 / rep;
    const int64_t blocks =
        (int64_t)HKV * kv_div * num_seqs * ((max_seqlen_q + bq - 1) / bq) +
        8 * 8;
    TMOPT_REQUIRE(blocks < 0x7fffffffll, TMOPT_EUNSUPPORTED,
                  "prefill: %lld work-groups exceed the grid limit",
                  (long long)blocks);
  }
  const bool pooled = block_table != nullptr;
  const bool own = k != nullptr || v != nullptr;
  const bool cm = own && (k_stride_dim != 1 || v_stride_dim != 1);
  const int src = !pooled ? (cm ? kPackedCM : kPacked)
                          : (own ? kMixed : kPaged);
  if (pooled) {
    TMOPT_REQUIRE(k_pool && v_pool && page_size > 0 && bt_stride > 0 &&
                      num_pages > 0 && table_wrap >= 0,
                  TMOPT_EINVAL,
                  "prefill: paged source needs pools, page_size, bt_stride");
    TMOPT_REQUIRE(page_size == kPage, TMOPT_EUNSUPPORTED,
                  "prefill: page_size=%d (only 16)", page_size);
    TMOPT_REQUIRE(((uintptr_t)k_pool | (uintptr_t)v_pool) % 16 == 0,
                  TMOPT_EINVAL, "prefill: pools must be 16-byte aligned");
    TMOPT_REQUIRE((int64_t)kPage * HKV * kD * 2 < (1ll << 31),
                  TMOPT_EUNSUPPORTED, "prefill: page too large");
    // A ring holds the last table_wrap * 16 positions: the run's own keys
    // would overwrite the prior context they must be read beside, so a
    // ring is read for the prior context only (mixed source), under a
    // window no wider than the ring.
    TMOPT_REQUIRE(table_wrap == 0 ||
                      (src == kMixed && table_wrap <= bt_stride && window > 0 &&
                       (int64_t)window <= (int64_t)table_wrap * kPage),
                  TMOPT_EINVAL,
                  "prefill: a ring table (table_wrap=%d) needs packed k/v for "
                  "the run's own keys and 0 < window <= %lld",
                  table_wrap, (long long)table_wrap * kPage);
  } else {
    TMOPT_REQUIRE(prior_lens == nullptr && table_wrap == 0, TMOPT_EINVAL,
                  "prefill: prior context needs a block table");
  }
  if (own) {
    TMOPT_REQUIRE(k && v, TMOPT_EINVAL, "prefill: k and v go together");
    TMOPT_REQUIRE(k_stride_run >= 0 && v_stride_run >= 0 &&
                      k_stride_run % 8 == 0 && v_stride_run % 8 == 0 &&
                      k_stride_head % 8 == 0 && v_stride_head % 8 == 0 &&
                      ((uintptr_t)k | (uintptr_t)v) % 16 == 0,
                  TMOPT_EINVAL,
                  "prefill: k/v runs and heads must start 16-byte aligned "
                  "(run and head strides %% 8)");
    if (cm) {
      // channel-major: tokens contiguous, dim rows 16-byte aligned and not
      // overlapping, runs placed by the run stride (a run's first token
      // must be 16-byte aligned, which cu_seqlens offsets do not promise)
      TMOPT_REQUIRE(!pooled, TMOPT_EUNSUPPORTED,
                    "prefill: channel-major k/v only as the packed source");
      TMOPT_REQUIRE(k_stride_tok == 1 && v_stride_tok == 1 &&
                        k_stride_dim != 1 && v_stride_dim != 1,
                    TMOPT_EINVAL,
                    "prefill: k and v must both be token-major (stride_dim "
                    "1) or both channel-major (stride_tok 1)");
      TMOPT_REQUIRE(k_stride_run > 0 && v_stride_run > 0, TMOPT_EINVAL,
                    "prefill: channel-major k/v need a run stride");
      TMOPT_REQUIRE(k_stride_dim % 8 == 0 && v_stride_dim % 8 == 0 &&
                        k_stride_dim >= max_seqlen_q &&
                        v_stride_dim >= max_seqlen_q,
                    TMOPT_EINVAL,
                    "prefill: channel-major dim rows must be 16-byte aligned "
                    "and hold max_seqlen_q tokens (stride_dim %% 8, >= %d)",
                    max_seqlen_q);
      const int64_t sd = k_stride_dim > v_stride_dim ? k_stride_dim
                                                     : v_stride_dim;
      TMOPT_REQUIRE(((kD - 1) * sd + max_seqlen_q) * 2 < kOob,
                    TMOPT_EUNSUPPORTED,
                    "prefill: a run's channel-major k/v span must stay below "
                    "2 GiB");
    } else {
      TMOPT_REQUIRE(((int64_t)max_seqlen_q * (k_stride_tok > v_stride_tok
                                                  ? k_stride_tok
                                                  : v_stride_tok) +
                     kD) * 2 < kOob,
                    TMOPT_EUNSUPPORTED,
                    "prefill: a run's packed k/v span must stay below 2 GiB");
      TMOPT_REQUIRE(k_stride_tok % 8 == 0 && v_stride_tok % 8 == 0,
                    TMOPT_EINVAL,
                    "prefill: k/v rows must be 16-byte aligned (strides %% 8)");
    }
  }
  TMOPT_REQUIRE(((int64_t)max_seqlen_q * q_stride_tok + kD) * 2 < kOob,
                TMOPT_EUNSUPPORTED,
                "prefill: a run's q span must stay below 2 GiB");
  TMOPT_REQUIRE(q_stride_tok % 8 == 0 && q_stride_head % 8 == 0 &&
                    o_stride_tok % 4 == 0 && o_stride_head % 4 == 0 &&
                    (uintptr_t)q % 16 == 0 && (uintptr_t)out % 8 == 0,
                TMOPT_EINVAL, "prefill: q/out rows misaligned");
  PrefillArgs a;
  a.q = (const __bf16*)q;
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.k = (const __bf16*)k;
  a.k_st = k_stride_tok;
  a.k_sh = k_stride_head;
  a.v = (const __bf16*)v;
  a.v_st = v_stride_tok;
  a.v_sh = v_stride_head;
  a.k_sd = own ? k_stride_dim : 1;
  a.v_sd = own ? v_stride_dim : 1;
  a.k_sr = own ? k_stride_run : 0;
  a.v_sr = own ? v_stride_run : 0;
  a.cu = cu_seqlens_q;
  a.prior = prior_lens;
  a.kpool = (const __bf16*)k_pool;
  a.vpool = (const __bf16*)v_pool;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.bt_width = bt_stride > 0x7fffffff ? 0x7fffffff : (int)bt_stride;
  a.table_wrap = table_wrap;
  a.num_pages = num_pages > 0x7fffffff ? 0x7fffffff : (int)num_pages;
  a.page_size = page_size > 0 ? page_size : 16;
  a.HQ = HQ;
  a.HKV = HKV * kv_div;
  a.kv_div = kv_div;
  a.HKV_stored = HKV;
  a.window = window;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.out = (__bf16*)out;
  a.o_st = o_stride_tok;
  a.o_sh = o_stride_head;
  a.lse = lse;
  a.S = num_seqs;
  a.rel = (const __bf16*)rel;
  a.r_st = rel_stride_tok;
  a.r_sh = rel_stride_head;
  a.rel_extent = rel ? rel_extent : 0;
  a.reject = reject;
  hipStream_t st = (hipStream_t)stream;
  if (rep == 8)
    launch<8>(a, src, num_seqs, max_seqlen_q, st);
  else if (rep == 4)
    launch<4>(a, src, num_seqs, max_seqlen_q, st);
  else if (rep == 2)
    launch<2>(a, src, num_seqs, max_seqlen_q, st);
  else
    launch<1>(a, src, num_seqs, max_seqlen_q, st);
  return check_launch("prefill");
}
