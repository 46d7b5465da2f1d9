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
//    owns one 32-row MFMA block (one head x 32 queries); about 200
//    registers per wave leave room for two waves per SIMD, so one wave's
//    MFMAs overlap the other's softmax.
//  * Transposed scores. S^T = K.Q^T (v_mfma_f32_32x32x16_bf16, keys on M,
//    queries on N) leaves one query per lane, so the running max needs one
//    cross-lane step (xor 32) and the running sum stays lane-local; P^T is
//    then already the B operand of O^T = V^T.P^T, and the rescale factor of
//    every O^T element a lane holds is that lane's own.
//  * K tiles are stored row-major in LDS (272-byte rows: conflict-free
//    16-byte fragment reads); V tiles are stored transposed, each thread
//    packing 2 keys of one dimension into one 4-byte write, with the keys
//    of a row permuted so that every P.V fragment is one 16-byte read, and
//    the 16-byte chunks XOR-swizzled by row group to spread the writes over
//    the banks. Tiles are double-buffered: the next tile's global loads fly
//    while the current tile's MFMAs run; one barrier per tile.
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
#include "common.h"

namespace tmopt {
namespace {

constexpr int kD = 128;
constexpr int kBN = 64;                   // keys per tile
constexpr int kRowB = 256;                // K / V tile row in LDS (one key)
constexpr int kTileB = kBN * kRowB;       // 16384
constexpr int kStage = 2 * kTileB;        // K tile then V tile
constexpr int kNStage = 4;                // 128 KB of LDS per work-group
constexpr int kPage = 16;                 // paged source: tokens per page
constexpr float kLazy = 8.0f;             // lazy-rescale threshold (log2)

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
// the compiler does not wait for it at every barrier; the kernel waits for
// these loads itself (wait_vm).
__device__ __forceinline__ void dma_b128(i32x4 rsrc, uint32_t lds, int voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds), "v"(voff), "s"(rsrc)
      : "memory");
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
  const int32_t* cu;
  const int32_t* prior;
  const __bf16* kpool;
  const __bf16* vpool;
  const int32_t* bt;
  int64_t bt_stride;
  int num_pages;
  int page_size;
  int HQ, HKV;
  int window;
  float scale_log2;
  __bf16* out;
  int64_t o_st, o_sh;
  float* lse;        // [HQ, cu[S]]
  int S;
  int nqb_max;       // query blocks of the longest run
  const __bf16* rel; // optional fused relative bias, rows like q
  int64_t r_st, r_sh;
  int rel_extent;
};

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
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
  int kvh, seq, qb;  // seq < 0: nothing to do
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
  Work w{kvh, -1, 0};
  const int nb0 = lane < a.S ? run_blocks(a, lane, BQ) : 0;
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
      w.seq = s0 + __builtin_ctzll(hit);
      w.qb = a.nqb_max - 1 - lo;
      return w;
    }
    rem -= pop;
  }
  return w;  // not reached for i < total
}

template <int REP, bool REL, bool PAGED>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
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
  const int seq = wk.seq;
  const int qb = wk.qb;

  const int t0 = as_const(a.cu)[seq];
  const int len = as_const(a.cu)[seq + 1] - t0;
  const int q0 = qb * BQ;
  const int prior = a.prior ? as_const(a.prior)[seq] : 0;
  const int nk = prior + len;                 // keys of this run
  const int qn = min(BQ, len - q0);
  const int pos_lo = prior + q0;              // first query position
  const int pos_hi = prior + q0 + qn - 1;     // last valid query position
  int k_lo = a.window > 0 ? max(0, pos_lo - a.window + 1) : 0;
  k_lo = (k_lo / kBN) * kBN;
  const int k_hi = pos_hi + 1;                // exclusive
  const int ntiles = (k_hi - k_lo + kBN - 1) / kBN;

  // ---- this wave's row block: head and 32-query sub-block ----------------
  const int head = kvh * REP + w / QSUB;
  const int qi = q0 + 32 * (w % QSUB) + l32;  // this lane's query (column)
  const bool qok = qi < len;
  const int qpos = prior + qi;

  // ---- Q fragments: B operand of S^T (column = query, k = dims) --------
  bf16x8 qf[8];
  {
    const __bf16* row = a.q + (int64_t)(t0 + (qok ? qi : 0)) * a.q_st +
                        (int64_t)head * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 x = *reinterpret_cast<const u32x4*>(row + 16 * kk + 8 * h2);
      if (!qok) x = u32x4{0, 0, 0, 0};
      qf[kk] = __builtin_bit_cast(bf16x8, x);
    }
  }

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
  i32x4 rk = {0, 0, 0, 0}, rv = {0, 0, 0, 0};
  int kst_b = 0, vst_b = 0, klane = 0, vlane = 0;
  [[maybe_unused]] const int row_b = a.HKV * kD * 2;   // paged: token row
  [[maybe_unused]] const int64_t page_b = (int64_t)kPage * row_b;
  if constexpr (!PAGED) {
    kst_b = (int)(a.k_st * 2);
    vst_b = (int)(a.v_st * 2);
    rk = make_rsrc(a.k + (int64_t)t0 * a.k_st + (int64_t)kvh * a.k_sh,
                   (uint32_t)(((int64_t)(len - 1) * a.k_st + kD) * 2));
    rv = make_rsrc(a.v + (int64_t)t0 * a.v_st + (int64_t)kvh * a.v_sh,
                   (uint32_t)(((int64_t)(len - 1) * a.v_st + kD) * 2));
    klane = grp * kst_b + 16 * kchunk;
    vlane = grp * vst_b + 16 * vchunk;
  } else {
    klane = grp * row_b + kvh * (kD * 2) + 16 * kchunk;
    vlane = grp * row_b + kvh * (kD * 2) + 16 * vchunk;
  }
  [[maybe_unused]] const int32_t __attribute__((address_space(4)))* trow =
      PAGED ? as_const(a.bt) + (int64_t)seq * a.bt_stride : nullptr;
  [[maybe_unused]] const int last_lp = (nk - 1) >> 4;

  // issue tile `t` (index from k_lo) into LDS stage `st`: 4 instructions
  auto issue_tile = [&](int t, int st) {
    const int kt = k_lo + t * kBN;
    const uint32_t sb = lds0 + st * kStage;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = 4 * w + 32 * i;          // first row of the block
      const uint32_t dk = sb + r0 * kRowB, dv = dk + kTileB;
      if constexpr (!PAGED) {
        dma_b128(rk, dk, klane + (kt + r0) * kst_b);
        dma_b128(rv, dv, vlane + (kt + r0) * vst_b);
      } else {
        // the 4 rows lie in one page; its resource covers only the rows
        // of the run (and nothing for a page id outside the pool)
        const int key0 = kt + r0;
        const int lp = key0 >> 4;
        const int pg = lp <= last_lp ? trow[lp] : -1;
        const bool valid = (unsigned)pg < (unsigned)a.num_pages;
        const int rows = min(kPage, max(0, nk - kPage * lp));
        const uint32_t nrec = valid ? (uint32_t)(rows * row_b) : 0u;
        const int64_t pofs = valid ? (int64_t)pg * page_b : 0;
        const int roff = (key0 & (kPage - 1)) * row_b;
        dma_b128(make_rsrc(reinterpret_cast<const char*>(a.kpool) + pofs,
                           nrec),
                 dk, klane + roff);
        dma_b128(make_rsrc(reinterpret_cast<const char*>(a.vpool) + pofs,
                           nrec),
                 dv, vlane + roff);
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

  // S^T = K.Q^T for the tile in `stage` (keys on M, queries on N)
  auto scores = [&](int stage, f32x16 (&s)[2]) {
    const uint32_t kb0 = ka0 + lds0 + stage * kStage;
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 kf = lds_ld128((kb0 ^ (32u * kk)) + 32 * kb * kRowB);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kb], 0,
                                                        0, 0);
      }
  };

  // V^T fragment (db, kb, kk) of the tile whose V rows start at vbase
  auto vfrag = [&](uint32_t vdb, int kb, int kk) {
    const uint32_t p = vdb + (32 * kb + 16 * kk) * kRowB;
    const bf16x4 lo = lds_tr16(p);
    const bf16x4 hi = lds_tr16(p + 8 * kRowB);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  // per-element mask (causal, window, run end) and optional fused bias
  auto mask_bias = [&](f32x16 (&s)[2], int kt) {
    if constexpr (REL) {
      // the scores move to the log2 domain: s*scale*log2e + rel*log2e,
      // rel gathered at rel[q, h, dist] for 0 <= dist < E, zero outside
      const __bf16* rrow = a.rel + (int64_t)(t0 + (qok ? qi : 0)) * a.r_st +
                           (int64_t)head * a.r_sh;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kp = kt + 32 * kb + 8 * (j >> 2) + 4 * h2 + (j & 3);
          const int dist = qpos - kp;
          const bool band = qok && dist >= 0 && dist < a.rel_extent;
          const float bias = band ? (float)rrow[dist] : 0.0f;
          s[kb][j] = __builtin_fmaf(s[kb][j], a.scale_log2, bias * kLog2e);
        }
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kp = kt + 32 * kb + 8 * (j >> 2) + 4 * h2 + (j & 3);
        const int dist = qpos - kp;
        const bool ok = qok && dist >= 0 && kp < nk &&
                        (a.window == 0 || dist < a.window);
        s[kb][j] = ok ? s[kb][j] : -INFINITY;
      }
  };

  // ---- accumulators -----------------------------------------------------
  f32x16 o_acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o_acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_part = 0.0f;
  // Without a bias the max runs on the raw scores (scale > 0 commutes with
  // max) and each probability is one fma + exp2: p = 2^(s*scale*log2e - m).
  const float sl2 = REL ? 1.0f : a.scale_log2;

  // Lazy rescaling: the running max (log2 domain) only moves when the
  // tile's max exceeds it by more than kLazy, so probabilities stay below
  // 2^kLazy and O^T / l are rescaled on few tiles; O / l and the LSE are
  // exact for any reference point.
  auto new_max = [&](float mx, bool& move, float& m_use) {
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
  auto prob_pair = [&](const f32x16 (&s)[2], int q, float m_use,
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

  // The softmax of a tile is done in two halves so that neither MFMA phase
  // runs alone: half 1 (max, reference point, probability pairs 0..7) runs
  // under the previous tile's P.V MFMAs, half 2 (pairs 8..15) under the
  // next tile's score MFMAs, about five VALU instructions per MFMA in
  // both phases.
  struct Soft {
    float alpha, m_use, psum;
    bool move;
    uint32_t pw[16];
  };
  auto tile_max = [&](const f32x16 (&s)[2]) {
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; j += 2)
        mx = fmaxf(fmaxf(mx, s[kb][j]), s[kb][j + 1]);
    return mx;
  };
  // half 1 without interleave (masked / biased tiles, the first tile)
  auto half1_plain = [&](const f32x16 (&s)[2], Soft& sf) {
    sf.alpha = new_max(tile_max(s), sf.move, sf.m_use);
    sf.psum = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) sf.pw[q] = prob_pair(s, q, sf.m_use, sf.psum);
  };
  auto half2_plain = [&](const f32x16 (&s)[2], Soft& sf) {
#pragma unroll
    for (int q = 8; q < 16; ++q) sf.pw[q] = prob_pair(s, q, sf.m_use, sf.psum);
  };

  // Phase A of tile it: the next tile's scores (16 MFMAs, K fragments read
  // three chunks ahead) with half 2 of this tile's softmax between them,
  // chunk by chunk. A scheduling fence after every chunk keeps the
  // interleave, and each chunk's results are pinned in place by an empty
  // asm that takes them as operands (pure arithmetic would otherwise be
  // sunk to its first use, past the fences, before scheduling starts).
  auto front = [&](int st_n, const f32x16 (&cur)[2], f32x16 (&nxt)[2],
                   Soft& sf) {
    const uint32_t kb0 = ka0 + lds0 + st_n * kStage;
    auto kfrag = [&](int n) {
      return lds_ld128((kb0 ^ (32u * (n >> 1))) + 32 * (n & 1) * kRowB);
    };
    bf16x8 kf[4];
    kf[0] = kfrag(0);
    kf[1] = kfrag(1);
    kf[2] = kfrag(2);
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      if (n + 3 < 16) kf[(n + 3) & 3] = kfrag(n + 3);
      const int kb = n & 1, kk = n >> 1;
      nxt[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          kf[n & 3], qf[kk], n < 2 ? f32x16{} : nxt[kb], 0, 0, 0);
      if (n & 1) {
        const int q = 8 + (n >> 1);
        sf.pw[q] = prob_pair(cur, q, sf.m_use, sf.psum);
        asm volatile("" : "+v"(sf.pw[q]), "+v"(sf.psum));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Phase B of tile it: O^T += V^T.P^T (16 MFMAs, V^T fragments read three
  // ahead, the four accumulators in turn) with half 1 of the next tile's
  // softmax between them: the max over chunks 0..3, the reference point in
  // chunk 4, pairs 0..7 over chunks 5..15.
  auto back = [&](int stage, const bf16x8 (&pf)[2][2],
                  const f32x16 (&nxt)[2], Soft& sn, bool with_next) {
    const uint32_t vb = va0 + lds0 + stage * kStage + kTileB;
    auto vf_n = [&](int n) {
      const int db = n & 3, kb = n >> 3, kk = (n >> 2) & 1;
      return vfrag(vb ^ (64u * db), kb, kk);
    };
    bf16x8 vf[4];
    vf[0] = vf_n(0);
    vf[1] = vf_n(1);
    vf[2] = vf_n(2);
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      if (n + 3 < 16) vf[(n + 3) & 3] = vf_n(n + 3);
      const int db = n & 3, kb = n >> 3, kk = (n >> 2) & 1;
      o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          vf[n & 3], pf[kb][kk], o_acc[db], 0, 0, 0);
      if (with_next) {
        if (n < 4) {
          const int kb2 = n >> 1, j0 = 8 * (n & 1);
#pragma unroll
          for (int j = 0; j < 8; j += 2)
            mx[n] = fmaxf(fmaxf(mx[n], nxt[kb2][j0 + j]), nxt[kb2][j0 + j + 1]);
          asm volatile("" : "+v"(mx[n]));
        } else if (n == 4) {
          sn.alpha = new_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])),
                             sn.move, sn.m_use);
          sn.psum = 0.0f;
          asm volatile("" : "+v"(sn.alpha), "+v"(sn.m_use));
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (5 + (q * 11) / 8 == n) {
              sn.pw[q] = prob_pair(nxt, q, sn.m_use, sn.psum);
              asm volatile("" : "+v"(sn.pw[q]), "+v"(sn.psum));
            }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto full_tile = [&](int kt) {
    return (kt + kBN - 1 <= pos_lo) && (kt + kBN <= nk) &&
           (a.window == 0 || pos_hi - kt < a.window) && (qn == BQ);
  };

  // ---- pipeline: 4 LDS stages, tiles issued two ahead ---------------------
  // At the top of step `it`, tiles it and it+1 are in LDS (published by a
  // barrier) and tile it+2 is in flight; step it issues tile it+3 into the
  // stage tile it-1 used, and before its closing barrier waits for tile
  // it+2 (every wave issues 4 instructions per tile).
  issue_tile(0, 0);
  if (ntiles > 1) issue_tile(1, 1);
  if (ntiles > 2) {
    issue_tile(2, 2);
    wait_vm<4>();
  } else {
    wait_vm<0>();
  }
  __syncthreads();

  int st_cur = 0;   // stage of tile it
  Soft sf;          // softmax state of tile it (half 1 done)
  auto step = [&](int it, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
    const int kt = k_lo + it * kBN;
    const int st_nxt = (st_cur + 1) & 3;
    const bool has_next = it + 1 < ntiles;
    // phase A: rescale O^T if some lane's reference point moved, then the
    // next tile's scores under half 2 of this tile's softmax
    if (__builtin_amdgcn_ballot_w64(sf.move)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o_acc[db] = o_acc[db] * sf.alpha;
    }
    if (!REL && has_next) {
      front(st_nxt, cur, nxt, sf);
    } else {
      half2_plain(cur, sf);
      if (has_next) scores(st_nxt, nxt);
    }
    bf16x8 pf[2][2];
    pack_p(sf.pw, pf);
    l_part = l_part * sf.alpha + sf.psum;
    // phase B: P.V of this tile under half 1 of the next tile's softmax
    const bool more = it + 3 < ntiles;
    if (more) issue_tile(it + 3, (st_cur + 3) & 3);
    if (has_next && !REL && full_tile(kt + kBN)) {
      back(st_cur, pf, nxt, sf, true);
    } else {
      back(st_cur, pf, nxt, sf, false);
      if (has_next) {
        mask_bias(nxt, kt + kBN);
        half1_plain(nxt, sf);
      }
    }
    if (more) wait_vm<4>(); else wait_vm<0>();
    __syncthreads();
    st_cur = st_nxt;
  };

  f32x16 sa[2], sb[2];
  scores(0, sa);
  if (REL || !full_tile(k_lo)) mask_bias(sa, k_lo);
  half1_plain(sa, sf);
  for (int it = 0; it < ntiles; ++it) {
    step(it, sa, sb);
    sa[0] = sb[0];
    sa[1] = sb[1];
  }

  // ---- finalise: l over both lane halves, normalise, store --------------
  const float l_tot = l_part + __shfl_xor(l_part, 32);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (!qok) return;
  __bf16* orow = a.out + (int64_t)(t0 + qi) * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const uint32_t w0 = pack_bf16x2(f32_to_bf16_bits(o_acc[db][4 * g4] * inv),
                                      f32_to_bf16_bits(o_acc[db][4 * g4 + 1] * inv));
      const uint32_t w1 = pack_bf16x2(f32_to_bf16_bits(o_acc[db][4 * g4 + 2] * inv),
                                      f32_to_bf16_bits(o_acc[db][4 * g4 + 3] * inv));
      *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * g4 + 4 * h2) =
          u32x2{w0, w1};
    }
  if (a.lse && h2 == 0)
    a.lse[(int64_t)head * as_const(a.cu)[a.S] + t0 + qi] =
        l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : -INFINITY;
}

template <int REP>
void launch(PrefillArgs a, int S, int max_seqlen, hipStream_t st) {
  constexpr int BQ = 256 / REP;
  a.nqb_max = (max_seqlen + BQ - 1) / BQ;
  // HKV * items-per-head work-groups, rounded up to whole XCD rounds
  const int64_t items = (int64_t)S * a.nqb_max;
  int64_t n = a.HKV * items;
  if (a.HKV <= 8 && 8 % a.HKV == 0) n = 8 * ((items + 8 / a.HKV - 1) / (8 / a.HKV));
  dim3 grid((unsigned)n);
  const bool paged = a.bt != nullptr;
  const size_t lds = kNStage * kStage;
  if (a.rel) {
    if (paged)
      hipLaunchKernelGGL((prefill_kernel<REP, true, true>), grid, dim3(512),
                         lds, st, a);
    else
      hipLaunchKernelGGL((prefill_kernel<REP, true, false>), grid, dim3(512),
                         lds, st, a);
  } else {
    if (paged)
      hipLaunchKernelGGL((prefill_kernel<REP, false, true>), grid, dim3(512),
                         lds, st, a);
    else
      hipLaunchKernelGGL((prefill_kernel<REP, false, false>), grid,
                         dim3(512), lds, st, a);
  }
}

}  // namespace
}  // namespace tmopt

using namespace tmopt;

extern "C" int tmopt_attn_prefill_varlen(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
    int64_t k_stride_tok, int64_t k_stride_head, const void* v,
    int64_t v_stride_tok, int64_t v_stride_head, const int32_t* cu_seqlens_q,
    const int32_t* prior_lens, int num_seqs, int max_seqlen_q,
    const void* k_pool, const void* v_pool, const int32_t* block_table,
    int64_t bt_stride, int page_size, int64_t num_pages, int HQ, int HKV, int D,
    int window, float scale, const void* rel, int64_t rel_stride_tok,
    int64_t rel_stride_head, int rel_extent, void* out, int64_t o_stride_tok,
    int64_t o_stride_head, float* lse, tmopt_stream_t stream) {
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
  const int rep = HQ / HKV;
  TMOPT_REQUIRE(rep == 4 || rep == 8, TMOPT_EUNSUPPORTED,
                "prefill: HQ/HKV=%d not in {4, 8}", rep);
  TMOPT_REQUIRE(window >= 0, TMOPT_EINVAL, "prefill: window=%d", window);
  TMOPT_REQUIRE(scale > 0.0f, TMOPT_EINVAL, "prefill: scale must be > 0");
  TMOPT_REQUIRE(rel == nullptr || rel_extent > 0, TMOPT_EINVAL,
                "prefill: rel_extent=%d", rel_extent);
  {
    const int bq = 256 / rep;
    const int64_t blocks =
        (int64_t)HKV * num_seqs * ((max_seqlen_q + bq - 1) / bq) + 8 * 8;
    TMOPT_REQUIRE(blocks < 0x7fffffffll, TMOPT_EUNSUPPORTED,
                  "prefill: %lld work-groups exceed the grid limit",
                  (long long)blocks);
  }
  const bool paged = block_table != nullptr;
  if (paged) {
    TMOPT_REQUIRE(k_pool && v_pool && page_size > 0 && bt_stride > 0 &&
                      num_pages > 0,
                  TMOPT_EINVAL,
                  "prefill: paged source needs pools, page_size, bt_stride");
    TMOPT_REQUIRE(page_size == kPage, TMOPT_EUNSUPPORTED,
                  "prefill: page_size=%d (only 16)", page_size);
    TMOPT_REQUIRE(((uintptr_t)k_pool | (uintptr_t)v_pool) % 16 == 0,
                  TMOPT_EINVAL, "prefill: pools must be 16-byte aligned");
  } else {
    TMOPT_REQUIRE(k && v && prior_lens == nullptr, TMOPT_EINVAL,
                  "prefill: packed source needs k/v and no prior context");
    TMOPT_REQUIRE(((int64_t)max_seqlen_q * (k_stride_tok > v_stride_tok
                                                ? k_stride_tok
                                                : v_stride_tok) +
                   kD) * 2 < (1ll << 31),
                  TMOPT_EUNSUPPORTED,
                  "prefill: a run's packed k/v span must stay below 2 GiB");
    TMOPT_REQUIRE(k_stride_tok % 8 == 0 && k_stride_head % 8 == 0 &&
                      v_stride_tok % 8 == 0 && v_stride_head % 8 == 0 &&
                      ((uintptr_t)k | (uintptr_t)v) % 16 == 0,
                  TMOPT_EINVAL,
                  "prefill: k/v rows must be 16-byte aligned (strides %% 8)");
  }
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
  a.cu = cu_seqlens_q;
  a.prior = prior_lens;
  a.kpool = (const __bf16*)k_pool;
  a.vpool = (const __bf16*)v_pool;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.num_pages = num_pages > 0x7fffffff ? 0x7fffffff : (int)num_pages;
  a.page_size = page_size > 0 ? page_size : 16;
  a.HQ = HQ;
  a.HKV = HKV;
  a.window = window;
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
  hipStream_t st = (hipStream_t)stream;
  if (rep == 8)
    launch<8>(a, num_seqs, max_seqlen_q, st);
  else
    launch<4>(a, num_seqs, max_seqlen_q, st);
  return check_launch("prefill");
}
