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
constexpr int kKRow = 272;                // K tile row: 256 B + 16 B pad
constexpr int kVRow = 144;                // V^T tile row: 128 B + 16 B pad
constexpr int kKBytes = kBN * kKRow;      // 17408
constexpr int kVBytes = kD * kVRow;       // 18432
constexpr int kStage = kKBytes + kVBytes; // 35840; two stages per block
constexpr float kLazy = 8.0f;             // lazy-rescale threshold (log2)

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

// LDS column of key kappa (0..63) in a V^T row: within each 16-key chunk the
// keys 4a+c go to 8*(a&1) + 4*(a>>1) + c, so that lane half h of the P.V
// MFMA finds its eight keys {4h+c, 8+4h+c} in columns 8h..8h+7.
__device__ __forceinline__ int vt_col(int kappa) {
  const int o = kappa & 15;
  return (kappa & ~15) + 8 * ((o >> 2) & 1) + 4 * (o >> 3) + (o & 3);
}

// byte offset of (row d, logical 16-byte chunk ch, byte-in-chunk b) in V^T
__device__ __forceinline__ int vt_off(int d, int ch, int b) {
  return d * kVRow + ((ch ^ ((d >> 3) & 7)) << 4) + b;
}

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

template <int REP, bool REL>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
  constexpr int BQ = 256 / REP;   // queries per work-group
  constexpr int QSUB = BQ / 32;   // 32-query sub-blocks per head
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;         // 8 waves: one 32-row block each
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
  const bool paged = a.bt != nullptr;

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

  // ---- tile loaders (global -> registers -> LDS) -------------------------
  // K: thread t stages keys (t>>4) + 32i (i = 0, 1), 16-byte chunk t & 15.
  // V: thread t stages keys 2*(t>>4) + i (i = 0, 1), dims 8*(t & 15)..+7.
  // The loads of tile j+1 are issued before tile j's math and consumed only
  // by the LDS stores after it, so nothing may look at the loaded values in
  // between (a select on them would make every load complete on the spot).
  // Packed source: buffer loads over the run's rows; keys past the run fall
  // outside the resource and read as zero. Paged source: global loads with
  // a clamped address; the validity bits are applied at store time.
  const int kc = tid & 15;
  const int kr = tid >> 4;                    // 0..31
  u32x4 kreg[2], vreg[2];
  unsigned okbits = 0xf;
  // (paged launches pass no k / v: their resources are empty and unused)
  const char* kb0 = paged ? nullptr : reinterpret_cast<const char*>(
      a.k + (int64_t)t0 * a.k_st + (int64_t)kvh * a.k_sh);
  const char* vb0 = paged ? nullptr : reinterpret_cast<const char*>(
      a.v + (int64_t)t0 * a.v_st + (int64_t)kvh * a.v_sh);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(kb0), (short)0,
      paged ? 0 : (int)(((int64_t)(len - 1) * a.k_st + kD) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(vb0), (short)0,
      paged ? 0 : (int)(((int64_t)(len - 1) * a.v_st + kD) * 2), 0x00020000);
  const int kst_b = (int)(a.k_st * 2), vst_b = (int)(a.v_st * 2);
  const int koff[2] = {kr * kst_b + 16 * kc, (kr + 32) * kst_b + 16 * kc};
  const int voff[2] = {2 * kr * vst_b + 16 * kc, (2 * kr + 1) * vst_b + 16 * kc};

  // page of tile-local key kl (0..63) among the tile's 4 pages, fetched
  // once per tile with wave-uniform scalar loads (a per-lane table load
  // would have to complete before the K/V loads it addresses)
  const int last_lp = (nk - 1) / a.page_size;
  auto paged_row = [&](int p0, int p1, int p2, int p3, int kt, int kl,
                       const __bf16* pool, bool& ok) {
    const int kappa = kt + kl;
    ok = kappa < nk;
    int pg = p0;
    pg = (kl >> 4) == 1 ? p1 : pg;
    pg = (kl >> 4) == 2 ? p2 : pg;
    pg = (kl >> 4) == 3 ? p3 : pg;
    if ((unsigned)pg >= (unsigned)a.num_pages) { ok = false; pg = 0; }
    const int64_t row = (int64_t)pg * a.page_size + (kappa % a.page_size);
    return pool + (row * a.HKV + kvh) * kD + 8 * kc;
  };

  auto load_tile = [&](int kt) {
    if (!paged) {
      // per-thread offsets are loop-invariant; the tile offset rides in the
      // scalar soffset field
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        kreg[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rk, koff[i], kt * kst_b, 0));
        vreg[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rv, voff[i], kt * vst_b, 0));
      }
    } else {
      const int32_t __attribute__((address_space(4)))* trow =
          as_const(a.bt) + (int64_t)seq * a.bt_stride;
      const int lp0 = kt / a.page_size;
      const int p0 = trow[min(lp0, last_lp)];
      const int p1 = trow[min(lp0 + 1, last_lp)];
      const int p2 = trow[min(lp0 + 2, last_lp)];
      const int p3 = trow[min(lp0 + 3, last_lp)];
      unsigned bits = 0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        bool ok;
        const __bf16* src =
            paged_row(p0, p1, p2, p3, kt, kr + 32 * i, a.kpool, ok);
        kreg[i] = *reinterpret_cast<const u32x4*>(src);
        bits |= ok ? (1u << i) : 0u;
        src = paged_row(p0, p1, p2, p3, kt, 2 * kr + i, a.vpool, ok);
        vreg[i] = *reinterpret_cast<const u32x4*>(src);
        bits |= ok ? (4u << i) : 0u;
      }
      okbits = bits;
    }
  };

  auto store_tile = [&](int stage) {
    char* ks = smem + stage * kStage;
    char* vs = ks + kKBytes;
    const u32x4 z = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(ks + (kr + 32 * i) * kKRow + 16 * kc) =
          (okbits & (1u << i)) ? kreg[i] : z;
    const u32x4 v0 = (okbits & 4u) ? vreg[0] : z;
    const u32x4 v1 = (okbits & 8u) ? vreg[1] : z;
    // V^T: dims 8kc+e, keys 2kr, 2kr+1 -> one 4-byte write per dim
    const int col = vt_col(2 * kr);
    const int ch = col >> 3;          // 16-byte chunk (8 keys)
    const int b = (col & 7) * 2;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = 8 * kc + 2 * c;
      *reinterpret_cast<uint32_t*>(vs + vt_off(d, ch, b)) =
          interleave_lo(v0[c], v1[c]);
      *reinterpret_cast<uint32_t*>(vs + vt_off(d + 1, ch, b)) =
          interleave_hi(v0[c], v1[c]);
    }
  };

  // ---- accumulators -----------------------------------------------------
  f32x16 o_acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o_acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_part = 0.0f;

  load_tile(k_lo);
  store_tile(0);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int kt = k_lo + it * kBN;
    const int stage = it & 1;
    if (it + 1 < ntiles) load_tile(kt + kBN);
    const char* ks = smem + stage * kStage;
    const char* vs = ks + kKBytes;

    // does any element of this tile need masking?
    const bool full = (kt + kBN - 1 <= pos_lo) && (kt + kBN <= nk) &&
                      (a.window == 0 || pos_hi - kt < a.window) &&
                      (qn == BQ);

    // ---- S^T = K.Q^T ----------------------------------------------------
    f32x16 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(
                        ks + (32 * kb + l32) * kKRow + 32 * kk + 16 * h2));
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sc[kb],
                                                         0, 0, 0);
      }
    }

    // ---- online softmax -------------------------------------------------
    // Without a bias the max runs on the raw scores (scale > 0 commutes with
    // max) and each probability is one fma + exp2: p = 2^(s*scale*log2e - m).
    // With the fused relative bias (attn_prefill.py:115-120) the scores are
    // first moved to the log2 domain, s*scale*log2e + rel*log2e, gathered at
    // rel[q, h, dist] for 0 <= dist < E and zero outside the band.
    float sl2 = a.scale_log2;
    if constexpr (REL) {
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
          sc[kb][j] = __builtin_fmaf(sc[kb][j], a.scale_log2, bias * kLog2e);
        }
      sl2 = 1.0f;
    }
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kp = kt + 32 * kb + 8 * (j >> 2) + 4 * h2 + (j & 3);
          const int dist = qpos - kp;
          const bool ok = qok && dist >= 0 && kp < nk &&
                          (a.window == 0 || dist < a.window);
          sc[kb][j] = ok ? sc[kb][j] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; j += 2)
        mx = fmaxf(fmaxf(mx, sc[kb][j]), sc[kb][j + 1]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy rescaling: the running max (log2 domain) only moves when the
    // tile's max exceeds it by more than kLazy, so probabilities stay below
    // 2^kLazy and O^T / l are rescaled on few tiles; O / l and the LSE are
    // exact for any reference point.
    const float m_cand = mx * sl2;
    const bool move = m_cand > m_run + kLazy;
    const float m_new = move ? m_cand : m_run;
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = move ? fast_exp2(m_run - m_use) : 1.0f;
    m_run = m_new;
    float psum = 0.0f;
    bf16x8 pf[2][2];  // [kb][kk]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint32_t pw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = fast_exp2(
              __builtin_fmaf(sc[kb][8 * kk + 2 * e], sl2, -m_use));
          const float p1 = fast_exp2(
              __builtin_fmaf(sc[kb][8 * kk + 2 * e + 1], sl2, -m_use));
          psum += p0 + p1;
          pw[e] = pack_bf16x2_rn(p0, p1);
        }
        pf[kb][kk] =
            __builtin_bit_cast(bf16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
      }
    l_part = l_part * alpha + psum;
    // rescale O^T only when some lane's reference point moved
    if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o_acc[db] = o_acc[db] * alpha;
    }

    // ---- O^T += V^T.P^T --------------------------------------------------
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 vf = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const u32x4*>(
                          vs + vt_off(d, 2 * (2 * kb + kk) + h2, 0)));
          o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              vf, pf[kb][kk], o_acc[db], 0, 0, 0);
        }
    }

    if (it + 1 < ntiles) store_tile(stage ^ 1);
    __syncthreads();
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
  if (a.rel)
    hipLaunchKernelGGL((prefill_kernel<REP, true>), grid, dim3(512),
                       2 * kStage, st, a);
  else
    hipLaunchKernelGGL((prefill_kernel<REP, false>), grid, dim3(512),
                       2 * kStage, st, a);
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
