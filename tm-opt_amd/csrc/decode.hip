// Split-KV paged decode attention for gfx950 (CDNA4).
//
// Replaces _attn_decode_kernel (engine/pyengine/kernels/attn_swa.py:49-117):
// one query token per sequence against its paged K/V history, GQA group of
// REP query heads per KV head, fp32 online softmax, probabilities rounded to
// bf16 for the P.V product (attn_swa.py:110-112), one bf16 rounding of the
// output. Differences from the reference kernel, all MI355X-driven:
//
//  * Split-KV. A work-group owns (sequence b, split s, group of 4 KV heads);
//    a split is `split_pages` consecutive pages of the visible range. Splits
//    of one sequence are merged by a second kernel through their log-sum-exp
//    (decode_combine_kernel). A sequence that needs one split is finalised
//    in place and skipped by the combine.
//  * Only pages holding visible keys are touched: [lo/16, ceil(n/16)) where
//    lo = max(0, n - window) on sliding-window layers, 0 on global ones.
//  * One wave per KV head. The four waves of a work-group read the four
//    256-byte head slices of the same token rows, so together they stream
//    whole 16 KB pages. K and V arrive by 16-byte buffer loads whose
//    resource is one page: a missing page (beyond the split, or a table
//    entry outside the pool) has zero records, so its loads return zeros
//    without touching memory and the next step's loads are always issued
//    ahead of the current step's math (no branch, no vmcnt(0) drain).
//  * Scores and P.V run on MFMA (v_mfma_f32_16x16x32_bf16). S^T = K.Q^T puts
//    16 tokens on the M axis and the REP heads (padded to 16) on N, so each
//    lane ends up owning 8 scores of one head: the running max needs two
//    cross-lane steps (xor 16, xor 32) and the running sum stays lane-local
//    until the end. P^T is then already in the B-operand layout of
//    O^T = V^T.P^T; V^T comes from a per-wave LDS tile written transposed
//    (two tokens packed per dword).
//
// Memory layout per step (two pages = 32 tokens, tile t = page t):
//  K tile t, MFMA row r <- token 16t + r; lane (r, g) loads dims 32kk+8g..+7.
//  V: lane (r, g) loads tokens r and 16 + r of the same dims and writes the
//  pair (V[r][d], V[16+r][d]) as one dword at LDS column pair 2r of row d.
//  Column c of the V^T tile therefore holds token 16*(c&1) + (c>>1), and
//  lane (r, g) of the P.V MFMA reads columns 8g..8g+7 (16 bytes), i.e.
//  tokens 4g+i (t = 0) and 16+4g+i (t = 1), matching the P^T lane layout.
#include "common.h"

namespace tmopt {
namespace {

constexpr int kD = 128;
constexpr int kPS = 16;                      // tokens per page
constexpr int kVtRowBytes = 88;              // 64 B of tokens + 24 B pad
constexpr int kVtBytes = kD * kVtRowBytes;   // per wave

struct DecodeArgs {
  const __bf16* q;
  const __bf16* kpool;
  const __bf16* vpool;
  const int32_t* bt;
  int64_t bt_stride;
  int table_wrap;
  const int32_t* ctx_lens;
  int HQ, HKV;
  int64_t num_pages;
  int window;
  float scale_log2;  // scale * log2(e)
  const __bf16* rel;
  int rel_extent;
  int split_pages;
  int max_splits;
  __bf16* out;
  float* lse;
  float* part_o;    // [B, max_splits, HQ, D]
  float* part_lse;  // [B, max_splits, HQ]
};

struct SeqGeom {
  int n, lo, p_lo, p_hi, sp, nsplit;
};

// Visible key range and split geometry of one sequence; shared by the split
// kernel and the combine kernel so that both agree on every split.
__device__ __forceinline__ SeqGeom seq_geom(int n, int window,
                                            int split_pages, int max_splits) {
  SeqGeom g;
  g.n = n;
  g.lo = (window > 0 && n > window) ? n - window : 0;
  g.p_lo = g.lo / kPS;
  g.p_hi = (n + kPS - 1) / kPS;
  const int npg = n > 0 ? g.p_hi - g.p_lo : 0;
  // a sequence longer than max_splits * split_pages widens its splits, so a
  // fixed (graph-captured) grid always covers every page
  int sp = split_pages;
  const int need = (npg + max_splits - 1) / max_splits;
  if (need > sp) sp = need;
  g.sp = sp;
  g.nsplit = npg > 0 ? (npg + sp - 1) / sp : 0;
  return g;
}

__device__ __forceinline__ int page_id(const DecodeArgs& a, int b, int lp) {
  const int idx = a.table_wrap > 0 ? lp % a.table_wrap : lp;
  const int64_t v = a.bt[(int64_t)b * a.bt_stride + idx];
  return (v >= 0 && v < a.num_pages) ? (int)v : -1;
}

struct StepBuf {
  u32x4 k[2][4];  // [tile][kk]
  u32x4 v[2][4];  // [tile][kk]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const __bf16* pool,
                                                            int phys,
                                                            int page_bytes) {
  const char* base =
      reinterpret_cast<const char*>(pool) +
      (phys >= 0 ? (int64_t)phys * page_bytes : 0);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0,
                                           phys >= 0 ? page_bytes : 0,
                                           0x00020000);
}

// Issue the 16 buffer loads of one 32-token step.
__device__ __forceinline__ void issue_step(StepBuf& buf, const DecodeArgs& a,
                                           int phys0, int phys1,
                                           int lane_off, int page_bytes) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int phys = t == 0 ? phys0 : phys1;
    __amdgpu_buffer_rsrc_t rk = page_rsrc(a.kpool, phys, page_bytes);
    __amdgpu_buffer_rsrc_t rv = page_rsrc(a.vpool, phys, page_bytes);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      buf.k[t][kk] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, lane_off + 64 * kk,
                                                       0, 0));
      buf.v[t][kk] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, lane_off + 64 * kk,
                                                       0, 0));
    }
  }
}

template <int REP>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int r = lane & 15;  // MFMA row / column index
  const int g = lane >> 4;  // MFMA k-group
  const int b = blockIdx.z;
  const int s = blockIdx.x;
  const int kvh = blockIdx.y * nw + w;
  char* vt = smem + w * kVtBytes;

  const int n = a.ctx_lens[b];
  const SeqGeom geo = seq_geom(n, a.window, a.split_pages, a.max_splits);
  const int hq = kvh * REP + r;  // query head owned as MFMA column r
  const bool head_ok = r < REP;

  if (geo.nsplit == 0) {
    // no visible key: output 0, lse -inf (only split 0 writes)
    if (s == 0 && head_ok) {
      __bf16* o = a.out + ((int64_t)b * a.HQ + hq) * kD;
#pragma unroll
      for (int blk = 0; blk < 8; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[16 * blk + 4 * g + i] = (__bf16)0.0f;
      if (a.lse && g == 0) a.lse[(int64_t)b * a.HQ + hq] = -INFINITY;
    }
    return;
  }
  if (s >= geo.nsplit) return;
  const int pb = geo.p_lo + s * geo.sp;
  const int pe = min(pb + geo.sp, geo.p_hi);
  const int pos = n - 1;

  // Q fragment: B operand of S^T = K.Q^T (column = head r, k = dims)
  bf16x8 qf[4];
  {
    const __bf16* qrow = a.q + ((int64_t)b * a.HQ + (head_ok ? hq : 0)) * kD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 x = *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * g);
      if (!head_ok) x = u32x4{0, 0, 0, 0};
      qf[kk] = __builtin_bit_cast(bf16x8, x);
    }
  }

  const int row_elems = a.HKV * kD;
  const int page_bytes = kPS * row_elems * 2;
  // byte offset of (token r, head kvh, dims 8g..) inside a page
  const int lane_off = (r * row_elems + kvh * kD + 8 * g) * 2;

  f32x4 o_acc[8];
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) o_acc[blk] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY;
  float l_part = 0.0f;

  const __bf16* relrow =
      a.rel ? a.rel + ((int64_t)b * a.HQ + (head_ok ? hq : 0)) * a.rel_extent
            : nullptr;

  auto compute = [&](const StepBuf& buf, int pg, int phys0, int phys1) {
    // ---- S^T = K.Q^T for the two 16-token tiles -------------------------
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sc[t] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, buf.k[t][kk]), qf[kk], sc[t], 0, 0, 0);
    }
    // ---- mask, bias, running max ----------------------------------------
    // lane (r, g) holds head r, tokens 16t + 4g + i of this step
    float x[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bool page_ok = (t == 0 ? phys0 : phys1) >= 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kpos = (pg + t) * kPS + 4 * g + i;
        const bool ok = page_ok && kpos >= geo.lo && kpos < n;
        float v = sc[t][i] * a.scale_log2;
        if (relrow) {
          const int dist = pos - kpos;
          if (dist >= 0 && dist < a.rel_extent)
            v += (float)relrow[dist] * kLog2e;
        }
        v = ok ? v : -INFINITY;
        x[t][i] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    // ---- probabilities: fp32 sum, bf16 operand --------------------------
    float psum = 0.0f;
    uint32_t pw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = fast_exp2(x[0][i] - m_use);
      const float p1 = fast_exp2(x[1][i] - m_use);
      psum += p0 + p1;
      // B-operand element j = 2i + t  <->  token 16t + 4g + i
      pw[i] = pack_bf16x2(f32_to_bf16_bits(p0), f32_to_bf16_bits(p1));
    }
    l_part = l_part * alpha + psum;
    const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
    // ---- V^T into LDS (zero rows of invalid tokens: NaN-safe) -----------
    const bool v0_ok = phys0 >= 0 && (pg * kPS + r) >= geo.lo &&
                       (pg * kPS + r) < n;
    const bool v1_ok = phys1 >= 0 && ((pg + 1) * kPS + r) >= geo.lo &&
                       ((pg + 1) * kPS + r) < n;
    wave_lds_sync();  // previous step's V^T reads are done
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t a0 = v0_ok ? buf.v[0][kk][c] : 0u;
        const uint32_t a1 = v1_ok ? buf.v[1][kk][c] : 0u;
        const int d = 32 * kk + 8 * g + 2 * c;
        *reinterpret_cast<uint32_t*>(vt + d * kVtRowBytes + 4 * r) =
            interleave_lo(a0, a1);
        *reinterpret_cast<uint32_t*>(vt + (d + 1) * kVtRowBytes + 4 * r) =
            interleave_hi(a0, a1);
      }
    }
    wave_lds_sync();
    // ---- O^T = O^T * alpha + V^T.P^T ------------------------------------
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const char* src = vt + (16 * blk + r) * kVtRowBytes + 16 * g;
      const u32x2 lo2 = *reinterpret_cast<const u32x2*>(src);
      const u32x2 hi2 = *reinterpret_cast<const u32x2*>(src + 8);
      const bf16x8 vf =
          __builtin_bit_cast(bf16x8, u32x4{lo2[0], lo2[1], hi2[0], hi2[1]});
      o_acc[blk] = o_acc[blk] * alpha;
      o_acc[blk] =
          __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o_acc[blk], 0, 0, 0);
    }
  };

  StepBuf A, B;
  int phA0 = page_id(a, b, pb);
  int phA1 = pb + 1 < pe ? page_id(a, b, pb + 1) : -1;
  issue_step(A, a, phA0, phA1, lane_off, page_bytes);
  int pg = pb;
  while (true) {
    const int phB0 = pg + 2 < pe ? page_id(a, b, pg + 2) : -1;
    const int phB1 = pg + 3 < pe ? page_id(a, b, pg + 3) : -1;
    issue_step(B, a, phB0, phB1, lane_off, page_bytes);
    compute(A, pg, phA0, phA1);
    pg += 2;
    if (pg >= pe) break;
    phA0 = pg + 2 < pe ? page_id(a, b, pg + 2) : -1;
    phA1 = pg + 3 < pe ? page_id(a, b, pg + 3) : -1;
    issue_step(A, a, phA0, phA1, lane_off, page_bytes);
    compute(B, pg, phB0, phB1);
    pg += 2;
    if (pg >= pe) break;
  }

  // ---- finalise: total l over the 4 k-groups, normalise, store ----------
  float l_tot = l_part;
  l_tot += __shfl_xor(l_tot, 16);
  l_tot += __shfl_xor(l_tot, 32);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const float lse_nat =
      l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : -INFINITY;
  if (!head_ok) return;
  if (geo.nsplit == 1) {
    __bf16* o = a.out + ((int64_t)b * a.HQ + hq) * kD;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const uint32_t w0 = pack_bf16x2(f32_to_bf16_bits(o_acc[blk][0] * inv),
                                      f32_to_bf16_bits(o_acc[blk][1] * inv));
      const uint32_t w1 = pack_bf16x2(f32_to_bf16_bits(o_acc[blk][2] * inv),
                                      f32_to_bf16_bits(o_acc[blk][3] * inv));
      *reinterpret_cast<u32x2*>(o + 16 * blk + 4 * g) = u32x2{w0, w1};
    }
    if (a.lse && g == 0) a.lse[(int64_t)b * a.HQ + hq] = lse_nat;
  } else {
    const int64_t slot = ((int64_t)b * a.max_splits + s) * a.HQ + hq;
    float* po = a.part_o + slot * kD;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk)
      *reinterpret_cast<f32x4*>(po + 16 * blk + 4 * g) = o_acc[blk] * inv;
    if (g == 0) a.part_lse[slot] = lse_nat;
  }
}

// Merge the splits of every multi-split sequence: one wave per query head,
// two dims per lane. Fixed split order, so the result is deterministic.
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int hq = blockIdx.y * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int b = blockIdx.x;
  if (hq >= a.HQ) return;
  const SeqGeom geo =
      seq_geom(a.ctx_lens[b], a.window, a.split_pages, a.max_splits);
  if (geo.nsplit <= 1) return;
  const int64_t base = (int64_t)b * a.max_splits * a.HQ + hq;
  float m = -INFINITY;
  for (int s = 0; s < geo.nsplit; ++s)
    m = fmaxf(m, a.part_lse[base + (int64_t)s * a.HQ]);
  const float m_use = m == -INFINITY ? 0.0f : m;
  float sum = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < geo.nsplit; ++s) {
    const int64_t slot = base + (int64_t)s * a.HQ;
    const float wgt = fast_exp2((a.part_lse[slot] - m_use) * kLog2e);
    const float2 v =
        *reinterpret_cast<const float2*>(a.part_o + slot * kD + 2 * lane);
    sum += wgt;
    o0 += wgt * v.x;
    o1 += wgt * v.y;
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  __bf16* o = a.out + ((int64_t)b * a.HQ + hq) * kD + 2 * lane;
  *reinterpret_cast<uint32_t*>(o) =
      pack_bf16x2(f32_to_bf16_bits(o0 * inv), f32_to_bf16_bits(o1 * inv));
  if (a.lse && lane == 0)
    a.lse[(int64_t)b * a.HQ + hq] =
        sum > 0.0f ? m_use + fast_log2(sum) * kLn2 : -INFINITY;
}

size_t ws_bytes(int B, int HQ, int max_splits) {
  if (max_splits <= 1) return 0;
  const size_t slots = (size_t)B * max_splits * HQ;
  const size_t o_bytes = slots * kD * sizeof(float);
  return o_bytes + ((slots * sizeof(float) + 255) & ~(size_t)255);
}

template <int REP>
void launch_split(const DecodeArgs& a, int B, int nw, hipStream_t st) {
  dim3 grid(a.max_splits, a.HKV / nw, B);
  hipLaunchKernelGGL(decode_split_kernel<REP>, grid, dim3(64 * nw),
                     nw * kVtBytes, st, a);
}

}  // namespace
}  // namespace tmopt

using namespace tmopt;

extern "C" size_t tmopt_attn_decode_workspace_size(int B, int HQ, int D,
                                                   int max_splits) {
  (void)D;
  if (B <= 0 || HQ <= 0 || max_splits <= 0) return 0;
  return ws_bytes(B, HQ, max_splits);
}

extern "C" int tmopt_attn_decode_paged(
    const void* q, const void* k_pool, const void* v_pool,
    const int32_t* block_table, int64_t bt_stride, int table_wrap,
    const int32_t* ctx_lens, int B, int HQ, int HKV, int D, int page_size,
    int64_t num_pages, int window, float scale, const void* rel,
    int rel_extent, int split_pages, int max_splits, void* out, float* lse,
    void* workspace, size_t workspace_bytes, tmopt_stream_t stream) {
  clear_error();
  if (B == 0) return TMOPT_OK;
  TMOPT_REQUIRE(B > 0 && B <= 65535, TMOPT_EINVAL,
                "decode: B=%d outside [0, 65535]", B);
  TMOPT_REQUIRE(q && k_pool && v_pool && block_table && ctx_lens && out,
                TMOPT_EINVAL, "decode: null tensor pointer");
  TMOPT_REQUIRE(D == kD, TMOPT_EUNSUPPORTED, "decode: D=%d (only 128)", D);
  TMOPT_REQUIRE(page_size == kPS, TMOPT_EUNSUPPORTED,
                "decode: page_size=%d (only 16)", page_size);
  TMOPT_REQUIRE(HKV > 0 && HQ > 0 && HQ % HKV == 0, TMOPT_EINVAL,
                "decode: HQ=%d HKV=%d", HQ, HKV);
  const int rep = HQ / HKV;
  TMOPT_REQUIRE(rep == 1 || rep == 2 || rep == 4 || rep == 8 || rep == 16,
                TMOPT_EUNSUPPORTED, "decode: HQ/HKV=%d not in {1,2,4,8,16}",
                rep);
  TMOPT_REQUIRE((int64_t)kPS * HKV * kD * 2 < (1ll << 31), TMOPT_EUNSUPPORTED,
                "decode: page too large");
  TMOPT_REQUIRE(num_pages > 0 && bt_stride > 0 && table_wrap >= 0 &&
                    (table_wrap == 0 || table_wrap <= bt_stride),
                TMOPT_EINVAL,
                "decode: num_pages=%lld bt_stride=%lld table_wrap=%d",
                (long long)num_pages, (long long)bt_stride, table_wrap);
  TMOPT_REQUIRE(window >= 0, TMOPT_EINVAL, "decode: window=%d", window);
  TMOPT_REQUIRE(split_pages > 0 && max_splits > 0 && max_splits <= 65535,
                TMOPT_EINVAL, "decode: split_pages=%d max_splits=%d",
                split_pages, max_splits);
  TMOPT_REQUIRE(rel == nullptr || rel_extent > 0, TMOPT_EINVAL,
                "decode: rel_extent=%d", rel_extent);
  TMOPT_REQUIRE(((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool |
                 (uintptr_t)out) % 16 == 0,
                TMOPT_EINVAL, "decode: tensors must be 16-byte aligned");
  const size_t need = ws_bytes(B, HQ, max_splits);
  TMOPT_REQUIRE(need == 0 || (workspace && workspace_bytes >= need),
                TMOPT_EWORKSPACE, "decode: workspace %zu bytes < %zu needed",
                workspace_bytes, need);

  DecodeArgs a;
  a.q = (const __bf16*)q;
  a.kpool = (const __bf16*)k_pool;
  a.vpool = (const __bf16*)v_pool;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.table_wrap = table_wrap;
  a.ctx_lens = ctx_lens;
  a.HQ = HQ;
  a.HKV = HKV;
  a.num_pages = num_pages;
  a.window = window;
  a.scale_log2 = scale * kLog2e;
  a.rel = (const __bf16*)rel;
  a.rel_extent = rel ? rel_extent : 0;
  a.split_pages = split_pages;
  a.max_splits = max_splits;
  a.out = (__bf16*)out;
  a.lse = lse;
  a.part_o = need ? (float*)workspace : nullptr;
  a.part_lse = need ? (float*)((char*)workspace +
                               (size_t)B * max_splits * HQ * kD * sizeof(float))
                    : nullptr;

  const int nw = HKV % 4 == 0 ? 4 : (HKV % 2 == 0 ? 2 : 1);
  hipStream_t st = (hipStream_t)stream;
  switch (rep) {
    case 1: launch_split<1>(a, B, nw, st); break;
    case 2: launch_split<2>(a, B, nw, st); break;
    case 4: launch_split<4>(a, B, nw, st); break;
    case 8: launch_split<8>(a, B, nw, st); break;
    default: launch_split<16>(a, B, nw, st); break;
  }
  int rc = check_launch("decode_split");
  if (rc) return rc;
  if (max_splits > 1) {
    dim3 grid(B, (HQ + 3) / 4);
    hipLaunchKernelGGL(decode_combine_kernel, grid, dim3(256), 0, st, a);
    rc = check_launch("decode_combine");
  }
  return rc;
}
