// Fused paged KV-cache write for gfx950.
//
// Replaces the reference's torch index_put_ appends
// (engine/pyengine/model.py:938-948 decode, engine/pyengine/kv.py:89-103 and
// :193-205 prefill). Pure byte movement: a lane moves 16-byte chunks of K
// and the same chunks of V (consecutive lanes, consecutive chunks of a
// token row), so global reads and writes are fully coalesced. Bit-exact.
// Index math is 32-bit: the 64-bit divisions of a first version cost more
// than the copy.
#include "common.h"

namespace tmopt {
namespace {

// One lane = one 16-byte chunk (8 bf16) of one (token, kv-head) row.
__global__ __launch_bounds__(256) void kv_write_slots_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, int64_t k_st,
    int64_t k_sh, int64_t v_st, int64_t v_sh,
    const int64_t* __restrict__ slots, int64_t T, int HKV, int D16,
    u32x4* __restrict__ kp, u32x4* __restrict__ vp, int64_t pool_rows) {
  // 32-bit index math (the host keeps T * HKV * D16 below 2^31)
  const int per_tok = HKV * D16;
  const int gid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const int t = gid / per_tok;
  if (t >= T) return;
  const int rem = gid - t * per_tok;
  const int h = rem / D16;
  const int c = rem - h * D16;
  const int64_t row = slots[t];
  if (row < 0 || row >= pool_rows) return;
  const int64_t dst = (row * HKV + h) * D16 + c;
  kp[dst] = k[t * k_st + h * k_sh + c];
  vp[dst] = v[t * v_st + h * v_sh + c];
}

// grid = (ceil(max_seqlen * per_tok / (256 R)), num_seqs): work-group x of
// sequence seq covers chunks [256 R x, 256 R (x+1)) of that sequence's
// tokens (chunk = 16 bytes of one (token, kv-head) row), lane i the chunks
// 256 R x + 256 p + i, p < R. Token positions and pages are derived
// in-kernel from cu_seqlens/start_pos/block_table. The grid is sized by the
// longest run, so R > 1 keeps a call with a few long runs and many one-token
// rows (a mixed prefill + decode step) from dispatching tens of thousands of
// empty work-groups; every load of a work-group (table entries, K and V) is
// issued before its first store.
//
// Rows of a batch (`lens` given): sequence seq's tokens are rows
// 0 .. lens[seq]-1 of its own source block, k + seq * k_sb (k_sb, v_sb in
// 16-byte chunks), instead of rows cu_seqlens[seq] .. of one packed source.
template <int R>
__global__ __launch_bounds__(256) void kv_write_paged_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, int64_t k_st,
    int64_t k_sh, int64_t v_st, int64_t v_sh,
    const int32_t* __restrict__ cu_seqlens,
    const int32_t* __restrict__ lens, int64_t k_sb, int64_t v_sb,
    const int32_t* __restrict__ start_pos,
    const int32_t* __restrict__ block_table, int64_t bt_stride,
    int table_wrap, int page_size, int HKV, int D16, u32x4* __restrict__ kp,
    u32x4* __restrict__ vp, int64_t num_pages) {
  const int seq = blockIdx.y;
  const int per_tok = HKV * D16;
  int t0 = seq, len = 1;
  if (lens != nullptr) {
    t0 = 0;
    len = lens[seq];
    k += seq * k_sb;
    v += seq * v_sb;
  } else if (cu_seqlens != nullptr) {
    t0 = cu_seqlens[seq];
    len = cu_seqlens[seq + 1] - t0;
  }
  // 32-bit index math (the host keeps max_seqlen * per_tok below 2^31;
  // positions are int32)
  const int base = blockIdx.x * (256 * R);
  if (base >= len * per_tok) return;
  const int p0 = start_pos[seq];
  // Ring pools keep only the last table_wrap*page_size positions: a token
  // that a later token of this same call overwrites is dropped, so the
  // parallel scatter has no write-write race (kv.py:97-98).
  const int keep_from = table_wrap > 0 ? p0 + len - table_wrap * page_size : 0;
  const int32_t* trow = block_table + (int64_t)seq * bt_stride;
  int page[R], off[R];
  u32x4 kx[R], vx[R];
  // branch-free, and nothing waits for a load before every load of the
  // work-group is out: a chunk that writes nothing reads from a valid
  // dummy address (the run's first row, table entry 0) and gets off = -1;
  // off = the chunk's offset inside its page row set, page = table entry
#pragma unroll
  for (int p = 0; p < R; ++p) {
    const int gid = base + 256 * p + (int)threadIdx.x;
    const int tl = gid / per_tok;
    const int pos = p0 + tl;
    const bool live = tl < len && pos >= 0 && pos >= keep_from;
    int lp = live ? pos / page_size : 0;
    if (table_wrap > 0) lp %= table_wrap;
    // a logical page past the row's width has no entry (reading on would
    // return the next row's page ids): the token is skipped
    page[p] = (int64_t)lp < bt_stride ? trow[lp] : -1;
    const int rem = live ? gid - tl * per_tok : 0;
    const int h = rem / D16;
    const int c = rem - h * D16;
    const int64_t t = t0 + (live ? tl : 0);
    kx[p] = k[t * k_st + h * k_sh + c];
    vx[p] = v[t * v_st + h * v_sh + c];
    off[p] = live ? ((pos % page_size) * HKV + h) * D16 + c : -1;
  }
  asm volatile("" ::: "memory");   // every load above goes out first
  const int64_t page_chunks = (int64_t)page_size * HKV * D16;
#pragma unroll
  for (int p = 0; p < R; ++p) {
    if (off[p] < 0 || page[p] < 0 || page[p] >= num_pages) continue;
    const int64_t dst = (int64_t)page[p] * page_chunks + off[p];
    kp[dst] = kx[p];
    vp[dst] = vx[p];
  }
}

// ---- channel-major input ------------------------------------------------
// K / V whose tokens are contiguous and whose head_dim is strided (the
// sconv's output layout in the reference's prefill, where the cache append
// receives views [T, HK, D] with strides (1, D*T, T): model.py:486-512,
// experiments/DEADENDS.md:631-645). A work-group moves 64 tokens x 128
// dims of one KV head for K and for V: coalesced 16-byte loads along the
// tokens of one dim into an LDS tile [128 dims][64 tokens], then transposed
// LDS reads (ds_read_b64_tr_b16: 4 dims of one token per lane and read)
// give each lane 8 dims of one token, stored as one 16-byte chunk of the
// token's page row. Bit-exact.
//
// LDS rows are 128 bytes (64 tokens of one dim), two per 256-byte bank row;
// the 16-byte chunk c of dim row d sits at slot c ^ swz(d), swz(d) =
// h((d >> 1) & 7), h(x) = ((x & 1) << 2) | (x >> 1): the 8 rows of one
// parity among 16 consecutive rows get distinct slots (row-chunk writes do
// not conflict), and rows d0, d0 + 2 (d0 % 4 == 0) get slots from opposite
// halves (a transposed read of 4 rows x 32 tokens does not conflict).
constexpr int kCmTok = 64;     // tokens per work-group
constexpr int kCmD = 128;      // head_dim of the channel-major path

__device__ __forceinline__ uint32_t cm_slot(int d, int c) {
  const int x = (d >> 1) & 7;
  return (uint32_t)(c ^ (((x & 1) << 2) | (x >> 1)));
}

// grid (tiles, num_seqs, HKV), 256 threads
// (rows of a batch: `lens` and the row strides k_sb / v_sb in elements,
// as in kv_write_paged_kernel)
__global__ __launch_bounds__(256) void kv_write_paged_cm_kernel(
    const __bf16* __restrict__ k, const __bf16* __restrict__ v, int64_t k_sh,
    int64_t k_sd, int64_t v_sh, int64_t v_sd,
    const int32_t* __restrict__ cu_seqlens,
    const int32_t* __restrict__ lens, int64_t k_sb, int64_t v_sb,
    const int32_t* __restrict__ start_pos,
    const int32_t* __restrict__ block_table, int64_t bt_stride,
    int table_wrap, int page_size, int HKV, u32x4* __restrict__ kp,
    u32x4* __restrict__ vp, int64_t num_pages) {
  __shared__ __align__(16) char tile[2][kCmD * kCmTok * 2];   // K, V: 32 KB
  const int seq = blockIdx.y;
  const int h = blockIdx.z;
  int t0 = seq, len = 1;
  if (lens != nullptr) {
    t0 = 0;
    len = lens[seq];
    k += seq * k_sb;
    v += seq * v_sb;
  } else if (cu_seqlens != nullptr) {
    t0 = cu_seqlens[seq];
    len = cu_seqlens[seq + 1] - t0;
  }
  // tiles start at a multiple of 8 tokens (16-byte aligned loads): the first
  // one may hold up to 7 rows before the run, the last rows after it; those
  // are loaded (inside the tensor, or zeros past the run's last row) and
  // never stored
  const int a0 = (t0 & ~7) + kCmTok * (int)blockIdx.x;
  if (a0 >= t0 + len) return;
  const int tid = threadIdx.x;
  // one resource per head: rows up to the run's end; the last dim's rows
  // after it read as zeros. The range check is per dword (a dword that
  // straddles the end reads as zero), so the range is rounded up to the
  // dword holding the run's last token: at most 2 bytes past the run,
  // never past a mapped page (page ends are dword aligned)
  const uint32_t nrec_k =
      (uint32_t)((((int64_t)(kCmD - 1) * k_sd + t0 + len) * 2 + 3) & ~3ll);
  const uint32_t nrec_v =
      (uint32_t)((((int64_t)(kCmD - 1) * v_sd + t0 + len) * 2 + 3) & ~3ll);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(k + (int64_t)h * k_sh), (short)0, nrec_k,
      0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(v + (int64_t)h * v_sh), (short)0, nrec_v,
      0x00020000);
  // loads: chunk c = tid + 256 j -> dim c >> 3, tokens a0 + 8 (c & 7) .. +7
  u32x4 xk[4], xv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = tid + 256 * j;
    const int d = c >> 3, t8 = c & 7;
    xk[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rk, (int)((d * k_sd + a0 + 8 * t8) * 2), 0, 0));
    xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rv, (int)((d * v_sd + a0 + 8 * t8) * 2), 0, 0));
  }
  const uint32_t lk =
      (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)tile[0]);
  const uint32_t lv =
      (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)tile[1]);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = tid + 256 * j;
    const int d = c >> 3, t8 = c & 7;
    const uint32_t off = d * 128 + 16 * cm_slot(d, t8);
    lds_st128(lk + off, xk[j]);
    lds_st128(lv + off, xv[j]);
  }
  __syncthreads();
  // transposed reads: 16-lane group G (of 16) takes tokens 16 (G & 3) ..+15
  // and dims 32 (G >> 2) .. +31; source lane s = 4 jj + m of the group names
  // dim row d0 + jj, tokens 16 (G & 3) + 4 m .. +3, and lane i then holds
  // dims d0 .. d0 + 3 of token 16 (G & 3) + i
  const int lane = tid & 63;
  const int G = (tid >> 6) * 4 + (lane >> 4);
  const int i = lane & 15;
  const int jj = i >> 2, m = i & 3;
  const int tb = G & 3;
  const int tok = 16 * tb + i;                    // token of this lane
  const int chunk = 2 * tb + (m >> 1);            // 16-byte chunk it names
  const int gtok = a0 + tok;
  const int p0 = start_pos[seq];
  const int keep_from = table_wrap > 0 ? p0 + len - table_wrap * page_size : 0;
  const int pos = p0 + (gtok - t0);
  const bool live = gtok >= t0 && gtok < t0 + len && pos >= 0 &&
                    pos >= keep_from;
  int page = -1;
  if (live) {
    int lp = pos / page_size;
    if (table_wrap > 0) lp %= table_wrap;
    if ((int64_t)lp < bt_stride) page = block_table[(int64_t)seq * bt_stride + lp];
  }
  const int64_t D16 = kCmD / 8;
  const int64_t row = (int64_t)page * page_size + pos % page_size;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int dq = 32 * (G >> 2) + 8 * q;
    u32x4 ok, ov;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int d = dq + 4 * half + jj;         // the row this lane names
      const uint32_t off = d * 128 + 16 * cm_slot(d, chunk) + 8 * (m & 1);
      const bf16x4 a = lds_tr16(lk + off);
      const bf16x4 b = lds_tr16(lv + off);
      const u32x2 ua = __builtin_bit_cast(u32x2, a);
      const u32x2 ub = __builtin_bit_cast(u32x2, b);
      ok[2 * half] = ua[0];
      ok[2 * half + 1] = ua[1];
      ov[2 * half] = ub[0];
      ov[2 * half + 1] = ub[1];
    }
    if (page >= 0 && page < num_pages) {
      const int64_t dst = (row * HKV + h) * D16 + (dq >> 3);
      kp[dst] = ok;
      vp[dst] = ov;
    }
  }
}

int check_kv_common(const void* k, const void* v, int64_t k_st, int64_t k_sh,
                    int64_t v_st, int64_t v_sh, int HKV, int D,
                    const void* kp, const void* vp) {
  TMOPT_REQUIRE(k && v && kp && vp, TMOPT_EINVAL,
                "kv_write: null tensor pointer");
  TMOPT_REQUIRE(HKV > 0 && D > 0, TMOPT_EINVAL, "kv_write: HKV=%d D=%d", HKV,
                D);
  TMOPT_REQUIRE(D % 8 == 0, TMOPT_EUNSUPPORTED,
                "kv_write: D=%d must be a multiple of 8", D);
  TMOPT_REQUIRE(k_st % 8 == 0 && k_sh % 8 == 0 && v_st % 8 == 0 &&
                    v_sh % 8 == 0,
                TMOPT_EUNSUPPORTED,
                "kv_write: token/head strides must be multiples of 8 "
                "elements (16-byte rows)");
  TMOPT_REQUIRE(((uintptr_t)k | (uintptr_t)v | (uintptr_t)kp |
                 (uintptr_t)vp) % 16 == 0,
                TMOPT_EINVAL, "kv_write: pointers must be 16-byte aligned");
  return TMOPT_OK;
}

}  // namespace
}  // namespace tmopt

using namespace tmopt;

extern "C" int tmopt_kv_write_slots(const void* k, const void* v,
                                    int64_t k_stride_tok, int64_t k_stride_head,
                                    int64_t v_stride_tok, int64_t v_stride_head,
                                    const int64_t* slot_mapping, int64_t T,
                                    int HKV, int D, void* k_pool, void* v_pool,
                                    int64_t pool_rows, tmopt_stream_t stream) {
  clear_error();
  if (T == 0) return TMOPT_OK;
  TMOPT_REQUIRE(T > 0 && slot_mapping, TMOPT_EINVAL,
                "kv_write_slots: T=%lld, slot_mapping=%p", (long long)T,
                (const void*)slot_mapping);
  int st = check_kv_common(k, v, k_stride_tok, k_stride_head, v_stride_tok,
                           v_stride_head, HKV, D, k_pool, v_pool);
  if (st) return st;
  const int D16 = D / 8;
  const int64_t work = T * HKV * D16;
  const int64_t blocks = (work + 255) / 256;
  TMOPT_REQUIRE(work + 256 < (1ll << 31), TMOPT_EINVAL,
                "kv_write_slots: T * HKV * D / 8 must stay below 2^31");
  hipLaunchKernelGGL(kv_write_slots_kernel, dim3((unsigned)blocks), dim3(256),
                     0, (hipStream_t)stream, (const u32x4*)k, (const u32x4*)v,
                     k_stride_tok / 8, k_stride_head / 8, v_stride_tok / 8,
                     v_stride_head / 8, slot_mapping, T, HKV, D16,
                     (u32x4*)k_pool, (u32x4*)v_pool, pool_rows);
  return check_launch("kv_write_slots");
}

// The paged write behind both entry points: runs of one packed source
// (cu_seqlens; null: one token per sequence) or rows of a batch (lens and
// the row strides k_sb / v_sb, in elements).
static int write_paged(
    const void* k, const void* v, int64_t k_stride_tok, int64_t k_stride_head,
    int64_t k_stride_dim, int64_t v_stride_tok, int64_t v_stride_head,
    int64_t v_stride_dim, const int32_t* cu_seqlens, const int32_t* lens,
    int64_t k_sb, int64_t v_sb, const int32_t* start_pos, int num_seqs,
    int max_seqlen, const int32_t* block_table, int64_t bt_stride,
    int table_wrap, int page_size, int HKV, int D, void* k_pool, void* v_pool,
    int64_t num_pages, tmopt_stream_t stream) {
  clear_error();
  if (num_seqs == 0) return TMOPT_OK;
  TMOPT_REQUIRE(num_seqs > 0 && num_seqs <= 65535, TMOPT_EINVAL,
                "kv_write_paged: num_seqs=%d outside [0, 65535]", num_seqs);
  TMOPT_REQUIRE(start_pos && block_table, TMOPT_EINVAL,
                "kv_write_paged: start_pos and block_table are required");
  TMOPT_REQUIRE(page_size > 0 && table_wrap >= 0 && bt_stride > 0,
                TMOPT_EINVAL,
                "kv_write_paged: page_size=%d table_wrap=%d bt_stride=%lld",
                page_size, table_wrap, (long long)bt_stride);
  TMOPT_REQUIRE(table_wrap == 0 || table_wrap <= bt_stride, TMOPT_EINVAL,
                "kv_write_paged: table_wrap=%d exceeds bt_stride=%lld",
                table_wrap, (long long)bt_stride);
  TMOPT_REQUIRE(lens == nullptr || (k_sb >= 0 && v_sb >= 0 &&
                                    k_sb % 8 == 0 && v_sb % 8 == 0),
                TMOPT_EUNSUPPORTED,
                "kv_write_paged: row strides must be multiples of 8 elements "
                "(k %lld, v %lld)", (long long)k_sb, (long long)v_sb);
  if (cu_seqlens == nullptr && lens == nullptr) max_seqlen = 1;
  TMOPT_REQUIRE(max_seqlen >= 0, TMOPT_EINVAL, "kv_write_paged: max_seqlen=%d",
                max_seqlen);
  if (max_seqlen == 0) return TMOPT_OK;
  if (k_stride_dim != 1 || v_stride_dim != 1) {
    // channel-major rows: tokens contiguous, head_dim strided
    TMOPT_REQUIRE(k && v && k_pool && v_pool, TMOPT_EINVAL,
                  "kv_write_paged: null tensor pointer");
    TMOPT_REQUIRE(D == kCmD && HKV > 0 && HKV <= 65535, TMOPT_EUNSUPPORTED,
                  "kv_write_paged: channel-major rows need D=%d (got %d)",
                  kCmD, D);
    TMOPT_REQUIRE(k_stride_tok == 1 && v_stride_tok == 1 &&
                      k_stride_dim % 8 == 0 && v_stride_dim % 8 == 0 &&
                      k_stride_head % 8 == 0 && v_stride_head % 8 == 0 &&
                      ((uintptr_t)k | (uintptr_t)v) % 16 == 0,
                  TMOPT_EUNSUPPORTED,
                  "kv_write_paged: strided head_dim needs contiguous tokens "
                  "and 16-byte aligned dim rows (strides tok=%lld dim=%lld "
                  "head=%lld)", (long long)k_stride_tok,
                  (long long)k_stride_dim, (long long)k_stride_head);
    TMOPT_REQUIRE(((uintptr_t)k_pool | (uintptr_t)v_pool) % 16 == 0,
                  TMOPT_EINVAL, "kv_write_paged: pools must be 16-byte aligned");
    // a dim row holds the tokens of every run (token index < dim stride),
    // so a head's 128 rows span 128 strides: 32-bit byte offsets
    TMOPT_REQUIRE(((int64_t)kCmD * (k_stride_dim > v_stride_dim
                                        ? k_stride_dim
                                        : v_stride_dim) +
                   2 * kCmTok) * 2 < (1ll << 31),
                  TMOPT_EUNSUPPORTED,
                  "kv_write_paged: a head's channel-major span must stay "
                  "below 2 GiB");
    const int64_t tiles = ((int64_t)max_seqlen + 7 + kCmTok - 1) / kCmTok;
    hipLaunchKernelGGL(kv_write_paged_cm_kernel,
                       dim3((unsigned)tiles, num_seqs, HKV), dim3(256), 0,
                       (hipStream_t)stream, (const __bf16*)k,
                       (const __bf16*)v, k_stride_head, k_stride_dim,
                       v_stride_head, v_stride_dim, cu_seqlens, lens, k_sb,
                       v_sb, start_pos, block_table, bt_stride, table_wrap,
                       page_size, HKV,
                       (u32x4*)k_pool, (u32x4*)v_pool, num_pages);
    return check_launch("kv_write_paged (channel-major)");
  }
  int st = check_kv_common(k, v, k_stride_tok, k_stride_head, v_stride_tok,
                           v_stride_head, HKV, D, k_pool, v_pool);
  if (st) return st;
  const int D16 = D / 8;
  const int64_t work = (int64_t)max_seqlen * HKV * D16;
  // chunks per lane: the smallest power of two (up to 16) that keeps the
  // grid within 32768 work-groups. Measured on config 5's append (2 runs of
  // 2048 tokens + 96 one-token rows, graph replays): 1 chunk per lane (50K
  // work-groups, mostly empty) 13.4 us, 2: 9.0 us, 4: 11.0 us, 16: 37 us
  // (too few busy work-groups for the long runs)
  int R = 1;
  for (;;) {
    const int64_t bx_r = (work + 256 * R - 1) / (256 * R);
    if (R == 16 || bx_r == 1 || bx_r * num_seqs <= 32768) break;
    R *= 2;
  }
  const int64_t bx = (work + 256 * R - 1) / (256 * R);
  TMOPT_REQUIRE(work + 256 * R < (1ll << 31), TMOPT_EINVAL,
                "kv_write_paged: max_seqlen * HKV * D / 8 must stay below "
                "2^31");
  const dim3 grid((unsigned)bx, num_seqs);
  hipStream_t hs = (hipStream_t)stream;
#define TMOPT_KVW(RR)                                                        \
  hipLaunchKernelGGL(kv_write_paged_kernel<RR>, grid, dim3(256), 0, hs,       \
                     (const u32x4*)k, (const u32x4*)v, k_stride_tok / 8,     \
                     k_stride_head / 8, v_stride_tok / 8, v_stride_head / 8, \
                     cu_seqlens, lens, k_sb / 8, v_sb / 8, start_pos,        \
                     block_table, bt_stride,                                 \
                     table_wrap, page_size, HKV, D16, (u32x4*)k_pool,        \
                     (u32x4*)v_pool, num_pages)
  switch (R) {
    case 1: TMOPT_KVW(1); break;
    case 2: TMOPT_KVW(2); break;
    case 4: TMOPT_KVW(4); break;
    case 8: TMOPT_KVW(8); break;
    default: TMOPT_KVW(16); break;
  }
#undef TMOPT_KVW
  return check_launch("kv_write_paged");
}

extern "C" int tmopt_kv_write_paged(
    const void* k, const void* v, int64_t k_stride_tok, int64_t k_stride_head,
    int64_t k_stride_dim, int64_t v_stride_tok, int64_t v_stride_head,
    int64_t v_stride_dim, const int32_t* cu_seqlens,
    const int32_t* start_pos, int num_seqs, int max_seqlen,
    const int32_t* block_table, int64_t bt_stride, int table_wrap,
    int page_size, int HKV, int D, void* k_pool, void* v_pool,
    int64_t num_pages, tmopt_stream_t stream) {
  return write_paged(k, v, k_stride_tok, k_stride_head, k_stride_dim,
                     v_stride_tok, v_stride_head, v_stride_dim, cu_seqlens,
                     nullptr, 0, 0, start_pos, num_seqs, max_seqlen,
                     block_table, bt_stride, table_wrap, page_size, HKV, D,
                     k_pool, v_pool, num_pages, stream);
}

extern "C" int tmopt_kv_append_rows(
    const void* k, const void* v, int64_t k_stride_row, int64_t k_stride_tok,
    int64_t k_stride_head, int64_t k_stride_dim, int64_t v_stride_row,
    int64_t v_stride_tok, int64_t v_stride_head, int64_t v_stride_dim,
    const int32_t* lens, const int32_t* start_pos, int num_rows,
    int max_len, const int32_t* block_table, int64_t bt_stride,
    int table_wrap, int page_size, int HKV, int D, void* k_pool, void* v_pool,
    int64_t num_pages, tmopt_stream_t stream) {
  clear_error();
  TMOPT_REQUIRE(num_rows <= 0 || lens != nullptr, TMOPT_EINVAL,
                "kv_append_rows: lens is required");
  return write_paged(k, v, k_stride_tok, k_stride_head, k_stride_dim,
                     v_stride_tok, v_stride_head, v_stride_dim, nullptr, lens,
                     k_stride_row, v_stride_row, start_pos, num_rows, max_len,
                     block_table, bt_stride, table_wrap, page_size, HKV, D,
                     k_pool, v_pool, num_pages, stream);
}
