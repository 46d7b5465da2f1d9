// Fused paged KV-cache write for gfx950.
//
// Replaces the reference's torch index_put_ appends
// (engine/pyengine/model.py:938-948 decode, engine/pyengine/kv.py:89-103 and
// :193-205 prefill). Pure byte movement: every lane moves one 16-byte chunk
// of K and the same chunk of V, so one wave covers 1 KB of a token row and
// global reads and writes are fully coalesced. HBM-bound; bit-exact.
#include "common.h"

namespace tmopt {
namespace {

// One lane = one 16-byte chunk (8 bf16) of one (token, kv-head) row.
__global__ __launch_bounds__(256) void kv_write_slots_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, int64_t k_st,
    int64_t k_sh, int64_t v_st, int64_t v_sh,
    const int64_t* __restrict__ slots, int64_t T, int HKV, int D16,
    u32x4* __restrict__ kp, u32x4* __restrict__ vp, int64_t pool_rows) {
  const int64_t per_tok = (int64_t)HKV * D16;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t t = gid / per_tok;
  if (t >= T) return;
  const int rem = (int)(gid - t * per_tok);
  const int h = rem / D16;
  const int c = rem - h * D16;
  const int64_t row = slots[t];
  if (row < 0 || row >= pool_rows) return;
  const int64_t dst = (row * HKV + h) * D16 + c;
  kp[dst] = k[t * k_st + h * k_sh + c];
  vp[dst] = v[t * v_st + h * v_sh + c];
}

// grid = (ceil(max_seqlen * per_tok / 256), num_seqs). Token positions and
// pages are derived in-kernel from cu_seqlens/start_pos/block_table.
__global__ __launch_bounds__(256) void kv_write_paged_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, int64_t k_st,
    int64_t k_sh, int64_t v_st, int64_t v_sh,
    const int32_t* __restrict__ cu_seqlens,
    const int32_t* __restrict__ start_pos,
    const int32_t* __restrict__ block_table, int64_t bt_stride,
    int table_wrap, int page_size, int HKV, int D16, u32x4* __restrict__ kp,
    u32x4* __restrict__ vp, int64_t num_pages) {
  const int seq = blockIdx.y;
  const int per_tok = HKV * D16;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t tl = gid / per_tok;
  int64_t t0 = seq, len = 1;
  if (cu_seqlens != nullptr) {
    t0 = cu_seqlens[seq];
    len = (int64_t)cu_seqlens[seq + 1] - t0;
  }
  if (tl >= len) return;
  const int64_t pos = (int64_t)start_pos[seq] + tl;
  if (pos < 0) return;
  // Ring pools keep only the last table_wrap*page_size positions: a token
  // that a later token of this same call overwrites is dropped, so the
  // parallel scatter has no write-write race (kv.py:97-98).
  if (table_wrap > 0 &&
      pos < (int64_t)start_pos[seq] + len - (int64_t)table_wrap * page_size)
    return;
  int64_t lp = pos / page_size;
  if (table_wrap > 0) lp %= table_wrap;
  const int64_t page = block_table[(int64_t)seq * bt_stride + lp];
  if (page < 0 || page >= num_pages) return;
  const int64_t row = page * page_size + pos % page_size;
  const int rem = (int)(gid - tl * per_tok);
  const int h = rem / D16;
  const int c = rem - h * D16;
  const int64_t t = t0 + tl;
  const int64_t dst = (row * HKV + h) * D16 + c;
  kp[dst] = k[t * k_st + h * k_sh + c];
  vp[dst] = v[t * v_st + h * v_sh + c];
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
  TMOPT_REQUIRE(blocks < (1ll << 31), TMOPT_EINVAL, "kv_write_slots: T too large");
  hipLaunchKernelGGL(kv_write_slots_kernel, dim3((unsigned)blocks), dim3(256),
                     0, (hipStream_t)stream, (const u32x4*)k, (const u32x4*)v,
                     k_stride_tok / 8, k_stride_head / 8, v_stride_tok / 8,
                     v_stride_head / 8, slot_mapping, T, HKV, D16,
                     (u32x4*)k_pool, (u32x4*)v_pool, pool_rows);
  return check_launch("kv_write_slots");
}

extern "C" int tmopt_kv_write_paged(
    const void* k, const void* v, int64_t k_stride_tok, int64_t k_stride_head,
    int64_t v_stride_tok, int64_t v_stride_head, const int32_t* cu_seqlens,
    const int32_t* start_pos, int num_seqs, int max_seqlen,
    const int32_t* block_table, int64_t bt_stride, int table_wrap,
    int page_size, int HKV, int D, void* k_pool, void* v_pool,
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
  if (cu_seqlens == nullptr) max_seqlen = 1;
  TMOPT_REQUIRE(max_seqlen >= 0, TMOPT_EINVAL, "kv_write_paged: max_seqlen=%d",
                max_seqlen);
  if (max_seqlen == 0) return TMOPT_OK;
  int st = check_kv_common(k, v, k_stride_tok, k_stride_head, v_stride_tok,
                           v_stride_head, HKV, D, k_pool, v_pool);
  if (st) return st;
  const int D16 = D / 8;
  const int64_t work = (int64_t)max_seqlen * HKV * D16;
  const int64_t bx = (work + 255) / 256;
  TMOPT_REQUIRE(bx < (1ll << 31), TMOPT_EINVAL,
                "kv_write_paged: max_seqlen too large");
  hipLaunchKernelGGL(kv_write_paged_kernel, dim3((unsigned)bx, num_seqs),
                     dim3(256), 0, (hipStream_t)stream, (const u32x4*)k,
                     (const u32x4*)v, k_stride_tok / 8, k_stride_head / 8,
                     v_stride_tok / 8, v_stride_head / 8, cu_seqlens,
                     start_pos, block_table, bt_stride, table_wrap, page_size,
                     HKV, D16, (u32x4*)k_pool, (u32x4*)v_pool, num_pages);
  return check_launch("kv_write_paged");
}
