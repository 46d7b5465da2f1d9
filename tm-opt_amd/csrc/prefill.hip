// Varlen causal prefill attention (bf16 MFMA) — entry point placeholder
// until the kernel lands; reports TMOPT_EUNSUPPORTED.
#include "common.h"

extern "C" int tmopt_attn_prefill_varlen(
    const void*, int64_t, int64_t, const void*, int64_t, int64_t, const void*,
    int64_t, int64_t, const int32_t*, const int32_t*, int, int, const void*,
    const void*, const int32_t*, int64_t, int, int64_t, int, int, int, int,
    float, void*, int64_t, int64_t, float*, tmopt_stream_t) {
  tmopt::set_error("prefill_varlen: not built yet");
  return TMOPT_EUNSUPPORTED;
}
