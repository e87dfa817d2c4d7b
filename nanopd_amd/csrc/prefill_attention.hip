// Chunked-prefill attention over a paged prefix plus the new chunk (MFMA).
#include "common.h"

extern "C" int64_t npd_paged_prefill_workspace_size(int64_t, int64_t, int64_t, int64_t, int64_t,
                                                    int64_t) {
  return 0;
}

extern "C" int npd_paged_prefill_attention(void*, const void*, const void*, const void*,
                                           const int32_t*, const int32_t*, const int32_t*, int64_t,
                                           int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                           int64_t, int64_t, int64_t, float, int64_t, int64_t,
                                           int64_t, int64_t, void*, int64_t, int32_t, void*) {
  return npd::fail(NPD_E_INVALID, "npd_paged_prefill_attention: not built yet");
}
