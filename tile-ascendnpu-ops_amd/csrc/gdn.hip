// Gated delta-rule chunked prefill for gfx950 (tileops_gdn_prefill_fwd): kernel in progress.
#include "common.h"

extern "C" int tileops_gdn_prefill_fwd(const void*, const void*, const void*, const float*,
                                       const float*, const float*, void*, float*, int64_t,
                                       int64_t, int64_t, int64_t, int64_t, int64_t, float, int,
                                       void*, size_t, void*) {
  return TILEOPS_EINVAL;
}

extern "C" size_t tileops_gdn_prefill_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t,
                                                      int64_t) {
  return 0;
}
