// Flash-attention forward for gfx950 (tileops_mha_fwd): kernel in progress.
#include "common.h"

extern "C" int tileops_mha_fwd(const void*, const void*, const void*, void*, float*, int64_t,
                               int64_t, int64_t, int64_t, int64_t, int64_t, int, float, int,
                               void*) {
  return TILEOPS_EINVAL;
}
