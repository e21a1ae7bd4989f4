// Library-wide entry points of the C ABI: version and error strings.
#include "common.h"

extern "C" int tileops_version(void) { return 100; }

extern "C" const char* tileops_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case TILEOPS_EINVAL: return "tileops: invalid dtype, operator selector or flags";
    case TILEOPS_ESHAPE: return "tileops: unsupported or negative size";
    case TILEOPS_ENULL: return "tileops: null pointer for a non-empty tensor";
    case TILEOPS_EWORKSPACE: return "tileops: workspace missing or too small";
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "tileops: unknown error";
}
