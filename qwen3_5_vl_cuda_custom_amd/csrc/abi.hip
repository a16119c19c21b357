// Version and error-string entry points of the C-ABI.
#include "q3_common.h"

extern "C" {

int q3_abi_version(void) { return Q3VL_ABI_VERSION; }

const char* q3_error_string(int code) {
  switch (code) {
    case Q3_OK:
      return "ok";
    case Q3_ERR_NULL:
      return "a required pointer is null";
    case Q3_ERR_SHAPE:
      return "inconsistent or negative sizes";
    case Q3_ERR_DTYPE:
      return "dtype not supported by this op";
    case Q3_ERR_ALIGN:
      return "pointer or stride alignment violated";
    case Q3_ERR_UNSUPPORTED:
      return "request outside what the kernels cover";
    case Q3_ERR_WORKSPACE:
      return "workspace missing or too small";
    case Q3_ERR_SCRATCH:
      return "request needs more than the static scratch buffer of the allocation-free entry point";
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown q3 status";
  }
}

}  // extern "C"
