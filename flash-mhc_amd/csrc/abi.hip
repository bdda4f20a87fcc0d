// Status strings and version of the C ABI declared in include/flash_mhc_hip.h.
#include "fmhc_common.h"

extern "C" const char* fmhc_error_string(int status) {
  if (status == FMHC_OK) return "ok";
  if (status == FMHC_ERR_INVALID_ARGUMENT)
    return "invalid argument (negative size, n != 4, D_out != 32 or null pointer)";
  if (status == FMHC_ERR_SCRATCH_LIMIT)
    return "the call needs more scratch memory than the no-allocation entry point holds";
  if (status >= FMHC_ERR_HIP_BASE)
    return hipGetErrorString(static_cast<hipError_t>(status - FMHC_ERR_HIP_BASE));
  return "unknown flash_mhc status";
}

extern "C" int fmhc_abi_version(void) { return FMHC_ABI_VERSION; }
