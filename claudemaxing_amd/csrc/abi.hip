// Version and error-name entry points of the C ABI.
#include "common.h"

extern "C" int cm_abi_version(void) { return CM_ABI_VERSION; }

extern "C" const char* cm_error_string(int code) {
  if (code == 0) return "success";
  if (code == static_cast<int>(hipErrorInvalidValue)) return "invalid argument";
  if (code == CM_ERROR_SCRATCH_TOO_SMALL)
    return "these sizes need more scratch than cm_lmhead_ce_noalloc holds "
           "(CM_LMHEAD_NOALLOC_SCRATCH_BYTES = 64 MiB): use a smaller vocabulary chunk or "
           "cm_lmhead_ce with a workspace";
  const char* s = hipGetErrorString(static_cast<hipError_t>(code));
  return s ? s : "unknown error";
}
