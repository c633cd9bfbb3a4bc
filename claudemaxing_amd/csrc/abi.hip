// Version and error-name entry points of the C ABI.
#include "common.h"

extern "C" int cm_abi_version(void) { return CM_ABI_VERSION; }

extern "C" const char* cm_error_string(int code) {
  if (code == 0) return "success";
  if (code == static_cast<int>(hipErrorInvalidValue)) return "invalid argument";
  const char* s = hipGetErrorString(static_cast<hipError_t>(code));
  return s ? s : "unknown error";
}
