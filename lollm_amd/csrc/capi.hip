// Library-level entry points of the C ABI (error strings, ABI version).
#include "common.h"

LOLLM_API const char* lollm_strerror(int code) {
  if (code == LOLLM_OK) return "ok";
  if (code == LOLLM_EINVAL) return "invalid argument";
  if (code == LOLLM_EUNSUPPORTED) return "unsupported shape or dtype";
  if (code >= LOLLM_EHIP_BASE) return hipGetErrorString((hipError_t)(code - LOLLM_EHIP_BASE));
  return "unknown error";
}

LOLLM_API int lollm_abi_version(void) { return 1; }
