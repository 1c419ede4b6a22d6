// Library-level entry points of the C ABI (declared in include/flicker_hip.h).

#include "common.h"

#define FLK_ABI_VERSION 1

extern "C" int flk_abi_version(void) { return FLK_ABI_VERSION; }

extern "C" const char* flk_status_string(int status) {
  switch (status) {
    case FLK_OK: return "ok";
    case FLK_E_INVALID: return "invalid argument (size, count or offset out of range)";
    case FLK_E_ALIGN: return "pointer or stride not 16-byte aligned";
    case FLK_E_UNSUPPORTED: return "unsupported shape (the kernels take head_dim 128 only)";
    case FLK_E_SCRATCH: return "the call needs more than the library's fixed scratch buffer holds";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
