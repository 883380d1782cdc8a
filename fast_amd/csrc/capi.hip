// Status strings and version of the C ABI.
#include "fa_common.hpp"

extern "C" const char* fa_status_string(int status) {
  switch (status) {
    case FA_OK: return "success";
    case FA_EINVAL: return "invalid argument (size, null pointer or inconsistent dimensions)";
    case FA_EUNSUPPORTED: return "unsupported shape for the built kernels";
    case FA_EALIGN: return "pointer or leading dimension is not 16-byte aligned";
    case FA_ESCRATCH: return "scratch buffer too small";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

extern "C" int fa_abi_version(void) { return 500; }
