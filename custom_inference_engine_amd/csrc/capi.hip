// Library-level entry points of the C ABI (version, status strings).
#include "cie_common.h"

extern "C" int cie_abi_version(void) { return 10; }

extern "C" const char* cie_status_string(int status) {
  switch (status) {
    case CIE_OK:
      return "ok";
    case CIE_EINVAL:
      return "invalid argument (sizes, strides, alignment or null pointer)";
    case CIE_EUNSUPPORTED:
      return "unsupported shape for the gfx950 kernels";
    case CIE_ESCRATCH:
      return "problem larger than the allocation-free entry point's static scratch";
    default:
      break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
