// Library-wide C-ABI helpers: status strings and the ABI version.
#include "dpa_common.hpp"

extern "C" const char* dpa_status_string(int status) {
  switch (status) {
    case DPA_OK: return "ok";
    case DPA_ERR_NULL: return "a required pointer is NULL";
    case DPA_ERR_SIZE: return "invalid size";
    case DPA_ERR_ALIGN: return "pointer alignment not supported";
    case DPA_ERR_SHAPE: return "shape not supported by the FP8 kernels";
    case DPA_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

extern "C" int dpa_abi_version(void) { return 1; }
