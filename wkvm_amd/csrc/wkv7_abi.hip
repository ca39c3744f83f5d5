// Library-level entry points of the C ABI: version and error text.
#include "wkv7_common.h"

extern "C" int wkv7_abi_version(void) { return WKV7_ABI_VERSION; }

extern "C" const char* wkv7_strerror(int code) {
  switch (code) {
    case WKV7_OK: return "success";
    case WKV7_ERR_ARG: return "invalid argument (null pointer, negative size or bad enum)";
    case WKV7_ERR_SHAPE: return "unsupported layout (row size beyond the slot stride, or inputs not 16-byte aligned)";
    case WKV7_ERR_WORKSPACE: return "workspace or staging buffer missing, or smaller than the entry point needs";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown wkv7 error";
}
