// Library-level entry points: version and error strings.
#include "tlx_common.h"

extern "C" int tlx_version(void) { return 1; }

extern "C" const char* tlx_strerror(int code) {
  switch (code) {
    case TLX_OK: return "ok";
    case TLX_E_ARG: return "argument out of range (M, sizes or layout)";
    case TLX_E_ALIGN: return "pointer or row stride misaligned for this layout";
    case TLX_E_NODEV: return "no usable gfx950 device";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown tlx error";
  }
}
