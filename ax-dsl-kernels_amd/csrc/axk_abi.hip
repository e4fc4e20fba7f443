// Library identification and status text for the axk C-ABI.
#include "axk_host.h"

extern "C" const char* axk_version(void) { return "axk 0.1.0 gfx950"; }

extern "C" const char* axk_status_string(int status) {
  switch (status) {
    case AXK_OK: return "ok";
    case AXK_E_NULL: return "a required pointer is NULL";
    case AXK_E_SHAPE: return "size / shape contract violated";
    case AXK_E_ALIGN: return "pointer or leading dimension not aligned as required";
    case AXK_E_DTYPE: return "unsupported dtype code";
    case AXK_E_ALIAS: return "buffers overlap where aliasing is not allowed";
    case AXK_E_WORKSPACE: return "workspace missing or too small";
    case AXK_E_LAUNCH: return "HIP launch failed";
    case AXK_E_ROLE: return "unknown role";
    case AXK_E_BUFFER: return "host output buffer too small";
    default: return "unknown status";
  }
}
