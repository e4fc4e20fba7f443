// Library identification and status text for the axk C-ABI.
#include <pthread.h>

#include "axk_host.h"

namespace {
pthread_key_t g_validate_key;
pthread_once_t g_validate_once = PTHREAD_ONCE_INIT;
void make_validate_key() { pthread_key_create(&g_validate_key, nullptr); }
}  // namespace

int axk_validate_only() {
  pthread_once(&g_validate_once, make_validate_key);
  return (int)(intptr_t)pthread_getspecific(g_validate_key);
}

void axk_validate_add(int delta) {
  const int v = axk_validate_only() + delta;
  pthread_setspecific(g_validate_key, reinterpret_cast<void*>((intptr_t)v));
}

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
    case AXK_E_SCRATCH: return "request exceeds the library's static scratch";
    default: return "unknown status";
  }
}
