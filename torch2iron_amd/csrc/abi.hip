// ABI-level helpers: version, error strings, thread-local last-error message.
#include <stdarg.h>
#include <stdio.h>

#include "t2i_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace t2i_host {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return T2I_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
  return (int)e;
}

}  // namespace t2i_host

extern "C" int t2i_abi_version(void) { return T2I_ABI_VERSION; }

extern "C" const char* t2i_last_error(void) { return g_last_error; }

extern "C" const char* t2i_strerror(int code) {
  switch (code) {
    case T2I_OK: return "ok";
    case T2I_ERR_NULL: return "required pointer is NULL";
    case T2I_ERR_SHAPE: return "unsupported shape";
    case T2I_ERR_ALIGN: return "pointer not 16-byte aligned";
    case T2I_ERR_GROUP: return "unsupported group size";
    case T2I_ERR_WORKSPACE: return "workspace missing or too small";
    case T2I_ERR_VALUE: return "argument out of range";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error";
}
