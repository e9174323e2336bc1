// Thread-local error reporting for the libsas C ABI.
#include <cstdarg>
#include <cstdio>

#include "../../include/sas.h"
#include "sas_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace sas {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace sas

extern "C" const char* sas_last_error(void) { return g_err; }

extern "C" const char* sas_version(void) { return "libsas 0.1 gfx950"; }
