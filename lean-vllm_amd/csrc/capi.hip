// Error state and version of the lvattn C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "lv_common.h"

namespace lv {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buf, sizeof(buf), fmt, args);
  va_end(args);
  g_last_error = buf;
}

const char* last_error() { return g_last_error.c_str(); }

}  // namespace lv

extern "C" const char* lv_last_error(void) { return lv::last_error(); }

extern "C" int lv_abi_version(void) { return LV_ABI_VERSION; }
