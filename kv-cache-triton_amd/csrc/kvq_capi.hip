// Library-wide C ABI pieces: version and the thread-local error message.
#include <stdarg.h>
#include <stdio.h>

#include "kvq_common.h"

namespace kvq {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace kvq

extern "C" int kvq_version(void) { return KVQ_VERSION; }

extern "C" const char* kvq_last_error(void) { return kvq::g_err; }
