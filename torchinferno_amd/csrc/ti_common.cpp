// Library-wide status helpers of libti_quant.so.
#include "ti_common.h"

#include <string.h>

namespace ti {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace ti

extern "C" int ti_version(void) { return 100; }  // 0.1.0

extern "C" const char* ti_last_error(void) { return ti::g_last_error; }
