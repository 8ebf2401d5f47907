// C-ABI plumbing shared by every entry point: version and error messages.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/dt_attention.h"

namespace dt {

static thread_local char g_msg[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_msg[0] = 0; }

}  // namespace dt

// 0.2.0: dt_flash_fwd_ex, packed V, workspaces; 0.2.1: dt_flash_fwd_plan,
// the fp32-input prologue entry points
extern "C" int dt_version(void) { return 201; }

extern "C" const char* dt_last_error(void) { return dt::g_msg; }
