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

// 0.2.0: dt_flash_fwd_ex, packed V, workspaces.
// 0.2.1: dt_flash_fwd_plan and the fp32-input prologue entry points; it also
//   CHANGED six signatures: dt_qk_norm_rope, dt_qk_norm_rope_table,
//   dt_pack_v, dt_flash_fwd_ex, dt_smooth_keys and dt_fixed_m_prepare each
//   gained a device-length pointer (kv_len_dev / valid_len_dev) after their
//   host length, so a caller built against 0.2.0 must be rebuilt.
// 0.3.0: per-batch device lengths (with a device length, the host length
//   argument is its entry count, 0/1 or B); a device length <= 0 now means
//   no keys / rows (the empty result) instead of all of them.  Callers
//   gate on dt_version() >= 300.
extern "C" int dt_version(void) { return 300; }

extern "C" const char* dt_last_error(void) { return dt::g_msg; }
