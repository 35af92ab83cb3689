// Library-wide C-ABI entry points: version and per-thread error reporting.
#include "fu_common.h"

namespace fu {
thread_local char g_last_error[512] = {0};
}  // namespace fu

extern "C" int fu_version(void) { return 100; }  // 0.1.0

extern "C" const char* fu_last_error(void) { return fu::g_last_error; }
