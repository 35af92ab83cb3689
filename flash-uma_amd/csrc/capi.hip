// Library-wide C-ABI entry points: version, per-thread error reporting and the matrix-core
// mode of the fp32 contractions.
#include <atomic>

#include "split_bf16.h"

namespace fu {
thread_local char g_last_error[512] = {0};

static std::atomic<int> g_matmul_mode{FU_MATMUL_SPLIT_F16};
int matmul_mode() { return g_matmul_mode.load(std::memory_order_relaxed); }
}  // namespace fu

extern "C" int fu_version(void) { return 600; }  // 0.6.0

extern "C" const char* fu_last_error(void) { return fu::g_last_error; }

extern "C" int fu_set_matmul_mode(int32_t mode) {
  if (mode != fu::FU_MATMUL_SPLIT_BF16 && mode != fu::FU_MATMUL_FP32 && mode != fu::FU_MATMUL_SPLIT_F16)
    return fu::set_error(FU_ERR_UNSUPPORTED, "fu_set_matmul_mode: mode=%d (0: split bf16, 1: fp32, 2: split fp16)",
                         mode);
  fu::g_matmul_mode.store(mode, std::memory_order_relaxed);
  return FU_OK;
}

extern "C" int fu_matmul_mode(void) { return fu::matmul_mode(); }
