// Error plumbing and identity of liblxops.
#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>

#include "lx_ops.h"

namespace lx {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return LX_ERR_LAUNCH;
  }
  return LX_OK;
}

}  // namespace lx

extern "C" const char* lx_version(void) {
  return "liblxops 0.1 (gfx950, fp32 MFMA; CosyVoice3 DiT + Qwen2 fused ops)";
}

extern "C" const char* lx_last_error(void) { return lx::g_err; }
