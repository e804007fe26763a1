// Error reporting for the C ABI: every entry point returns 0 on success and a
// nonzero status otherwise; ekv_last_error() names the failed check.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include "ekv_internal.h"

namespace ekv {

static thread_local char g_error[512] = "";

void set_error(const char* msg) { snprintf(g_error, sizeof(g_error), "%s", msg); }

int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_error, sizeof(g_error), "kernel launch failed: %s", hipGetErrorString(e));
    return kLaunchFailed;
  }
  return kOk;
}

}  // namespace ekv

extern "C" const char* ekv_last_error(void) { return ekv::g_error; }

extern "C" int ekv_abi_version(void) { return 1; }
