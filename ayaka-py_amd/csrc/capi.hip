// Error state, version and device checks of the libayaka_fp8 C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "ayk_common.h"

namespace ayk {

static thread_local char g_last_error[512] = "";
static thread_local char g_last_plan[160] = "";

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

void note_plan(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_plan, sizeof(g_last_plan), fmt, args);
  va_end(args);
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(AYK_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return AYK_OK;
}

// Per-device cache of "is gfx950" (-1 unknown). 64 devices is far above any node.
static int g_arch_ok[64];
static bool g_arch_init = false;

static int device_is_gfx950(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int check_device() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    return fail(AYK_EARCH, "no HIP device is available");
  }
  if (!g_arch_init) {
    for (int i = 0; i < 64; ++i) g_arch_ok[i] = -1;
    g_arch_init = true;
  }
  if (device < 0 || device >= 64) return fail(AYK_EARCH, "device index %d out of range", device);
  if (g_arch_ok[device] < 0) g_arch_ok[device] = device_is_gfx950(device);
  if (!g_arch_ok[device]) {
    return fail(AYK_EARCH, "device %d is not gfx950 (MI355X); libayaka_fp8 has no code for it",
                device);
  }
  return AYK_OK;
}

}  // namespace ayk

extern "C" {

const char* ayk_last_error(void) { return ayk::g_last_error; }

const char* ayk_last_plan(void) { return ayk::g_last_plan; }

int ayk_abi_version(void) { return 100; }

int ayk_device_supported(int device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return 0;
  return ayk::device_is_gfx950(device);
}

}  // extern "C"
