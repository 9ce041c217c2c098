// Thread-local error message and the two trivial exports.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "flw_common.h"

namespace flw {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

static thread_local hipEvent_t g_timer_start = nullptr, g_timer_stop = nullptr;

Timer take_timer() {
  Timer t;
  t.start = g_timer_start;
  t.stop = g_timer_stop;
  g_timer_start = g_timer_stop = nullptr;
  return t;
}

void arm_timer(Timer t) {
  g_timer_start = t.start;
  g_timer_stop = t.stop;
}

int compute_units() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FLW_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return FLW_OK;
}

}  // namespace flw

extern "C" const char* flw_last_error(void) { return flw::g_last_error; }
extern "C" int flw_abi_version(void) { return FLW_ABI_VERSION; }

extern "C" int flw_time_next_launch(void* start_event, void* stop_event) {
  FLW_REQUIRE((start_event == nullptr) == (stop_event == nullptr), FLW_E_INVALID,
              "flw_time_next_launch: pass both events or neither");
  flw::g_timer_start = static_cast<hipEvent_t>(start_event);
  flw::g_timer_stop = static_cast<hipEvent_t>(stop_event);
  return FLW_OK;
}
