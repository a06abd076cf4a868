// api.hip -- library identity and launch-error bookkeeping for libak355.
#include "ak_common.h"

namespace {
thread_local char g_last_error[256] = "no error";
// events the calling thread's next timed launch records (see ak_set_launch_events)
thread_local hipEvent_t g_ev_start = nullptr, g_ev_stop = nullptr;
}

namespace ak {
LaunchEvents take_launch_events(void) {
  const LaunchEvents e{g_ev_start, g_ev_stop};
  g_ev_start = g_ev_stop = nullptr;
  return e;
}

int record_launch(void) { return record_hip_error(hipGetLastError()); }

int record_hip_error(hipError_t e) {
  if (e == hipSuccess) return AK_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s (%d): %s", hipGetErrorName(e), (int)e,
           hipGetErrorString(e));
  return AK_EHIP;
}
}  // namespace ak

extern "C" const char* ak_version(void) { return "ak355 0.1.0 gfx950"; }

extern "C" const char* ak_status_string(int status) {
  switch (status) {
    case AK_OK: return "ok";
    case AK_EINVAL: return "invalid argument";
    case AK_EUNSUPPORTED: return "unsupported configuration";
    case AK_EHIP: return "HIP launch error";
    default: return "unknown status";
  }
}

extern "C" const char* ak_last_hip_error_string(void) { return g_last_error; }

extern "C" int ak_set_launch_events(hipEvent_t start, hipEvent_t stop) {
  g_ev_start = start;
  g_ev_stop = stop;
  return AK_OK;
}
