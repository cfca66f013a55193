// Error reporting of the C ABI: every entry point returns 0 or a negative
// PpoStatus and leaves a message for ppo_last_error() on the calling thread.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace ppo {
int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace ppo

PPO_EXPORT const char* ppo_last_error(void) { return g_last_error; }

PPO_EXPORT void ppo_clear_error(void) { g_last_error[0] = '\0'; }

PPO_EXPORT int ppo_abi_version(void) { return 1; }

// Reports whether a HIP device is usable from this process (0 = yes).
PPO_EXPORT int ppo_device_check(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= device || device < 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_device_check: device %d unavailable (%d devices, %s)", device, n,
                          hipGetErrorString(e));
  return PPO_OK;
}

// ---- stream ordering for the learner's two-tower fork / join ----
// An event without timing, for ppo_stream_wait.
PPO_EXPORT int ppo_event_create(void** event) {
  if (!event) return ppo::set_error(PPO_ERR_ARG, "ppo_event_create: null output");
  hipEvent_t e = nullptr;
  const hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming);
  if (r != hipSuccess) return ppo::set_error(PPO_ERR_LAUNCH, "ppo_event_create: %s", hipGetErrorString(r));
  *event = e;
  return PPO_OK;
}

PPO_EXPORT int ppo_event_destroy(void* event) {
  if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
  return PPO_OK;
}

// Work issued on `waiter` after this call starts after everything issued on
// `signaller` before it (the event is recorded on signaller, then waited on
// by waiter).  Inside a stream capture this forks / joins the captured graph.
// Stream handles are hipStream_t values (0: the null stream).
PPO_EXPORT int ppo_stream_wait(void* waiter, void* signaller, void* event) {
  if (!event) return ppo::set_error(PPO_ERR_ARG, "ppo_stream_wait: null event");
  hipEvent_t e = static_cast<hipEvent_t>(event);
  hipError_t r = hipEventRecord(e, ppo::as_stream(signaller));
  if (r == hipSuccess) r = hipStreamWaitEvent(ppo::as_stream(waiter), e, 0);
  if (r != hipSuccess) return ppo::set_error(PPO_ERR_LAUNCH, "ppo_stream_wait: %s", hipGetErrorString(r));
  return PPO_OK;
}
