// Error reporting for the C ABI: every entry point returns 0 or an error code
// and leaves a message retrievable with iron_last_error() on the calling thread.
#include <stdarg.h>
#include <stdio.h>

#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail_einval(const char* fmt, ...) {
  disarm_timing();
  disarm_trace();
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return IRON_EINVAL;
}

int check_launch(const char* what) {
  disarm_timing();
  disarm_trace();
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return 0;
}

static thread_local TimingEvents g_timing = {nullptr, nullptr};
static thread_local bool g_timing_started = false;

TimingEvents take_timing_events() {
  TimingEvents t = g_timing;
  if (t.stop && g_timing_started) t.start = nullptr;  // start stays on the first kernel
  g_timing_started = g_timing.stop != nullptr;
  return t;
}

void disarm_timing() {
  g_timing = {nullptr, nullptr};
  g_timing_started = false;
}

struct TraceState {
  void* buffer;
  long long bytes;
};
static thread_local TraceState g_trace = {nullptr, 0};

void disarm_trace() { g_trace = {nullptr, 0}; }

int take_trace(const char* who, long long records, void** buffer) {
  const TraceState t = g_trace;
  disarm_trace();
  *buffer = nullptr;
  if (!t.buffer) return 0;
  if (t.bytes < records * 64)
    return fail_einval("%s: the armed trace buffer of %lld bytes holds %lld records; this launch writes %lld", who,
                       t.bytes, t.bytes / 64, records);
  *buffer = t.buffer;
  return 0;
}

}  // namespace iron

extern "C" const char* iron_last_error(void) { return iron::g_last_error; }

extern "C" int iron_trace_next_launch(void* buffer, long long bytes) {
  if (buffer && (bytes < 64 || (reinterpret_cast<uintptr_t>(buffer) & 63u)))
    return iron::fail_einval("iron_trace_next_launch: the buffer must be 64-byte aligned and hold a record");
  iron::g_trace = {buffer, buffer ? bytes : 0};
  return 0;
}

extern "C" int iron_time_next_launch(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr))
    return iron::fail_einval("iron_time_next_launch: give both events or neither");
  iron::g_timing = {static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  iron::g_timing_started = false;
  return 0;
}

extern "C" int iron_abi_version(void) { return IRON_HIP_ABI_VERSION; }
