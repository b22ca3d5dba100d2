// Optional per-launch timing with HIP events (bench.py's live kernel timing).
//
// When enabled, every kernel launch of the library is dispatched with a
// start/stop event pair (hipExtLaunchKernelGGL), which the runtime stamps
// with that dispatch's own begin and end times; wz_prof_get() returns each
// launch's name and elapsed milliseconds.  Disabled (the default) it costs
// one branch per launch.  Launches made while the stream is being captured
// into a graph are never instrumented.
#include <vector>

#include "common.h"

namespace {
struct Slot {
  const char* name;
  hipEvent_t b, e;
};
std::vector<Slot> g_slots;
int g_used = 0;
bool g_on = false;
}  // namespace

namespace wz {

int prof_pre(hipStream_t s, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_on || g_used >= int(g_slots.size())) return -1;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return -1;
  *start = g_slots[g_used].b;
  *stop = g_slots[g_used].e;
  return g_used++;
}

void prof_post(int slot, const char* name) {
  if (slot >= 0) g_slots[slot].name = name;
}

}  // namespace wz

extern "C" int wz_prof_begin(int max_launches) {
  using namespace wz;
  if (max_launches <= 0) return set_error(WZ_EINVAL, "prof_begin: max_launches must be positive");
  while (int(g_slots.size()) < max_launches) {
    Slot s{nullptr, nullptr, nullptr};
    if (hipEventCreate(&s.b) != hipSuccess || hipEventCreate(&s.e) != hipSuccess)
      return set_error(WZ_ELAUNCH, "prof_begin: hipEventCreate failed");
    g_slots.push_back(s);
  }
  g_used = 0;
  g_on = true;
  return WZ_OK;
}

extern "C" int wz_prof_end(void) {
  g_on = false;
  return g_used;
}

extern "C" int wz_prof_get(int i, const char** name, float* ms) {
  using namespace wz;
  if (i < 0 || i >= g_used) return set_error(WZ_EINVAL, "prof_get: index %d out of range", i);
  if (hipEventSynchronize(g_slots[i].e) != hipSuccess) return set_error(WZ_ELAUNCH, "prof_get: sync failed");
  float t = 0.0f;
  if (hipEventElapsedTime(&t, g_slots[i].b, g_slots[i].e) != hipSuccess)
    return set_error(WZ_ELAUNCH, "prof_get: elapsed failed");
  if (name) *name = g_slots[i].name;
  if (ms) *ms = t;
  return WZ_OK;
}
