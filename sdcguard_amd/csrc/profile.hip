// Optional per-kernel timing with HIP events recorded on the launch stream (off by default).
//
// When enabled (sdc_profile_enable(1)), every kernel launch of the library is bracketed by two events on its own
// stream; sdc_profile_read() waits for them and returns the summed duration and the launch count of one kernel
// name.  The events come from a pool created on first use, so nothing is allocated per launch once warm.
#include <atomic>
#include <mutex>
#include <string.h>
#include <string>
#include <vector>

#include "common.h"
#include "profile.h"

namespace {
struct Rec {
  const char* name;
  hipEvent_t a, b;
};
std::mutex g_mu;
std::atomic<bool> g_on{false};     // read without the lock: a launch with profiling off costs one relaxed load
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_pool;
size_t g_used = 0;

hipEvent_t take() {
  if (g_used == g_pool.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    g_pool.push_back(e);
  }
  return g_pool[g_used++];
}
}  // namespace

SdcProf::SdcProf(const char* name, hipStream_t stream) : name_(name), stream_(stream), b_(nullptr) {
  if (!g_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_on.load(std::memory_order_relaxed)) return;
  hipEvent_t a = take(), b = take();
  if (!a || !b) return;
  hipEventRecord(a, stream_);
  g_recs.push_back({name_, a, b});
  b_ = b;
}

SdcProf::~SdcProf() {
  if (b_) hipEventRecord(b_, stream_);
}

extern "C" int sdc_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_on.store(on != 0, std::memory_order_relaxed);
  return SDC_OK;
}

extern "C" int sdc_profile_reset(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& r : g_recs) hipEventSynchronize(r.b);
  g_recs.clear();
  g_used = 0;
  return SDC_OK;
}

// total milliseconds and launches of kernel `name` since the last reset (waits for the recorded events)
extern "C" int sdc_profile_read(const char* name, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lk(g_mu);
  double tot = 0.0;
  int64_t cnt = 0;
  for (auto& r : g_recs) {
    if (strcmp(r.name, name) != 0) continue;
    if (hipEventSynchronize(r.b) != hipSuccess) return SDC_ELAUNCH;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return SDC_ELAUNCH;
    tot += ms;
    ++cnt;
  }
  *total_ms = tot;
  *launches = cnt;
  return SDC_OK;
}

namespace {
thread_local hipError_t g_last = hipSuccess;
}

void sdc_note_error(hipError_t e) { g_last = e; }

// name of the HIP error behind the last SDC_ELAUNCH returned to this thread
extern "C" const char* sdc_last_error(void) { return hipGetErrorString(g_last); }
