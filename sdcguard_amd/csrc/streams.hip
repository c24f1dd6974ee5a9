// One side stream per device plus two reusable events, for fork/join inside one library call.
#include <mutex>

#include "common.h"
#include "streams.h"

namespace {
constexpr int MAXDEV = 64;
struct Side {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
Side g_side[MAXDEV];
std::mutex g_mu;

Side* side_for_current() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return nullptr;
  Side& sd = g_side[dev];
  if (!sd.s) {
    if (hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&sd.join, hipEventDisableTiming) != hipSuccess) return nullptr;
  }
  return &sd;
}
}  // namespace

hipStream_t sdc_fork(hipStream_t main) {
  std::lock_guard<std::mutex> lk(g_mu);
  Side* sd = side_for_current();
  if (!sd) return nullptr;
  if (hipEventRecord(sd->fork, main) != hipSuccess) return nullptr;
  if (hipStreamWaitEvent(sd->s, sd->fork, 0) != hipSuccess) return nullptr;
  return sd->s;
}

int sdc_join(hipStream_t main, hipStream_t side) {
  std::lock_guard<std::mutex> lk(g_mu);
  Side* sd = side_for_current();
  if (!sd || sd->s != side) return SDC_ELAUNCH;
  if (hipEventRecord(sd->join, side) != hipSuccess) return SDC_ELAUNCH;
  if (hipStreamWaitEvent(main, sd->join, 0) != hipSuccess) return SDC_ELAUNCH;
  return SDC_OK;
}
