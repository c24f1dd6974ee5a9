// Scope guard that brackets one kernel launch with HIP events when profiling is on (profile.hip).
#pragma once
#include <hip/hip_runtime.h>

class SdcProf {
 public:
  SdcProf(const char* name, hipStream_t stream);
  ~SdcProf();

 private:
  const char* name_;
  hipStream_t stream_;
  hipEvent_t b_;
};
