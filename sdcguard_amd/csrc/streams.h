// Fork/join of a side stream for kernels that can run concurrently with the caller's stream (streams.hip).
#pragma once
#include <hip/hip_runtime.h>

// After sdc_fork(main) work queued on the returned side stream runs after everything already queued on `main`;
// sdc_join(main, side) makes later work on `main` wait for everything queued on `side`.  One side stream per
// device, created on first use at the default priority; both calls are graph-capture safe (event record/wait).
hipStream_t sdc_fork(hipStream_t main);
int sdc_join(hipStream_t main, hipStream_t side);
