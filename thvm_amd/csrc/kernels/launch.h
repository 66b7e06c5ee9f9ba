// launch.h -- host-side launch helper of the kernel launchers.  A launcher
// whose call was preceded by thvm_k_time_next() binds the start event to its
// first kernel and the stop event to its last (hipExtLaunchKernel records
// the dispatch's own start/end timestamps into them); otherwise it is a
// plain launch.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include "../kern_api.h"

template <typename F, typename... Args>
static inline void thvm_launch(bool first, bool last, F f, dim3 grid, dim3 block,
                               uint32_t shared, hipStream_t s, Args... args) {
  // the launchers check hipGetLastError() after their launches: drop a stale
  // error an earlier, already handled runtime call left behind
  if (first) (void)hipGetLastError();
  hipEvent_t e0 = first ? thvm_k_take_start() : nullptr;
  hipEvent_t e1 = last ? thvm_k_take_stop() : nullptr;
  if (e0 || e1)
    hipExtLaunchKernelGGL(f, grid, block, shared, s, e0, e1, 0u, args...);
  else
    hipLaunchKernelGGL(f, grid, block, shared, s, args...);
}
