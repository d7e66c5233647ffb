// Kernel launch helpers shared by the HIP translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "k3_internal.h"

namespace k3 {

// Every launch goes through hipExtLaunchKernel so that an open timing window
// gets the dispatch's own start/end stamps (null events: an ordinary launch).
template <typename F, typename... Args>
inline void launch_timed(const TimedLaunch& tl, F kernel, const dim3& grid, const dim3& block,
                         uint32_t lds, hipStream_t st, Args... args) {
  hipExtLaunchKernelGGL(kernel, grid, block, lds, st, tl.start(), tl.stop(), 0u, args...);
}

// Status of the launch just made (K3_HIP_OK, or the HIP error as a status).
inline int launched(TimedLaunch& tl, const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_HIP_OK;
  tl.failed();
  return hip_fail(what, e);
}

}  // namespace k3
