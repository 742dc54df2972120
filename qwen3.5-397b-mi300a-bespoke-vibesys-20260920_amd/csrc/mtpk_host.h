// Host-side helpers shared by the libmtpk translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtpk {

// Compute units of the current device (cached per device id).
int device_cu_count();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t align256(int64_t n) { return (n + 255) & ~int64_t(255); }

inline int status_of(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

// Workgroups of `kernel` at `threads` per workgroup that fit on one CU (cached by caller).
template <typename K>
int occupancy_per_cu(K kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1)
    n = 1;
  return n;
}

}  // namespace mtpk
