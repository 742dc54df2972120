// libmtpk runtime pieces: status strings, ABI version, cached device properties.

#include <atomic>

#include "mtpk.h"
#include "mtpk_host.h"

namespace mtpk {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 1;
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
    n = 1;
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace mtpk

extern "C" {

int mtpk_abi_version(void) { return MTPK_ABI_VERSION; }

const char* mtpk_status_string(int status) {
  if (status == MTPK_OK) return "success";
  if (status == MTPK_EINVAL) return "mtpk: invalid argument (shape, dtype, alignment or null pointer)";
  if (status == MTPK_ENODEV) return "mtpk: no usable HIP device";
  if (status == MTPK_ETOOBIG)
    return "mtpk: the call needs more scratch than the static buffer holds (MTPK_MOE_STATIC_SCRATCH)";
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "mtpk: unknown status";
}

}  // extern "C"
