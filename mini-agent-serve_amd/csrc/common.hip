// common.hip - library-wide entry points (version, status text) and the cached device query.
#include <mutex>

#include "device.h"

namespace mas {

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_cu_once[kMaxDevices];
int g_cu_count[kMaxDevices];
}  // namespace

int device_cu_count(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MAS_ERR_DEVICE;
  std::call_once(g_cu_once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cu_count[dev] = n;
  });
  *cus = g_cu_count[dev];
  return MAS_OK;
}

}  // namespace mas

extern "C" int mas_version(void) { return (0 << 16) | (1 << 8) | 0; }

extern "C" const char* mas_status_string(int status) {
  switch (status) {
    case MAS_OK: return "ok";
    case MAS_ERR_INVALID_VALUE: return "invalid argument (null pointer, negative size, bad stride or eps)";
    case MAS_ERR_UNSUPPORTED: return "unsupported shape";
    case MAS_ERR_MISALIGNED: return "pointer or stride breaks the kernel's 16-byte alignment";
    case MAS_ERR_DEVICE: return "device query failed";
    case MAS_ERR_SCRATCH: return "the call needs more scratch than the no-allocation entry point holds";
    case MAS_ERR_NOT_READY:
      return "the no-allocation entry point's first call on a device came under graph capture; make one call outside "
             "capture first";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
