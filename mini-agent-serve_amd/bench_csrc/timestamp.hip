// timestamp.hip - a one-lane kernel that stores the GPU's constant-rate wall clock, for the
// benchmark only (built into libmas_bench.so; nothing in the product path calls it).
//
// Captured into a HIP graph before and after the timed steps, two stamps bracket exactly those
// steps inside one graph replay: no graph launch and no host gap falls between them (ROCm does not
// allow timing events as graph nodes). The interval includes one kernel boundary (the stop stamp's
// dispatch after the last timed kernel).
#include "../csrc/device.h"

namespace mas {
namespace {

__global__ __launch_bounds__(64) void wall_clock_stamp(uint64_t* dst) {
  const uint64_t t = static_cast<uint64_t>(wall_clock64());
  if (threadIdx.x == 0) dst[0] = t;
}

}  // namespace
}  // namespace mas

// Stores the wall clock (ticks) into *dst (a device word) when the stream reaches this point.
extern "C" int mas_bench_timestamp(void* dst, hipStream_t stream) {
  using namespace mas;
  if (dst == nullptr || (reinterpret_cast<uintptr_t>(dst) & 7u) != 0) return MAS_ERR_INVALID_VALUE;
  hipLaunchKernelGGL(wall_clock_stamp, dim3(1), dim3(64), 0, stream, static_cast<uint64_t*>(dst));
  return launch_status();
}

// Wall clock ticks per millisecond of the current device (hipDeviceAttributeWallClockRate, kHz).
extern "C" int mas_bench_wall_clock_khz(int* khz) {
  using namespace mas;
  int dev = 0;
  if (khz == nullptr) return MAS_ERR_INVALID_VALUE;
  if (hipGetDevice(&dev) != hipSuccess) return MAS_ERR_DEVICE;
  if (hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return MAS_ERR_DEVICE;
  return MAS_OK;
}
