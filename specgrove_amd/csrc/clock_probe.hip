// Clock probe for measurement: every workgroup's first lane records which XCD
// it runs on, its hardware id (shader engine, array and CU), the shader-clock
// counter (s_memtime, counts shader cycles; the counters of different CUs are
// not aligned, so only two readings of one CU are compared) and the
// constant-rate counter (s_memrealtime, the device's wall clock).  Two probes
// on one stream bracket a timed region; per CU seen by both, the shader-cycle
// delta over the wall-clock delta is the region's average shader clock.
#include "sg_common.h"

namespace sg {
namespace {

constexpr int kProbeFields = 4;  // xcc, shader cycles, wall ticks, HW_ID

__global__ __launch_bounds__(kWave) void clock_probe_kernel(int64_t* __restrict__ out) {
  if (threadIdx.x != 0) return;
  // HW_REG_XCC_ID (hwreg 20), bits [3:0]: the XCD this workgroup runs on.
  const int xcc = __builtin_amdgcn_s_getreg(20 | (3 << 11));
  // HW_REG_HW_ID (hwreg 4), all 32 bits: wave, SIMD, CU, array, engine ids.
  const uint32_t hw_id = static_cast<uint32_t>(__builtin_amdgcn_s_getreg(4 | (31 << 11)));
  const int64_t cycles = static_cast<int64_t>(clock64());
  const int64_t ticks = static_cast<int64_t>(wall_clock64());
  int64_t* o = out + static_cast<int64_t>(blockIdx.x) * kProbeFields;
  o[0] = xcc;
  o[1] = cycles;
  o[2] = ticks;
  o[3] = hw_id;
}

}  // namespace
}  // namespace sg

extern "C" int sg_clock_probe(int64_t* out_dev, int32_t blocks, sg_stream_t stream) {
  using namespace sg;
  clear_error();
  SG_REQUIRE(out_dev != nullptr, "null device pointer");
  SG_REQUIRE(blocks > 0 && blocks <= 4096, "blocks must be in [1, 4096]");
  hipLaunchKernelGGL(clock_probe_kernel, dim3(blocks), dim3(kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), out_dev);
  SG_LAUNCH_CHECK();
  return SG_OK;
}

extern "C" int64_t sg_wall_clock_khz(int32_t device) {
  using namespace sg;
  clear_error();
  int khz = 0;
  const hipError_t err = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device);
  if (err != hipSuccess) {
    set_error(SG_EHIP, std::string("hipDeviceGetAttribute(WallClockRate): ") +
                           hipGetErrorString(err));
    return -1;
  }
  return khz;
}
