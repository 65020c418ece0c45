// Shared host/device helpers of libspecgrove_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "specgrove_hip.h"

namespace sg {

// Records the message returned by sg_last_error() and passes the code through.
int set_error(int code, const std::string& message);
void clear_error();

#define SG_REQUIRE(cond, msg)                                   \
  do {                                                          \
    if (!(cond)) return ::sg::set_error(SG_EINVAL, (msg));      \
  } while (0)

#define SG_HIP_CHECK(expr)                                                   \
  do {                                                                       \
    hipError_t sg_err_ = (expr);                                             \
    if (sg_err_ != hipSuccess)                                               \
      return ::sg::set_error(SG_EHIP, std::string(#expr) + ": " +            \
                                          hipGetErrorString(sg_err_));       \
  } while (0)

// Launch check: reports the launch error of the last kernel on this thread.
#define SG_LAUNCH_CHECK() SG_HIP_CHECK(hipGetLastError())

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (inputs are finite in this library).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) |
         (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

}  // namespace sg
