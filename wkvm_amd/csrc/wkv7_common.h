// Shared device helpers for the gfx950 WKV7 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7.h"

namespace wkv7 {

constexpr int kHead = 64;    // head size N = K = V (RWKV-7 uses 64 everywhere)
constexpr int kWave = 64;    // CDNA wavefront width

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// Round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace wkv7
