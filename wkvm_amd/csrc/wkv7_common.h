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

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (a in the low half), round to nearest even,
// on the hardware converter (v_cvt_pk_bf16_f32): branch free, NaN stays NaN.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pack_bf16(f, 0.f));
}

__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace wkv7
