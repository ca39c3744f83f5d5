// Slot-indexed WKV7 decode step (one token per slot), in place on the pool.
//
// Mapping: one wavefront per (batch row, head). Lane i owns value column
// h[:, i] of the 64x64 fp32 head state, 64 values held in VGPRs, so both
// contractions (p_i = sum_j a_j h[j][i] and y_i = sum_j r_j h'[j][i]) are
// lane-local: no cross-lane reduction. Row j of the state is 256 contiguous
// bytes, so each of the 64 row loads/stores of a wave is one fully coalesced
// 256 B access. The per-token vectors (decay, b, k, scaled r, a) are
// broadcast from LDS; v_i is per lane. Pure HBM streaming: 32 KiB of state
// traffic per wave against ~320 FMAs per lane.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

template <bool kF32Out>
__global__ __launch_bounds__(kWave) void decode_slots_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const uint16_t* __restrict__ r, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, void* __restrict__ y,
    float scale) {
  __shared__ float4 s_dbkr[kHead];       // (decay, b, k, scale*r) per key index j
  __shared__ float4 s_a[kHead / 4];      // a, four key indices per entry
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x;         // batch row * H + head
  const int64_t row = bh / H;
  const int64_t head = bh - row * H;
  const int64_t slot = slot_ids[row];
  if (slot < 0 || slot >= num_rows) return;  // uniform: the whole block skips

  float* hp = wkv + (slot * H + head) * (kHead * kHead) + lane;
  float h[kHead];
#pragma unroll
  for (int j = 0; j < kHead; ++j) h[j] = hp[j * kHead];

  const int64_t io = bh * kHead + lane;
  s_dbkr[lane] = make_float4(expf(bf16_to_f32(w[io])), bf16_to_f32(b[io]), bf16_to_f32(k[io]),
                             bf16_to_f32(r[io]) * scale);
  reinterpret_cast<float*>(s_a)[lane] = bf16_to_f32(a[io]);
  const float vi = bf16_to_f32(v[io]);
  __syncthreads();

  // p_i = sum_j a_j h[j][i]; four partial sums keep the FMA chains short.
  float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
  for (int q = 0; q < kHead / 4; ++q) {
    const float4 aq = s_a[q];
    p0 = fmaf(aq.x, h[4 * q + 0], p0);
    p1 = fmaf(aq.y, h[4 * q + 1], p1);
    p2 = fmaf(aq.z, h[4 * q + 2], p2);
    p3 = fmaf(aq.w, h[4 * q + 3], p3);
  }
  const float p = (p0 + p1) + (p2 + p3);

  float y0 = 0.f, y1 = 0.f, y2 = 0.f, y3 = 0.f;
#pragma unroll
  for (int j = 0; j < kHead; ++j) {
    const float4 c = s_dbkr[j];
    const float hn = fmaf(c.x, h[j], fmaf(c.y, p, c.z * vi));
    hp[j * kHead] = hn;
    switch (j & 3) {
      case 0: y0 = fmaf(c.w, hn, y0); break;
      case 1: y1 = fmaf(c.w, hn, y1); break;
      case 2: y2 = fmaf(c.w, hn, y2); break;
      default: y3 = fmaf(c.w, hn, y3); break;
    }
  }
  const float yi = (y0 + y1) + (y2 + y3);
  if (kF32Out)
    static_cast<float*>(y)[io] = yi;
  else
    static_cast<uint16_t*>(y)[io] = f32_to_bf16(yi);
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_decode_slots(float* wkv_layer, int64_t num_rows, int32_t H,
                                 const int32_t* slot_ids, int32_t B, const uint16_t* r,
                                 const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* a, const uint16_t* b, void* y, int32_t y_dtype,
                                 float scale, void* stream) {
  if (B < 0 || H < 1 || num_rows < 1) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (B == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || !r || !w || !k || !v || !a || !b || !y) return WKV7_ERR_ARG;
  const int64_t blocks = int64_t(B) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  if (y_dtype == WKV7_Y_F32)
    decode_slots_kernel<true><<<unsigned(blocks), kWave, 0, s>>>(wkv_layer, num_rows, H, slot_ids,
                                                                 r, w, k, v, a, b, y, scale);
  else
    decode_slots_kernel<false><<<unsigned(blocks), kWave, 0, s>>>(wkv_layer, num_rows, H, slot_ids,
                                                                  r, w, k, v, a, b, y, scale);
  return launch_status();
}
