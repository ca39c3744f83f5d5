// Slot-indexed WKV7 decode step (one token per slot), in place on the pool.
//
// Mapping: one 256-thread workgroup per (batch row, head). Wave q owns key
// rows j in [16q, 16q+16) of the 64x64 fp32 head state and lane i owns value
// column i, so each of the 16 row loads/stores of a wave is one full 256 B
// state row. The two contractions over j are lane-local partial sums, combined
// across the four waves through LDS:
//   p_i = sum_j a_j h[j][i]            (before the update)
//   h'[j][i] = d_j h[j][i] + b_j p_i + k_j v_i
//   y_i = sum_j (scale r_j) h'[j][i]
// Each wave stages the per-token vectors of its key rows (decay d = exp(w), b,
// k, scale*r, a) in LDS; the partial sums of p and of y use separate LDS
// arrays, so a workgroup passes two barriers. State traffic is pure streaming (32 KiB per head, read
// once and written once), issued with non-temporal hints. Workgroups visit the
// batch rows in the caller's `row_order` (slot-sorted order keeps the HBM
// access stream inside a few neighbouring slot regions at a time).
#include "wkv7_common.h"

namespace wkv7 {
namespace {

constexpr int kDecWaves = 4;
constexpr int kRowsPerWave = kHead / kDecWaves;  // 16

template <bool kF32Out>
__global__ __launch_bounds__(kWave * kDecWaves) void decode_slots_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ row_order, int B, const uint16_t* __restrict__ r,
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ b, void* __restrict__ y, float scale) {
  __shared__ float4 s_dbkr[kHead];            // (decay, b, k, scale*r) per key row j
  __shared__ float s_a[kHead];
  __shared__ float s_p[kDecWaves][kHead];  // per-wave partial p
  __shared__ float s_y[kDecWaves][kHead];  // per-wave partial y

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t pos = blockIdx.x / H;
  const int64_t head = blockIdx.x - pos * H;
  int64_t row = pos;
  if (row_order) {
    row = row_order[pos];
    if (row < 0 || row >= B) return;  // uniform: the whole block skips
  }
  const int64_t slot = slot_ids[row];
  if (slot < 0 || slot >= num_rows) return;

  float* hp = wkv + (slot * H + head) * (kHead * kHead) + (kRowsPerWave * wave) * kHead + lane;
  float h[kRowsPerWave];
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) h[j] = __builtin_nontemporal_load(hp + j * kHead);

  const int64_t io = (row * H + head) * kHead + lane;
  const int j0 = kRowsPerWave * wave;
  // Each wave stages the vectors of its own key rows and is their only
  // reader, so a wavefront-scope fence orders the LDS writes before the reads
  // (no workgroup barrier).
  if (lane < kRowsPerWave) {
    const int64_t jo = io + j0;  // key row j0 + lane
    s_dbkr[j0 + lane] = make_float4(expf(bf16_to_f32(w[jo])), bf16_to_f32(b[jo]),
                                    bf16_to_f32(k[jo]), bf16_to_f32(r[jo]) * scale);
    s_a[j0 + lane] = bf16_to_f32(a[jo]);
  }
  const float vi = bf16_to_f32(v[io]);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float p0 = 0.f, p1 = 0.f;
#pragma unroll
  for (int j = 0; j < kRowsPerWave; j += 2) {
    p0 = fmaf(s_a[j0 + j], h[j], p0);
    p1 = fmaf(s_a[j0 + j + 1], h[j + 1], p1);
  }
  s_p[wave][lane] = p0 + p1;
  __syncthreads();
  const float p = (s_p[0][lane] + s_p[1][lane]) + (s_p[2][lane] + s_p[3][lane]);

  float y0 = 0.f, y1 = 0.f;
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) {
    const float4 c = s_dbkr[j0 + j];
    const float hn = fmaf(c.x, h[j], fmaf(c.y, p, c.z * vi));
    __builtin_nontemporal_store(hn, hp + j * kHead);
    if (j & 1)
      y1 = fmaf(c.w, hn, y1);
    else
      y0 = fmaf(c.w, hn, y0);
  }
  s_y[wave][lane] = y0 + y1;
  __syncthreads();
  if (wave == 0) {
    const float yi = (s_y[0][lane] + s_y[1][lane]) + (s_y[2][lane] + s_y[3][lane]);
    if (kF32Out)
      static_cast<float*>(y)[io] = yi;
    else
      static_cast<uint16_t*>(y)[io] = f32_to_bf16(yi);
  }
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_decode_slots(float* wkv_layer, int64_t num_rows, int32_t H,
                                 const int32_t* slot_ids, const int32_t* row_order, int32_t B,
                                 const uint16_t* r, const uint16_t* w, const uint16_t* k,
                                 const uint16_t* v, const uint16_t* a, const uint16_t* b, void* y,
                                 int32_t y_dtype, float scale, void* stream) {
  if (B < 0 || H < 1 || num_rows < 1) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (B == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || !r || !w || !k || !v || !a || !b || !y) return WKV7_ERR_ARG;
  const int64_t blocks = int64_t(B) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  const unsigned threads = kWave * kDecWaves;
  if (y_dtype == WKV7_Y_F32)
    decode_slots_kernel<true><<<unsigned(blocks), threads, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, row_order, B, r, w, k, v, a, b, y, scale);
  else
    decode_slots_kernel<false><<<unsigned(blocks), threads, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, row_order, B, r, w, k, v, a, b, y, scale);
  return launch_status();
}
