// Varlen WKV7 prefill over slot states.
//
// Recurrent form: one wavefront per (sequence, head) walks the sequence token
// by token with the 64x64 fp32 state resident in VGPRs (lane i owns value
// column i), reading the slot state once and writing the final state once.
// Per token the wave reads 6 x 128 B of bf16 inputs and writes 128 B of y;
// the next token's inputs are prefetched into registers while the current one
// is computed, and the broadcast vectors are double-buffered in LDS so one
// barrier per token suffices.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

template <bool kF32Out>
__global__ __launch_bounds__(kWave) void prefill_recurrent_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu_seqlens, const uint16_t* __restrict__ r,
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ b, void* __restrict__ y, int64_t total_tokens, int zero_init,
    float scale) {
  __shared__ float4 s_dbkr[2][kHead];
  __shared__ float4 s_a[2][kHead / 4];
  const int lane = threadIdx.x;
  const int64_t seq = blockIdx.x / H;
  const int64_t head = blockIdx.x - seq * H;
  const int64_t slot = slot_ids[seq];
  if (slot < 0 || slot >= num_rows) return;
  // Clamp to the packed inputs so a malformed cu_seqlens cannot read past them.
  const int64_t t1 = min(max(int64_t(cu_seqlens[seq + 1]), int64_t(0)), total_tokens);
  const int64_t t0 = min(max(int64_t(cu_seqlens[seq]), int64_t(0)), t1);

  float* hp = wkv + (slot * H + head) * (kHead * kHead) + lane;
  float h[kHead];
#pragma unroll
  for (int j = 0; j < kHead; ++j) h[j] = zero_init ? 0.f : hp[j * kHead];

  const int64_t stride = int64_t(H) * kHead;
  int64_t io = t0 * stride + head * kHead + lane;
  uint16_t nr = 0, nw = 0, nk = 0, nv = 0, na = 0, nb = 0;
  if (t0 < t1) {
    nr = r[io]; nw = w[io]; nk = k[io]; nv = v[io]; na = a[io]; nb = b[io];
  }
  for (int64_t t = t0; t < t1; ++t, io += stride) {
    const int buf = int(t & 1);
    s_dbkr[buf][lane] =
        make_float4(expf(bf16_to_f32(nw)), bf16_to_f32(nb), bf16_to_f32(nk), bf16_to_f32(nr) * scale);
    reinterpret_cast<float*>(s_a[buf])[lane] = bf16_to_f32(na);
    const float vi = bf16_to_f32(nv);
    if (t + 1 < t1) {
      const int64_t nx = io + stride;
      nr = r[nx]; nw = w[nx]; nk = k[nx]; nv = v[nx]; na = a[nx]; nb = b[nx];
    }
    __syncthreads();

    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
    for (int q = 0; q < kHead / 4; ++q) {
      const float4 aq = s_a[buf][q];
      p0 = fmaf(aq.x, h[4 * q + 0], p0);
      p1 = fmaf(aq.y, h[4 * q + 1], p1);
      p2 = fmaf(aq.z, h[4 * q + 2], p2);
      p3 = fmaf(aq.w, h[4 * q + 3], p3);
    }
    const float p = (p0 + p1) + (p2 + p3);
    float y0 = 0.f, y1 = 0.f, y2 = 0.f, y3 = 0.f;
#pragma unroll
    for (int j = 0; j < kHead; ++j) {
      const float4 c = s_dbkr[buf][j];
      h[j] = fmaf(c.x, h[j], fmaf(c.y, p, c.z * vi));
      switch (j & 3) {
        case 0: y0 = fmaf(c.w, h[j], y0); break;
        case 1: y1 = fmaf(c.w, h[j], y1); break;
        case 2: y2 = fmaf(c.w, h[j], y2); break;
        default: y3 = fmaf(c.w, h[j], y3); break;
      }
    }
    const float yi = (y0 + y1) + (y2 + y3);
    if (kF32Out)
      static_cast<float*>(y)[io] = yi;
    else
      static_cast<uint16_t*>(y)[io] = f32_to_bf16(yi);
  }
#pragma unroll
  for (int j = 0; j < kHead; ++j) hp[j * kHead] = h[j];
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" size_t wkv7_prefill_workspace_bytes(int32_t H, int32_t nseq, int64_t total_tokens) {
  (void)H;
  (void)nseq;
  (void)total_tokens;
  return 0;
}

extern "C" int wkv7_prefill_varlen(float* wkv_layer, int64_t num_rows, int32_t H,
                                   const int32_t* slot_ids, const int32_t* cu_seqlens,
                                   int32_t nseq, int64_t total_tokens, const uint16_t* r,
                                   const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                   const uint16_t* a, const uint16_t* b, void* y, int32_t y_dtype,
                                   int32_t zero_init, float scale, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (nseq < 0 || H < 1 || num_rows < 1 || total_tokens < 0) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (nseq == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || !cu_seqlens) return WKV7_ERR_ARG;
  if (total_tokens > 0 && (!r || !w || !k || !v || !a || !b || !y)) return WKV7_ERR_ARG;
  if (workspace_bytes < wkv7_prefill_workspace_bytes(H, nseq, total_tokens)) return WKV7_ERR_WORKSPACE;
  (void)workspace;
  const int64_t blocks = int64_t(nseq) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  if (y_dtype == WKV7_Y_F32)
    prefill_recurrent_kernel<true><<<unsigned(blocks), kWave, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, cu_seqlens, r, w, k, v, a, b, y, total_tokens, zero_init,
        scale);
  else
    prefill_recurrent_kernel<false><<<unsigned(blocks), kWave, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, cu_seqlens, r, w, k, v, a, b, y, total_tokens, zero_init,
        scale);
  return launch_status();
}
