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
#include "wkv7_timemix_head.h"

namespace wkv7 {
namespace {

constexpr int kDecWaves = 4;
constexpr int kRowsPerWave = kHead / kDecWaves;  // 16

// The state update of one (row, head) once the per-key-row vectors (decay,
// b, k, scale*r, a) of the wave's own rows are staged in LDS and vi is the
// lane's value: p partials, one barrier, the update with its non-temporal
// stores, y partials, one barrier. Returns y_i on wave 0 (unspecified on the
// others).
__device__ __forceinline__ float decode_core(float* hp, float (&h)[kRowsPerWave], int lane,
                                             int wave, const float4* s_dbkr, const float* s_a,
                                             float (*s_p)[kHead], float (*s_y)[kHead], float vi) {
  const int j0 = kRowsPerWave * wave;
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
  return (s_y[0][lane] + s_y[1][lane]) + (s_y[2][lane] + s_y[3][lane]);
}

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
  const float yi = decode_core(hp, h, lane, wave, s_dbkr, s_a, s_p, s_y, vi);
  if (wave == 0) {
    if (kF32Out)
      static_cast<float*>(y)[io] = yi;
    else
      static_cast<uint16_t*>(y)[io] = f32_to_bf16(yi);
  }
}

struct BlockIn {
  const uint16_t *r, *k, *v, *w_lora, *a_lora, *v_lora, *v_first, *g;  // [B, H*64]
  const uint16_t *k_k, *k_a, *r_k, *ln_w, *ln_b;                        // [H*64]
};

// The time-mix decode of one (row, head) in one workgroup: the WKV inputs
// from the projection outputs (head_inputs, rounded to bf16 as the
// element-wise kernel stores them), the state update (decode_core), and the
// GroupNorm / bonus / gate of the bf16-rounded y (head_output). Every wave
// derives the head's inputs on 16 lanes x 4 channels (lanes 16..63 repeat
// the work of lanes 0..15), stages its own key rows and its copy of v in LDS,
// and wave 0 finishes the output. Same arithmetic, in the same order, as
// wkv7_time_mix_inputs -> wkv7_decode_slots (bf16 y) -> wkv7_time_mix_output.
__global__ __launch_bounds__(kWave * kDecWaves, 8) void decode_block_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ row_order, int B, BlockIn in, float eps, float scale,
    uint16_t* __restrict__ out, uint16_t* __restrict__ v_out) {
  __shared__ float4 s_dbkr[kHead];
  __shared__ float s_a[kHead];
  __shared__ float s_r[kHead];             // r (unscaled), for the bonus term
  __shared__ float s_v[kDecWaves][kHead];  // each wave's copy of v
  __shared__ float s_p[kDecWaves][kHead];
  __shared__ float s_y[kDecWaves][kHead];
  __shared__ float s_yo[kHead];            // y rounded to bf16

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t pos = blockIdx.x / H;
  const int64_t head = blockIdx.x - pos * H;
  int64_t row = pos;
  if (row_order) {
    row = row_order[pos];
    if (row < 0 || row >= B) return;
  }
  const int64_t slot = slot_ids[row];
  if (slot < 0 || slot >= num_rows) return;

  float* hp = wkv + (slot * H + head) * (kHead * kHead) + (kRowsPerWave * wave) * kHead + lane;
  float h[kRowsPerWave];
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) h[j] = __builtin_nontemporal_load(hp + j * kHead);

  // channels 4 sub .. 4 sub + 3 of this (row, head)
  const int sub = lane & 15;
  const int64_t o = (row * H + head) * kHead + 4 * sub;
  const int pc = int(head * kHead + 4 * sub);
  float rr[4], k[4], v[4], wl[4], al[4], kks[4], ka[4], vl[4] = {}, vf[4] = {};
  {
    const Bf4 rb = ld4(in.r + o), kb = ld4(in.k + o), vb = ld4(in.v + o),
              wlb = ld4(in.w_lora + o), alb = ld4(in.a_lora + o);
    const Bf4 kksb = ld4(in.k_k + pc), kab = ld4(in.k_a + pc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      rr[e] = el(rb, e);
      k[e] = el(kb, e);
      v[e] = el(vb, e);
      wl[e] = el(wlb, e);
      al[e] = el(alb, e);
      kks[e] = el(kksb, e);
      ka[e] = el(kab, e);
    }
    if (in.v_lora) {
      const Bf4 vlb = ld4(in.v_lora + o), vfb = ld4(in.v_first + o);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vl[e] = el(vlb, e);
        vf[e] = el(vfb, e);
      }
    }
  }
  float wv[4], kv[4], vv[4], av[4], bv[4];
  head_inputs(k, v, wl, al, kks, ka, in.v_lora != nullptr, vl, vf, wv, kv, vv, av, bv);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    wv[e] = round_bf16(wv[e]);
    kv[e] = round_bf16(kv[e]);
    vv[e] = round_bf16(vv[e]);
    av[e] = round_bf16(av[e]);
    bv[e] = round_bf16(bv[e]);
  }
  if (lane < 16) {
    if ((sub >> 2) == wave) {  // this wave's key rows 4 sub .. 4 sub + 3
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_dbkr[4 * sub + e] = make_float4(expf(wv[e]), bv[e], kv[e], rr[e] * scale);
        s_a[4 * sub + e] = av[e];
        s_r[4 * sub + e] = rr[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) s_v[wave][4 * sub + e] = vv[e];
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float vi = s_v[wave][lane];
  const float yi = decode_core(hp, h, lane, wave, s_dbkr, s_a, s_p, s_y, vi);
  if (wave == 0) {
    // y goes to the output stage rounded to bf16, as the unfused path stores
    // it; r, k and v come back from LDS (every wave's rows are visible after
    // decode_core's barriers), so nothing stays live across the update
    s_yo[lane] = round_bf16(yi);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float y4[4], r4[4], k4[4], v4[4], g[4], rk[4], lw[4], lb[4], ov[4];
    const Bf4 gb = ld4(in.g + o), rkb = ld4(in.r_k + pc), lwb = ld4(in.ln_w + pc),
              lbb = ld4(in.ln_b + pc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 4 * sub + e;
      y4[e] = s_yo[c];
      r4[e] = s_r[c];
      k4[e] = s_dbkr[c].z;
      v4[e] = s_v[0][c];
      g[e] = el(gb, e);
      rk[e] = el(rkb, e);
      lw[e] = el(lwb, e);
      lb[e] = el(lbb, e);
    }
    head_output(y4, r4, k4, v4, g, rk, lw, lb, eps, ov);
    if (lane < 16) {
      st4(out + o, ov[0], ov[1], ov[2], ov[3]);
      if (v_out) st4(v_out + o, v4[0], v4[1], v4[2], v4[3]);
    }
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

extern "C" int wkv7_decode_block(float* wkv_layer, int64_t num_rows, int32_t H,
                                 const int32_t* slot_ids, const int32_t* row_order, int32_t B,
                                 const uint16_t* r, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* w_lora, const uint16_t* a_lora,
                                 const uint16_t* v_lora, const uint16_t* v_first,
                                 const uint16_t* g, const uint16_t* k_k, const uint16_t* k_a,
                                 const uint16_t* r_k, const uint16_t* ln_w, const uint16_t* ln_b,
                                 float eps, float scale, uint16_t* out, uint16_t* v_out,
                                 void* stream) {
  if (B < 0 || H < 1 || num_rows < 1 || !(eps >= 0.f)) return WKV7_ERR_ARG;
  if (B == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || !r || !k || !v || !w_lora || !a_lora || !g || !k_k || !k_a ||
      !r_k || !ln_w || !ln_b || !out || (!v_lora != !v_first))
    return WKV7_ERR_ARG;
  const void* ptrs[] = {r, k, v, w_lora, a_lora, g, k_k, k_a, r_k, ln_w, ln_b, out};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 7u) return WKV7_ERR_SHAPE;
  if ((v_lora && ((reinterpret_cast<uintptr_t>(v_lora) | reinterpret_cast<uintptr_t>(v_first)) &
                  7u)) ||
      (v_out && (reinterpret_cast<uintptr_t>(v_out) & 7u)))
    return WKV7_ERR_SHAPE;
  const int64_t blocks = int64_t(B) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  const BlockIn in{r, k, v, w_lora, a_lora, v_lora, v_first, g, k_k, k_a, r_k, ln_w, ln_b};
  decode_block_kernel<<<unsigned(blocks), kWave * kDecWaves, 0, as_stream(stream)>>>(
      wkv_layer, num_rows, H, slot_ids, row_order, B, in, eps, scale, out, v_out);
  return launch_status();
}
