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
//
// The same kernel serves the in-place slot decode (source and destination are
// one pool and one id list) and the out-of-place form of fla's recurrent op
// (state read from one tensor, written to another; no source = zero state, no
// destination = the state is not written). A row whose source or destination
// id is out of range touches no state and gets y = 0.
#include <type_traits>

#include "wkv7_common.h"
#include "wkv7_timemix_head.h"

namespace wkv7 {
namespace {

constexpr int kDecWaves = 4;
constexpr int kRowsPerWave = kHead / kDecWaves;  // 16

// The state update of one (row, head) once the per-key-row vectors (decay,
// b, k, scale*r, a) of the wave's own rows are staged in LDS and vi is the
// lane's value: p partials, one barrier, the update with its non-temporal
// stores (kStore; hp is the wave's first destination row), y partials, one
// barrier. Returns y_i on wave 0 (unspecified on the others).
template <bool kStore>
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
    if (kStore) __builtin_nontemporal_store(hn, hp + j * kHead);
    if (j & 1)
      y1 = fmaf(c.w, hn, y1);
    else
      y0 = fmaf(c.w, hn, y0);
  }
  s_y[wave][lane] = y0 + y1;
  __syncthreads();
  return (s_y[0][lane] + s_y[1][lane]) + (s_y[2][lane] + s_y[3][lane]);
}

// State addressing of one decode launch: row b reads src[src_ids[b]] (or
// src[b] when src_ids is null; zero state when src is null) and writes
// dst[dst_ids[b]] (dst[b] when dst_ids is null; nothing when dst is null).
struct DecodeIO {
  const float* src;
  const int32_t* src_ids;
  int64_t src_rows;
  float* dst;
  const int32_t* dst_ids;
  int64_t dst_rows;
};

// How a launch addresses state; one kernel instantiation per form, so that
// no branch separates the state loads from their uses (a branch around them
// makes the compiler wait for every load before the first use).
enum DecodeForm : int {
  kInPlace = 0,    // src == dst, one id list (wkv7_decode_slots)
  kSeparate = 1,   // read src, write dst
  kZeroIn = 2,     // zero initial state, write dst
  kNoOut = 3,      // read src, state not written
  kZeroNoOut = 4,  // zero initial state, state not written
};

template <bool kF32Out>
__device__ __forceinline__ void store_y(void* y, int64_t io, float yi) {
  if (kF32Out)
    static_cast<float*>(y)[io] = yi;
  else
    static_cast<uint16_t*>(y)[io] = f32_to_bf16(yi);
}

template <bool kF32Out, int kForm>
__global__ __launch_bounds__(kWave * kDecWaves) void decode_slots_kernel(
    DecodeIO st, int H, const int32_t* __restrict__ row_order, int B,
    const uint16_t* __restrict__ r, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, void* __restrict__ y,
    float scale) {
  constexpr bool kLoad = kForm == kInPlace || kForm == kSeparate || kForm == kNoOut;
  constexpr bool kStore = kForm == kInPlace || kForm == kSeparate || kForm == kZeroIn;
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
  const int64_t io = (row * H + head) * kHead + lane;
  int64_t src_slot = 0, dst_slot = 0;
  bool ok = true;
  if (kForm == kInPlace) {
    src_slot = dst_slot = st.dst_ids[row];
    ok = dst_slot >= 0 && dst_slot < st.dst_rows;
  } else {
    if (kLoad) {
      src_slot = st.src_ids ? int64_t(st.src_ids[row]) : row;
      ok = src_slot >= 0 && src_slot < st.src_rows;
    }
    if (kStore) {
      dst_slot = st.dst_ids ? int64_t(st.dst_ids[row]) : row;
      ok = ok && dst_slot >= 0 && dst_slot < st.dst_rows;
    }
  }
  if (!ok) {  // uniform: a rejected row touches no state and reads out zero
    if (wave == 0) store_y<kF32Out>(y, io, 0.f);
    return;
  }

  // The per-token vectors are loaded before the state rows: load counts
  // retire in issue order, so waiting for the vectors does not wait for the
  // state stream, and the staging arithmetic overlaps it. Lanes 16..63 read
  // the key rows of lanes 0..15 again (same addresses, no extra traffic) so
  // that no branch separates the loads from the state loads.
  const int j0 = kRowsPerWave * wave;
  const int64_t jo = (row * H + head) * kHead + j0 + (lane & (kRowsPerWave - 1));
  const uint16_t wb = w[jo], bb = b[jo], kb = k[jo], rb = r[jo], ab = a[jo], vb = v[io];
  __builtin_amdgcn_sched_barrier(0);

  const int64_t wave_off = (kRowsPerWave * wave) * kHead + lane;
  float h[kRowsPerWave];
  if (kLoad) {
    const float* hs = (kForm == kInPlace ? st.dst : st.src) +
                      (src_slot * H + head) * (kHead * kHead) + wave_off;
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) h[j] = __builtin_nontemporal_load(hs + j * kHead);
  } else {
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) h[j] = 0.f;
  }
  // an empty asm that consumes the vectors here keeps their loads above the
  // state loads (the compiler would otherwise sink them into the lane < 16
  // branch); it waits for the vectors only
  asm volatile("" ::"v"(wb), "v"(bb), "v"(kb), "v"(rb), "v"(ab), "v"(vb));

  // Each wave stages the vectors of its own key rows and is their only
  // reader, so a wavefront-scope fence orders the LDS writes before the reads
  // (no workgroup barrier).
  if (lane < kRowsPerWave) {
    s_dbkr[j0 + lane] = make_float4(expf(bf16_to_f32(wb)), bf16_to_f32(bb), bf16_to_f32(kb),
                                    bf16_to_f32(rb) * scale);
    s_a[j0 + lane] = bf16_to_f32(ab);
  }
  const float vi = bf16_to_f32(vb);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float* hd = kStore ? st.dst + (dst_slot * H + head) * (kHead * kHead) + wave_off : nullptr;
  const float yi = decode_core<kStore>(hd, h, lane, wave, s_dbkr, s_a, s_p, s_y, vi);
  if (wave == 0) store_y<kF32Out>(y, io, yi);
}

struct BlockIn {
  const uint16_t *r, *k, *v, *w_lora, *a_lora, *v_lora, *v_first, *g;  // [B, H*64]
  const uint16_t *k_k, *k_a, *r_k, *ln_w, *ln_b;                        // [H*64]
};

// The time-mix decode of one (row, head) in one workgroup: the WKV inputs
// from the projection outputs (rounded to bf16 as the element-wise kernel
// stores them), the state update (decode_core), and the GroupNorm / bonus /
// gate of the bf16-rounded y. Lane c of every wave holds channel c of the
// head, which is both key row c and value column c: each wave derives all 64
// channels' inputs (head_inputs1, one channel per lane), keeps its own value
// column's v in a register and stages its own 16 key rows in LDS; wave 0's
// lanes then hold y, r, k and v of their channel for the output stage
// (head_output1). Same arithmetic, in the same order, as
// wkv7_time_mix_inputs -> wkv7_decode_slots (bf16 y) -> wkv7_time_mix_output.
template <bool kLerpV>
__global__ __launch_bounds__(kWave * kDecWaves, 8) void decode_block_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ row_order, int B, BlockIn in, float eps, float scale,
    uint16_t* __restrict__ out, uint16_t* __restrict__ v_out) {
  __shared__ float4 s_dbkr[kHead];
  __shared__ float s_a[kHead];
  __shared__ float s_p[kDecWaves][kHead];
  __shared__ float s_y[kDecWaves][kHead];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t pos = blockIdx.x / H;
  const int64_t head = blockIdx.x - pos * H;
  int64_t row = pos;
  if (row_order) {
    row = row_order[pos];
    if (row < 0 || row >= B) return;
  }
  // This row-head's and this head's first elements are uniform: every input
  // is a scalar base plus the lane's channel.
  const int64_t ro = (row * H + head) * kHead;
  const int64_t po = head * kHead;
  const int64_t slot = slot_ids[row];
  if (slot < 0 || slot >= num_rows) {  // a rejected row reads out zero
    if (wave == 0) {
      out[ro + lane] = 0;
      if (v_out) v_out[ro + lane] = 0;
    }
    return;
  }

  // The projection rows are loaded before the state rows (load counts retire
  // in issue order), so the input arithmetic waits for them only and
  // overlaps the state stream.
  const uint16_t rb = in.r[ro + lane], kb = in.k[ro + lane], vb = in.v[ro + lane],
                 wlb = in.w_lora[ro + lane], alb = in.a_lora[ro + lane],
                 kkb = in.k_k[po + lane], kab = in.k_a[po + lane];
  uint16_t vlb = 0, vfb = 0;
  if (kLerpV) {
    vlb = in.v_lora[ro + lane];
    vfb = in.v_first[ro + lane];
  }
  __builtin_amdgcn_sched_barrier(0);

  float* hp = wkv + (slot * H + head) * (kHead * kHead) + (kRowsPerWave * wave) * kHead + lane;
  float h[kRowsPerWave];
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) h[j] = __builtin_nontemporal_load(hp + j * kHead);

  float wv, kv, vv, av, bv;
  head_inputs1(bf16_to_f32(kb), bf16_to_f32(vb), bf16_to_f32(wlb), bf16_to_f32(alb),
               bf16_to_f32(kkb), bf16_to_f32(kab), kLerpV, bf16_to_f32(vlb), bf16_to_f32(vfb),
               wv, kv, vv, av, bv);
  wv = round_bf16(wv);
  kv = round_bf16(kv);
  vv = round_bf16(vv);
  av = round_bf16(av);
  bv = round_bf16(bv);
  const float rr = bf16_to_f32(rb);
  if ((lane >> 4) == wave) {  // this wave's key rows 16 wave .. 16 wave + 15
    s_dbkr[lane] = make_float4(expf(wv), bv, kv, rr * scale);
    s_a[lane] = av;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float yi = decode_core<true>(hp, h, lane, wave, s_dbkr, s_a, s_p, s_y, vv);
  if (wave == 0) {
    // y goes to the output stage rounded to bf16, as the unfused path stores it
    const float o = head_output1(round_bf16(yi), rr, kv, vv, bf16_to_f32(in.g[ro + lane]),
                                 bf16_to_f32(in.r_k[po + lane]), bf16_to_f32(in.ln_w[po + lane]),
                                 bf16_to_f32(in.ln_b[po + lane]), eps);
    out[ro + lane] = f32_to_bf16(o);
    if (v_out) v_out[ro + lane] = f32_to_bf16(vv);
  }
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

static int launch_decode(const DecodeIO& st, int32_t H, const int32_t* row_order, int32_t B,
                         const uint16_t* r, const uint16_t* w, const uint16_t* k,
                         const uint16_t* v, const uint16_t* a, const uint16_t* b, void* y,
                         int32_t y_dtype, float scale, void* stream) {
  if (B < 0 || H < 1) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if ((st.src && st.src_rows < 1) || (st.dst && st.dst_rows < 1)) return WKV7_ERR_ARG;
  if (B == 0) return WKV7_OK;
  if (!r || !w || !k || !v || !a || !b || !y) return WKV7_ERR_ARG;
  const int64_t blocks = int64_t(B) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  int form = kSeparate;
  if (st.src && st.src == st.dst && st.src_ids && st.src_ids == st.dst_ids &&
      st.src_rows == st.dst_rows)
    form = kInPlace;
  else if (!st.src)
    form = st.dst ? kZeroIn : kZeroNoOut;
  else if (!st.dst)
    form = kNoOut;
  hipStream_t s = as_stream(stream);
  const unsigned grid = unsigned(blocks), threads = kWave * kDecWaves;
  auto launch = [&](auto f32) {
    constexpr bool F = decltype(f32)::value;
    switch (form) {
      case kInPlace:
        decode_slots_kernel<F, kInPlace><<<grid, threads, 0, s>>>(st, H, row_order, B, r, w, k,
                                                                  v, a, b, y, scale);
        break;
      case kSeparate:
        decode_slots_kernel<F, kSeparate><<<grid, threads, 0, s>>>(st, H, row_order, B, r, w, k,
                                                                   v, a, b, y, scale);
        break;
      case kZeroIn:
        decode_slots_kernel<F, kZeroIn><<<grid, threads, 0, s>>>(st, H, row_order, B, r, w, k,
                                                                 v, a, b, y, scale);
        break;
      case kNoOut:
        decode_slots_kernel<F, kNoOut><<<grid, threads, 0, s>>>(st, H, row_order, B, r, w, k, v,
                                                                a, b, y, scale);
        break;
      default:
        decode_slots_kernel<F, kZeroNoOut><<<grid, threads, 0, s>>>(st, H, row_order, B, r, w, k,
                                                                    v, a, b, y, scale);
    }
  };
  if (y_dtype == WKV7_Y_F32)
    launch(std::true_type{});
  else
    launch(std::false_type{});
  return launch_status();
}

extern "C" int wkv7_decode_slots(float* wkv_layer, int64_t num_rows, int32_t H,
                                 const int32_t* slot_ids, const int32_t* row_order, int32_t B,
                                 const uint16_t* r, const uint16_t* w, const uint16_t* k,
                                 const uint16_t* v, const uint16_t* a, const uint16_t* b, void* y,
                                 int32_t y_dtype, float scale, void* stream) {
  if (num_rows < 1) return WKV7_ERR_ARG;
  if (B > 0 && (!wkv_layer || !slot_ids)) return WKV7_ERR_ARG;
  const DecodeIO st{wkv_layer, slot_ids, num_rows, wkv_layer, slot_ids, num_rows};
  return launch_decode(st, H, row_order, B, r, w, k, v, a, b, y, y_dtype, scale, stream);
}

extern "C" int wkv7_decode_into(const float* state_in, int64_t in_rows, const int32_t* in_ids,
                                float* state_out, int64_t out_rows, const int32_t* out_ids,
                                int32_t H, const int32_t* row_order, int32_t B,
                                const uint16_t* r, const uint16_t* w, const uint16_t* k,
                                const uint16_t* v, const uint16_t* a, const uint16_t* b, void* y,
                                int32_t y_dtype, float scale, void* stream) {
  if ((!state_in && in_ids) || (!state_out && out_ids)) return WKV7_ERR_ARG;
  // without ids, row b addresses state row b: the tensor needs B rows
  if ((state_in && !in_ids && in_rows < B) || (state_out && !out_ids && out_rows < B))
    return WKV7_ERR_SHAPE;
  const DecodeIO st{state_in, in_ids, in_rows, state_out, out_ids, out_rows};
  return launch_decode(st, H, row_order, B, r, w, k, v, a, b, y, y_dtype, scale, stream);
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
  if (v_lora)
    decode_block_kernel<true><<<unsigned(blocks), kWave * kDecWaves, 0, as_stream(stream)>>>(
        wkv_layer, num_rows, H, slot_ids, row_order, B, in, eps, scale, out, v_out);
  else
    decode_block_kernel<false><<<unsigned(blocks), kWave * kDecWaves, 0, as_stream(stream)>>>(
        wkv_layer, num_rows, H, slot_ids, row_order, B, in, eps, scale, out, v_out);
  return launch_status();
}
