// RWKV-7 time-mix element-wise stages around the WKV7 op, over the slot pool.
//
//  * token_shift_mix: the token shift of one state family (bank.shift[l, f],
//    [num_rows, D] bf16, row 0 = pad slot) fused with the lerp mixes that
//    consume it. Token t of sequence s sees prev = x[t-1], or the slot's
//    cached row for the sequence's first token; the sequence's last row of x
//    becomes the slot's cache (in place). Outputs
//        out[m][t] = bf16(x[t] + bf16(prev - x[t]) * mix[m])   (one fp32 fma)
//  * time_mix_inputs: projection outputs -> the WKV op's inputs (log-decay w,
//    k, v, a = -kk, b = kk * a) with the per-head L2 normalisation of
//    kk = k * k_k.
//  * time_mix_output: per-head GroupNorm of the WKV output, the bonus term
//    (sum_c r k r_k) v and the output gate.
//
// All three are HBM-streaming kernels: 16-byte vector loads and stores of
// bf16 rows, fp32 arithmetic, one bf16 rounding per output element. A head
// (64 channels) is 16 lanes x 4 channels, so per-head sums are reductions
// inside one 16-lane DPP row.
#include "wkv7_common.h"
#include "wkv7_timemix_head.h"

namespace wkv7 {
namespace {

constexpr int kMixThreads = 256;

struct Bf8 {
  uint32_t p[4];  // 8 bf16, element 2i in the low half of p[i]
};

__device__ __forceinline__ Bf8 ld8(const uint16_t* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return Bf8{{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ void st8(uint16_t* p, const Bf8& v) {
  *reinterpret_cast<uint4*>(p) = make_uint4(v.p[0], v.p[1], v.p[2], v.p[3]);
}

__device__ __forceinline__ float el(const Bf8& v, int e) {
  return (e & 1) ? bf16_hi(v.p[e >> 1]) : bf16_lo(v.p[e >> 1]);
}

// Sequence of token t: the largest s with cu[s] <= t (empty sequences have
// cu[s] == cu[s+1] and are skipped by taking the largest such s), which holds
// token t when t is inside a sequence. s = t is tried first (one token per
// sequence): one load pair instead of a binary search of dependent loads,
// which dominated the latency of a small launch.
__device__ __forceinline__ int seq_of(const int32_t* cu, int nseq, int64_t t) {
  const int g = int(t < int64_t(nseq - 1) ? t : int64_t(nseq - 1));
  if (int64_t(cu[g]) <= t && t < int64_t(cu[g + 1])) return g;
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(cu[mid]) <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(kMixThreads) void token_shift_mix_kernel(
    const uint16_t* __restrict__ x, int64_t T, int D, uint16_t* __restrict__ shift,
    int64_t num_rows, int64_t row_stride, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int nseq, const uint16_t* __restrict__ mix, int n_mix,
    uint16_t* __restrict__ out, int64_t out_stride) {
  for (int64_t t = blockIdx.x; t < T; t += gridDim.x) {
    int s = int(t);  // no offsets: one token per sequence
    int64_t beg = t, end = t + 1;
    if (cu) {
      s = seq_of(cu, nseq, t);
      beg = max(int64_t(cu[s]), int64_t(0));
      end = min(int64_t(cu[s + 1]), T);
      if (t < beg || t >= end) continue;  // tokens outside every sequence (uniform)
    }
    const bool first = t == beg;
    const int64_t slot = first ? int64_t(slot_ids[s]) : -1;
    const bool cached = slot >= 0 && slot < num_rows;
    for (int c = 8 * threadIdx.x; c < D; c += 8 * kMixThreads) {
      const Bf8 xv = ld8(x + t * D + c);
      Bf8 pv{{0u, 0u, 0u, 0u}};
      if (!first) {
        pv = ld8(x + (t - 1) * D + c);
      } else if (cached) {
        uint16_t* row = shift + slot * row_stride + c;
        pv = ld8(row);
        st8(row, ld8(x + (end - 1) * D + c));  // the sequence's last row becomes the cache
      }
      float xf[8], df[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xf[e] = el(xv, e);
        // prev - x of two bf16 values is exact in fp32; the shift's output is bf16
        df[e] = bf16_lo(pack_bf16(el(pv, e) - xf[e], 0.f));
      }
      for (int m = 0; m < n_mix; ++m) {
        const Bf8 mu = ld8(mix + int64_t(m) * D + c);
        Bf8 o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o.p[i] = pack_bf16(fmaf(df[2 * i], el(mu, 2 * i), xf[2 * i]),
                             fmaf(df[2 * i + 1], el(mu, 2 * i + 1), xf[2 * i + 1]));
        st8(out + int64_t(m) * out_stride + t * D + c, o);
      }
    }
  }
}

struct MixIn {
  const uint16_t *k, *v, *w_lora, *a_lora, *v_lora, *v_first, *k_k, *k_a;
};
struct MixOut {
  uint16_t *w, *k, *v, *a, *b;
};

// One (token, head) per 16 lanes, 4 channels per lane.
__global__ __launch_bounds__(kMixThreads) void time_mix_inputs_kernel(int64_t units, int H,
                                                                       MixIn in, MixOut out) {
  const int64_t unit = (int64_t(blockIdx.x) * kMixThreads + threadIdx.x) >> 4;
  if (unit >= units) return;  // whole 16-lane groups leave together
  const int sub = threadIdx.x & 15;
  const int64_t h = unit % H;
  const int64_t o = unit * kHead + 4 * sub;  // element offset: token row, head, channels
  const int pc = int(h * kHead + 4 * sub);   // parameter offset (channel within D)
  const Bf4 kb = ld4_nt(in.k + o), vb = ld4_nt(in.v + o), wlb = ld4_nt(in.w_lora + o),
            alb = ld4_nt(in.a_lora + o);
  const Bf4 kksb = ld4(in.k_k + pc), kab = ld4(in.k_a + pc);
  float k[4], v[4], wl[4], al[4], kks[4], ka[4], vl[4] = {}, vf[4] = {};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    k[e] = el(kb, e);
    v[e] = el(vb, e);
    wl[e] = el(wlb, e);
    al[e] = el(alb, e);
    kks[e] = el(kksb, e);
    ka[e] = el(kab, e);
  }
  if (in.v_lora) {  // uniform: lerp(v, v_first, sigmoid(v_lora)) for layers > 0
    const Bf4 vlb = ld4_nt(in.v_lora + o), vfb = ld4_nt(in.v_first + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vl[e] = el(vlb, e);
      vf[e] = el(vfb, e);
    }
  }
  float wv[4], kv[4], vv[4], av[4], bv[4];
  head_inputs(k, v, wl, al, kks, ka, in.v_lora != nullptr, vl, vf, wv, kv, vv, av, bv);
  st4(out.w + o, wv[0], wv[1], wv[2], wv[3]);
  st4(out.k + o, kv[0], kv[1], kv[2], kv[3]);
  st4(out.v + o, vv[0], vv[1], vv[2], vv[3]);
  st4(out.a + o, av[0], av[1], av[2], av[3]);
  st4(out.b + o, bv[0], bv[1], bv[2], bv[3]);
}

struct OutIn {
  const void* y;
  const uint16_t *r, *k, *v, *g, *r_k, *ln_w, *ln_b;
};

template <bool kF32Y>
__global__ __launch_bounds__(kMixThreads) void time_mix_output_kernel(int64_t units, int H,
                                                                       OutIn in, float eps,
                                                                       uint16_t* __restrict__ out) {
  const int64_t unit = (int64_t(blockIdx.x) * kMixThreads + threadIdx.x) >> 4;
  if (unit >= units) return;
  const int sub = threadIdx.x & 15;
  const int64_t h = unit % H;
  const int64_t o = unit * kHead + 4 * sub;
  const int pc = int(h * kHead + 4 * sub);
  float y[4];
  if (kF32Y) {
    const float4 yv = *reinterpret_cast<const float4*>(static_cast<const float*>(in.y) + o);
    y[0] = yv.x; y[1] = yv.y; y[2] = yv.z; y[3] = yv.w;
  } else {
    const Bf4 yv = ld4_nt(static_cast<const uint16_t*>(in.y) + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = el(yv, e);
  }
  const Bf4 rb = ld4_nt(in.r + o), kb = ld4_nt(in.k + o), vb = ld4_nt(in.v + o),
            gb = ld4_nt(in.g + o);
  const Bf4 rkb = ld4(in.r_k + pc), lwb = ld4(in.ln_w + pc), lbb = ld4(in.ln_b + pc);
  float r[4], k[4], v[4], g[4], rk[4], lw[4], lb[4], ov[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = el(rb, e);
    k[e] = el(kb, e);
    v[e] = el(vb, e);
    g[e] = el(gb, e);
    rk[e] = el(rkb, e);
    lw[e] = el(lwb, e);
    lb[e] = el(lbb, e);
  }
  head_output(y, r, k, v, g, rk, lw, lb, eps, ov);
  st4(out + o, ov[0], ov[1], ov[2], ov[3]);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

unsigned unit_grid(int64_t units) {
  const int64_t per_block = kMixThreads / 16;
  return static_cast<unsigned>((units + per_block - 1) / per_block);
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_token_shift_mix(const uint16_t* x, int64_t total_tokens, int32_t D,
                                    uint16_t* shift_rows, int64_t num_rows, int64_t row_stride,
                                    const int32_t* slot_ids, const int32_t* cu_seqlens,
                                    int32_t nseq, const uint16_t* mix, int32_t n_mix,
                                    uint16_t* out, int64_t out_stride, void* stream) {
  if (total_tokens < 0 || D < 1 || nseq < 0 || n_mix < 0 || num_rows < 1 || row_stride < D)
    return WKV7_ERR_ARG;
  if (total_tokens == 0 || nseq == 0) return WKV7_OK;
  if (!x || !shift_rows || !slot_ids || (n_mix > 0 && (!mix || !out))) return WKV7_ERR_ARG;
  if (!cu_seqlens && int64_t(nseq) != total_tokens) return WKV7_ERR_ARG;
  if (n_mix > 1 && out_stride < total_tokens * int64_t(D)) return WKV7_ERR_ARG;
  if ((D & 7) || (row_stride & 7) || (out_stride & 7) || !aligned16(x) || !aligned16(shift_rows) ||
      (n_mix > 0 && (!aligned16(mix) || !aligned16(out))))
    return WKV7_ERR_SHAPE;
  const int64_t cap = int64_t(1) << 20;
  const unsigned grid = static_cast<unsigned>(total_tokens < cap ? total_tokens : cap);
  token_shift_mix_kernel<<<grid, kMixThreads, 0, as_stream(stream)>>>(
      x, total_tokens, D, shift_rows, num_rows, row_stride, slot_ids, cu_seqlens, nseq, mix, n_mix,
      out, out_stride);
  return launch_status();
}

extern "C" int wkv7_time_mix_inputs(int64_t total_tokens, int32_t H, const uint16_t* k,
                                    const uint16_t* v, const uint16_t* w_lora,
                                    const uint16_t* a_lora, const uint16_t* v_lora,
                                    const uint16_t* v_first, const uint16_t* k_k,
                                    const uint16_t* k_a, uint16_t* w_out, uint16_t* k_out,
                                    uint16_t* v_out, uint16_t* a_out, uint16_t* b_out,
                                    void* stream) {
  if (total_tokens < 0 || H < 1) return WKV7_ERR_ARG;
  if (total_tokens == 0) return WKV7_OK;
  if (!k || !v || !w_lora || !a_lora || !k_k || !k_a || !w_out || !k_out || !v_out || !a_out ||
      !b_out || (v_lora != nullptr) != (v_first != nullptr))
    return WKV7_ERR_ARG;
  const void* ptrs[] = {k, v, w_lora, a_lora, k_k, k_a, w_out, k_out, v_out, a_out, b_out};
  for (const void* p : ptrs)
    if (!aligned8(p)) return WKV7_ERR_SHAPE;
  if (v_lora && (!aligned8(v_lora) || !aligned8(v_first))) return WKV7_ERR_SHAPE;
  const int64_t units = total_tokens * H;
  if (units > int64_t(0x7fffffff) / 16) return WKV7_ERR_ARG;
  time_mix_inputs_kernel<<<unit_grid(units), kMixThreads, 0, as_stream(stream)>>>(
      units, H, MixIn{k, v, w_lora, a_lora, v_lora, v_first, k_k, k_a},
      MixOut{w_out, k_out, v_out, a_out, b_out});
  return launch_status();
}

extern "C" int wkv7_time_mix_output(int64_t total_tokens, int32_t H, const void* y,
                                    int32_t y_dtype, const uint16_t* r, const uint16_t* k,
                                    const uint16_t* v, const uint16_t* g, const uint16_t* r_k,
                                    const uint16_t* ln_w, const uint16_t* ln_b, float eps,
                                    uint16_t* out, void* stream) {
  if (total_tokens < 0 || H < 1 || !(eps >= 0.f)) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (total_tokens == 0) return WKV7_OK;
  if (!y || !r || !k || !v || !g || !r_k || !ln_w || !ln_b || !out) return WKV7_ERR_ARG;
  const void* ptrs[] = {r, k, v, g, r_k, ln_w, ln_b, out};
  for (const void* p : ptrs)
    if (!aligned8(p)) return WKV7_ERR_SHAPE;
  if (y_dtype == WKV7_Y_F32 ? !aligned16(y) : !aligned8(y)) return WKV7_ERR_SHAPE;
  const int64_t units = total_tokens * H;
  if (units > int64_t(0x7fffffff) / 16) return WKV7_ERR_ARG;
  const OutIn in{y, r, k, v, g, r_k, ln_w, ln_b};
  if (y_dtype == WKV7_Y_F32)
    time_mix_output_kernel<true><<<unit_grid(units), kMixThreads, 0, as_stream(stream)>>>(
        units, H, in, eps, out);
  else
    time_mix_output_kernel<false><<<unit_grid(units), kMixThreads, 0, as_stream(stream)>>>(
        units, H, in, eps, out);
  return launch_status();
}
