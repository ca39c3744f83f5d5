// RWKV-7 time-mix arithmetic of one head, shared by the element-wise kernels
// (wkv7_mix.hip) and the fused decode block (wkv7_decode.hip), so that both
// paths round and reduce in the same order. A head's 64 channels are held by
// 16 lanes x 4 channels; per-head sums are butterflies inside a 16-lane DPP
// row.
#pragma once

#include "wkv7_common.h"

namespace wkv7 {

constexpr float kLog2e = 1.4426950408889634f;
// RWKV-7 log-decay scale: w = -exp(-0.5) * sigmoid(.) (decay in (0.545, 1))
constexpr float kDecayScale = 0.6065306597126334f;

// Sum over the 16 lanes of a DPP row (butterfly: every lane gets the total).
__device__ __forceinline__ float row_sum16(float x) {
  x += __shfl_xor(x, 1, 16);
  x += __shfl_xor(x, 2, 16);
  x += __shfl_xor(x, 4, 16);
  x += __shfl_xor(x, 8, 16);
  return x;
}

__device__ __forceinline__ float sigmoidf(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// Four bf16 of a 16-lane head slice (8-byte loads).
struct Bf4 {
  uint32_t p[2];
};
__device__ __forceinline__ Bf4 ld4(const uint16_t* p) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  return Bf4{{v.x, v.y}};
}
// Rows streamed once by time_mix_inputs / time_mix_output are read and written
// with non-temporal hints (9-10 % faster than plain accesses; the token shift's
// outputs are not: non-temporal stores made it 7 % slower).
__device__ __forceinline__ Bf4 ld4_nt(const uint16_t* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return Bf4{{v.x, v.y}};
}
__device__ __forceinline__ void st4(uint16_t* p, float a, float b, float c, float d) {
  __builtin_nontemporal_store(u32x2_t{pack_bf16(a, b), pack_bf16(c, d)}, reinterpret_cast<u32x2_t*>(p));
}
__device__ __forceinline__ float el(const Bf4& v, int e) {
  return (e & 1) ? bf16_hi(v.p[e >> 1]) : bf16_lo(v.p[e >> 1]);
}

// bf16 rounding of an fp32 value, returned as fp32.
__device__ __forceinline__ float round_bf16(float x) { return bf16_lo(pack_bf16(x, 0.f)); }

// Projection outputs -> the WKV op's inputs for 4 channels (every lane of the
// 16-lane row must call it: the L2 norm of kk = k * k_k is a row reduction).
// vl and vf are the v LoRA output and v_first, used when lerp_v (layers after
// the first). Outputs are fp32 values before their bf16 rounding.
__device__ __forceinline__ void head_inputs(const float (&k)[4], const float (&v)[4],
                                            const float (&wl)[4], const float (&al)[4],
                                            const float (&kks)[4], const float (&ka)[4],
                                            bool lerp_v, const float (&vl)[4],
                                            const float (&vf)[4], float (&w)[4],
                                            float (&ko)[4], float (&vo)[4], float (&a)[4],
                                            float (&b)[4]) {
  float kk[4], sa[4], ssq = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    kk[e] = k[e] * kks[e];
    ssq = fmaf(kk[e], kk[e], ssq);
    sa[e] = sigmoidf(al[e]);
  }
  ssq = row_sum16(ssq);
  // x / max(||x||, 1e-12), the F.normalize convention
  const float inv = 1.f / fmaxf(sqrtf(ssq), 1e-12f);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float n = kk[e] * inv;
    w[e] = -kDecayScale * sigmoidf(wl[e]);
    ko[e] = k[e] * fmaf(sa[e] - 1.f, ka[e], 1.f);
    a[e] = -n;
    b[e] = n * sa[e];
    vo[e] = lerp_v ? fmaf(vf[e] - v[e], sigmoidf(vl[e]), v[e]) : v[e];
  }
}

// WKV output -> the output projection's input for 4 channels: per-head
// GroupNorm (biased variance), the bonus (sum_c r k r_k) v and the gate g.
// k and v are the WKV op's (bf16) k and v; every lane of the row must call it.
__device__ __forceinline__ void head_output(const float (&yin)[4], const float (&r)[4],
                                            const float (&k)[4], const float (&v)[4],
                                            const float (&g)[4], const float (&rk)[4],
                                            const float (&lw)[4], const float (&lb)[4], float eps,
                                            float (&o)[4]) {
  float y[4], sum = 0.f, bonus = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] = yin[e];
    sum += y[e];
    bonus = fmaf(r[e] * k[e], rk[e], bonus);
  }
  const float mean = row_sum16(sum) * (1.f / kHead);
  bonus = row_sum16(bonus);
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] -= mean;
    sq = fmaf(y[e], y[e], sq);
  }
  const float rstd = 1.f / sqrtf(fmaf(row_sum16(sq), 1.f / kHead, eps));  // biased variance
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = fmaf(bonus, v[e], fmaf(y[e] * rstd, lw[e], lb[e])) * g[e];
}

// -- one channel per lane over a whole wave (lane c = channel c of the head) --
// The same values as head_inputs / head_output, bit for bit: every reduction
// is rebuilt in the 4-channel layout's order. The 4-channel lane `sub` holds
// channels 4 sub .. 4 sub + 3 and runs a sequential chain over them; here the
// four lanes of a quad are those channels, each gathers the quad's values by
// DPP and runs the same chain. row_sum16's butterfly over subs (xor 1, 2, 4,
// 8) is the lane butterfly xor 4, 8, 16, 32, with the same operand order.

// Lane E of this lane's quad, on every lane of the quad.
template <int E>
__device__ __forceinline__ float quad_get(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), E | (E << 2) | (E << 4) | (E << 6),
                                                 0xf, 0xf, false));
}

// row_sum16 of the per-sub partials (each equal on its quad's lanes).
__device__ __forceinline__ float sub_sum64(float x) {
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ void head_inputs1(float k, float v, float wl, float al, float kks,
                                             float ka, bool lerp_v, float vl, float vf, float& w,
                                             float& ko, float& vo, float& a, float& b) {
  const float kk = k * kks;
  const float sa = sigmoidf(al);
  const float q0 = quad_get<0>(kk), q1 = quad_get<1>(kk), q2 = quad_get<2>(kk),
              q3 = quad_get<3>(kk);
  float ssq = 0.f;
  ssq = fmaf(q0, q0, ssq);
  ssq = fmaf(q1, q1, ssq);
  ssq = fmaf(q2, q2, ssq);
  ssq = fmaf(q3, q3, ssq);
  ssq = sub_sum64(ssq);
  const float inv = 1.f / fmaxf(sqrtf(ssq), 1e-12f);
  const float n = kk * inv;
  w = -kDecayScale * sigmoidf(wl);
  ko = k * fmaf(sa - 1.f, ka, 1.f);
  a = -n;
  b = n * sa;
  vo = lerp_v ? fmaf(vf - v, sigmoidf(vl), v) : v;
}

__device__ __forceinline__ float head_output1(float y, float r, float k, float v, float g,
                                              float rk, float lw, float lb, float eps) {
  const float rkp = r * k;
  const float y0 = quad_get<0>(y), y1 = quad_get<1>(y), y2 = quad_get<2>(y), y3 = quad_get<3>(y);
  const float p0 = quad_get<0>(rkp), p1 = quad_get<1>(rkp), p2 = quad_get<2>(rkp),
              p3 = quad_get<3>(rkp);
  const float c0 = quad_get<0>(rk), c1 = quad_get<1>(rk), c2 = quad_get<2>(rk),
              c3 = quad_get<3>(rk);
  float sum = 0.f, bonus = 0.f;
  sum += y0;
  bonus = fmaf(p0, c0, bonus);
  sum += y1;
  bonus = fmaf(p1, c1, bonus);
  sum += y2;
  bonus = fmaf(p2, c2, bonus);
  sum += y3;
  bonus = fmaf(p3, c3, bonus);
  const float mean = sub_sum64(sum) * (1.f / kHead);
  bonus = sub_sum64(bonus);
  const float yc = y - mean;
  const float s0 = quad_get<0>(yc), s1 = quad_get<1>(yc), s2 = quad_get<2>(yc),
              s3 = quad_get<3>(yc);
  float sq = 0.f;
  sq = fmaf(s0, s0, sq);
  sq = fmaf(s1, s1, sq);
  sq = fmaf(s2, s2, sq);
  sq = fmaf(s3, s3, sq);
  const float rstd = 1.f / sqrtf(fmaf(sub_sum64(sq), 1.f / kHead, eps));  // biased variance
  return fmaf(bonus, v, fmaf(yc * rstd, lw, lb)) * g;
}

}  // namespace wkv7
