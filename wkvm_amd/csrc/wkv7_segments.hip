// Combination step of the segmented prefill (wkv7_prefill_runs + these two).
//
// The WKV7 scan is linear in its initial state. A sequence cut into segments
// runs segment 0 from its slot state and every later segment g twice, side by
// side: from zero state with the real inputs (y0_g, final state H0_g) and from
// the identity with k = v = 0, which gives the segment's transition Phi_g as
// the final state and q_g = (scale r)^T Phi_t as y. With H_in the state
// entering segment g:
//   H_out = H0_g + Phi_g H_in          (wkv7_segment_chain, in segment order)
//   y_g   = y0_g + q_g H_in            (wkv7_segment_correct, all tokens at once)
// Both in fp32; state matrices use the pool layout [j][i] (key j, value i),
// on which Phi acts from the left.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

constexpr int kCombThreads = 256;
constexpr int kMat = kHead * kHead;  // floats per 64 x 64 head matrix

// One (sequence, head) per workgroup; thread t owns row j = t / 4 and the 16
// columns 16 (t % 4) .. + 15 of the 64 x 64 products.
__global__ __launch_bounds__(kCombThreads) void segment_chain_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const float* __restrict__ alt,
    int64_t alt_rows, const int32_t* __restrict__ seq_tab, int nseq,
    const int32_t* __restrict__ seg_tab, int nsegs, float* __restrict__ hin) {
  __shared__ float4 cur[kMat / 4];  // H_in, row-major [m][c]
  const int64_t s = blockIdx.x / H;
  const int64_t head = blockIdx.x - s * H;
  if (s >= nseq) return;
  const int64_t slot = seq_tab[3 * s];
  const int first = seq_tab[3 * s + 1], count = seq_tab[3 * s + 2];
  if (slot < 0 || slot >= num_rows || first < 0 || count < 0 || first + count > nsegs) return;
  float4* state = reinterpret_cast<float4*>(wkv + (slot * H + head) * kMat);
  const int t = threadIdx.x;
  for (int i = t; i < kMat / 4; i += kCombThreads) cur[i] = state[i];
  __syncthreads();
  const int j = t >> 2, c4 = (t & 3) * 4;  // row j, float4 columns c4 .. c4 + 3
  for (int n = 0; n < count; ++n) {
    const int seg = first + n;
    const int64_t row_main = seg_tab[2 * seg], row_phi = seg_tab[2 * seg + 1];
    float4* hout = reinterpret_cast<float4*>(hin + (int64_t(seg) * H + head) * kMat);
    for (int i = t; i < kMat / 4; i += kCombThreads) hout[i] = cur[i];
    const bool ok = row_main >= 0 && row_main < alt_rows && row_phi >= 0 && row_phi < alt_rows;
    float4 acc[4];
    if (ok) {
      const float4* phi = reinterpret_cast<const float4*>(alt + (row_phi * H + head) * kMat);
      const float4* h0 = reinterpret_cast<const float4*>(alt + (row_main * H + head) * kMat);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = h0[j * 16 + c4 + q];
      for (int m4 = 0; m4 < 16; ++m4) {
        const float4 p = phi[j * 16 + m4];
        const float pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 4 * m4 + e;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 hv = cur[m * 16 + c4 + q];
            acc[q].x = fmaf(pv[e], hv.x, acc[q].x);
            acc[q].y = fmaf(pv[e], hv.y, acc[q].y);
            acc[q].z = fmaf(pv[e], hv.z, acc[q].z);
            acc[q].w = fmaf(pv[e], hv.w, acc[q].w);
          }
        }
      }
    }
    __syncthreads();  // every thread has read cur
    if (ok) {
#pragma unroll
      for (int q = 0; q < 4; ++q) cur[j * 16 + c4 + q] = acc[q];
    }
    __syncthreads();
  }
  for (int i = t; i < kMat / 4; i += kCombThreads) state[i] = cur[i];
}

// One block of at most 64 tokens of one head per workgroup; thread t owns
// token t / 4 of the block and the 16 value columns 16 (t % 4) .. + 15.
template <bool kF32Out>
__global__ __launch_bounds__(kCombThreads) void segment_correct_kernel(
    int64_t total_tokens, int H, const float* __restrict__ y0, const float* __restrict__ q,
    const int32_t* __restrict__ blk_tab, int nblk, const float* __restrict__ hin, int nsegs,
    void* __restrict__ y) {
  __shared__ float4 mat[kMat / 4];
  const int64_t blk = blockIdx.x / H;
  const int64_t head = blockIdx.x - blk * H;
  if (blk >= nblk) return;
  const int64_t tok0 = blk_tab[3 * blk];
  const int cnt = blk_tab[3 * blk + 1], seg = blk_tab[3 * blk + 2];
  const bool corr = seg >= 0 && seg < nsegs;
  const int t = threadIdx.x;
  if (corr) {
    const float4* src = reinterpret_cast<const float4*>(hin + (int64_t(seg) * H + head) * kMat);
    for (int i = t; i < kMat / 4; i += kCombThreads) mat[i] = src[i];
  }
  __syncthreads();
  const int ti = t >> 2, c4 = (t & 3) * 4;
  const int64_t tok = tok0 + ti;
  if (ti >= cnt || tok < 0 || tok >= total_tokens) return;
  const int64_t base = (tok * H + head) * kHead;
  const float4* y0r = reinterpret_cast<const float4*>(y0 + base);
  float4 acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = y0r[c4 + e];
  if (corr) {
    const float4* qr = reinterpret_cast<const float4*>(q + base);
    for (int m4 = 0; m4 < 16; ++m4) {
      const float4 qv = qr[m4];
      const float qs[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 4 * m4 + e;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float4 hv = mat[m * 16 + c4 + u];
          acc[u].x = fmaf(qs[e], hv.x, acc[u].x);
          acc[u].y = fmaf(qs[e], hv.y, acc[u].y);
          acc[u].z = fmaf(qs[e], hv.z, acc[u].z);
          acc[u].w = fmaf(qs[e], hv.w, acc[u].w);
        }
      }
    }
  }
  if (kF32Out) {
    float4* yr = reinterpret_cast<float4*>(static_cast<float*>(y) + base);
#pragma unroll
    for (int e = 0; e < 4; ++e) yr[c4 + e] = acc[e];
  } else {
    uint2* yr = reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + base);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      yr[c4 + e] = make_uint2(pack_bf16(acc[e].x, acc[e].y), pack_bf16(acc[e].z, acc[e].w));
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_segment_chain(float* wkv_layer, int64_t num_rows, int32_t H,
                                  const float* state_alt, int64_t alt_rows,
                                  const int32_t* seq_tab, int32_t nseq, const int32_t* seg_tab,
                                  int32_t nsegs, float* hin, void* stream) {
  if (num_rows < 1 || H < 1 || alt_rows < 0 || nseq < 0 || nsegs < 0) return WKV7_ERR_ARG;
  if (nseq == 0) return WKV7_OK;
  if (!wkv_layer || !seq_tab || (nsegs > 0 && (!seg_tab || !state_alt || !hin)))
    return WKV7_ERR_ARG;
  if (!aligned16(wkv_layer) || (nsegs > 0 && (!aligned16(state_alt) || !aligned16(hin))))
    return WKV7_ERR_SHAPE;
  const int64_t blocks = int64_t(nseq) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  segment_chain_kernel<<<unsigned(blocks), kCombThreads, 0, as_stream(stream)>>>(
      wkv_layer, num_rows, H, state_alt, alt_rows, seq_tab, nseq, seg_tab, nsegs, hin);
  return launch_status();
}

extern "C" int wkv7_segment_correct(int64_t total_tokens, int32_t H, const float* y0,
                                    const float* q, const int32_t* blk_tab, int32_t nblk,
                                    const float* hin, int32_t nsegs, void* y, int32_t y_dtype,
                                    void* stream) {
  if (total_tokens < 0 || H < 1 || nblk < 0 || nsegs < 0) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (nblk == 0 || total_tokens == 0) return WKV7_OK;
  if (!y0 || !blk_tab || !y || (nsegs > 0 && (!q || !hin))) return WKV7_ERR_ARG;
  if (!aligned16(y0) || (nsegs > 0 && (!aligned16(q) || !aligned16(hin))) ||
      (y_dtype == WKV7_Y_F32 ? !aligned16(y) : (reinterpret_cast<uintptr_t>(y) & 7u)))
    return WKV7_ERR_SHAPE;
  const int64_t blocks = int64_t(nblk) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  if (y_dtype == WKV7_Y_F32)
    segment_correct_kernel<true><<<unsigned(blocks), kCombThreads, 0, s>>>(
        total_tokens, H, y0, q, blk_tab, nblk, hin, nsegs, y);
  else
    segment_correct_kernel<false><<<unsigned(blocks), kCombThreads, 0, s>>>(
        total_tokens, H, y0, q, blk_tab, nblk, hin, nsegs, y);
  return launch_status();
}
