// Varlen WKV7 prefill over slot states: chunked scan on MFMA.
//
// One workgroup (4 wavefronts) walks one (sequence, head) in 64-token chunks;
// the 64x64 fp32 state stays in MFMA accumulator registers for the whole
// sequence (wave q owns value columns [16q, 16q+16)) and touches HBM only to
// load the slot state at the start and store it at the end.
//
// A chunk is solved as four 16-token sub-chunks. With G_t the inclusive
// cumulative log-decay inside a sub-chunk (G_{-1} = 0):
//   A^_t = a_t e^{G_{t-1}}   R^_t = scale r_t e^{G_t}   B~_s = b_s e^{-G_s}   K~_s = k_s e^{-G_s}
//   L_ab = tril(A^ B~^T, -1)  L_ak = tril(A^ K~^T, -1)  M_rb = tril(R^ B~^T)  M_rk = tril(R^ K~^T)
//   P  = (I - L_ab)^{-1} (A^ h + L_ak V)            (row t: p_t = a_t^T h_{t-1})
//   Y  = R^ h + M_rb P + M_rk V
//   h' = diag(e^{G_15}) (h + B~^T P + K~^T V)
// Sub-chunk referencing keeps every decay factor within e^{+-16 |w|}, far from
// fp32/bf16 range limits. Padding tokens past the end of a sequence enter as
// w = 0 (decay 1) and zero vectors, i.e. identity steps.
//
// Phase I (state independent, wave u builds sub-chunk u): decays, the four
// operand matrices, the four 16x16 scores and T = (I - L_ab)^{-1} (forward
// substitution in fp32), all staged in LDS. Phase II (state chain, wave q for
// its 16 columns, sub-chunks in order): the products above on MFMA.
//
// Precision: every MFMA operand that is not an exact bf16 input is split into
// bf16 hi + lo parts and a product is formed as hi*hi + hi*lo + lo*hi with
// fp32 accumulation (~2^-16 relative per product); products with the exact
// bf16 v need two MFMAs. Operand layouts used below (v_mfma_f32_16x16x32_bf16,
// lane l, li = l%16, lg = l/16): A lane holds A[li][8lg..8lg+7] of a 32-wide k
// block, B lane holds B[8lg..8lg+7][li], the accumulator holds D[4lg..4lg+3][li].
// Contractions over 16 tokens put k = 4lg..4lg+3 in elements 0..3 of both
// operands and zeros in 4..7; with that labelling a 16x16 accumulator is
// already the B operand of the next 16-token product, straight from registers.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr int kSub = 16;
constexpr int kNumSub = kChunk / kSub;
constexpr int kThreads = 256;
// LDS row pitches (in bf16 elements), padded so that the 16 rows one MFMA
// operand load touches fall in distinct banks: 144 B rows for the 64-wide
// arrays, 40 B rows for the 16-wide ones.
constexpr int kPR = kHead + 8;  // [row][64] arrays
constexpr int kPS = kSub + 4;   // [row][16] arrays

struct __align__(16) SubShared {
  uint16_t A[2][kSub * kPR];      // A^ hi/lo  [t][j]
  uint16_t R[2][kSub * kPR];      // R^ hi/lo  [t][j]
  uint16_t BT[2][kHead * kPS];    // B~^T hi/lo [j][s]
  uint16_t KT[2][kHead * kPS];    // K~^T hi/lo [j][s]
  uint16_t VT[kHead * kPS];       // v^T (exact bf16) [i][s]
  uint16_t Lak[2][kSub * kPS];    // [t][s]
  uint16_t Mrb[2][kSub * kPS];
  uint16_t Mrk[2][kSub * kPS];
  uint16_t T[2][kSub * kPS];
  float gam[kHead];               // e^{G_15} per key index
};

struct __align__(16) WaveScratch {
  union {
    struct {
      uint16_t Bs[2][kSub * kPR];    // B~ hi/lo [s][j] (score B operand)
      uint16_t Ks[2][kSub * kPR];    // K~ hi/lo [s][j]
      float L[kSub * kSub];          // L_ab fp32 [t][s] (broadcast reads only)
    } p1;
    struct {
      uint16_t hT[2][kSub * kPR];    // this wave's state columns, hi/lo [i][j]
    } p2;
  };
};

// x = hi + lo: hi = bf16(x) and lo = bf16(x - hi) (the difference is exact in
// fp32), both rounded to nearest even; |x - hi - lo| <= 2^-18 |x|. Two values
// per call, packed as bf16 pairs (first value in the low half).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16(a, b);
  lo = pack_bf16(a - bf16_lo(hi), b - bf16_hi(hi));
}

__device__ __forceinline__ void pack_split(const f32x4& x, uint2& hi, uint2& lo) {
  split2(x[0], x[1], hi.x, lo.x);
  split2(x[2], x[3], hi.y, lo.y);
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }

__device__ __forceinline__ f32x4 mma32(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// K = 16 product on the 16x16x32 instruction, upper half of k zero-padded.
// (Results of the legacy 16x16x16 bf16 instruction read back by VALU came out
// nondeterministically wrong on gfx950 with this toolchain's wait-state
// insertion; the padded 16x16x32 form costs the same issue slot and is exact.)
__device__ __forceinline__ f32x4 mma16(const uint2& a, const uint2& b, f32x4 c) {
  const uint4 a8 = make_uint4(a.x, a.y, 0u, 0u), b8 = make_uint4(b.x, b.y, 0u, 0u);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a8),
                                                 __builtin_bit_cast(bf16x8, b8), c, 0, 0, 0);
}
// (ah + al)(bh + bl) without the lo*lo term, small terms first.
__device__ __forceinline__ f32x4 mma32x3(const uint4& ah, const uint4& al, const uint4& bh,
                                         const uint4& bl, f32x4 c) {
  c = mma32(al, bh, c);
  c = mma32(ah, bl, c);
  return mma32(ah, bh, c);
}
__device__ __forceinline__ f32x4 mma16x3(const uint2& ah, const uint2& al, const uint2& bh,
                                         const uint2& bl, f32x4 c) {
  c = mma16(al, bh, c);
  c = mma16(ah, bl, c);
  return mma16(ah, bh, c);
}
__device__ __forceinline__ f32x4 mma16x2(const uint2& ah, const uint2& al, const uint2& b, f32x4 c) {
  c = mma16(al, b, c);
  return mma16(ah, b, c);
}

// Orders this wave's LDS writes before its later LDS reads by other lanes of
// the same wave. The LDS executes one wave's instructions in order, so only
// the compiler has to be kept from reordering across this point.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Inputs {
  const uint16_t *r, *w, *k, *v, *a, *b;
};

// One sub-chunk of inputs as lane (t = lane % 16, g = lane / 16) sees it:
// channels [16g, 16g + 16) of token t for each vector, as 2 x 8 bf16.
struct SubLoad {
  uint4 r[2], w[2], k[2], v[2], a[2], b[2];
};

__device__ __forceinline__ void load_vec(uint4 (&d)[2], const uint16_t* base, int64_t io, bool valid) {
  const uint4* p = reinterpret_cast<const uint4*>(base + io);
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  const uint4 x0 = p[0], x1 = p[1];
  d[0] = valid ? x0 : z;
  d[1] = valid ? x1 : z;
}

// Tokens past the end of the sequence load the last real token's row (always
// in bounds) and are replaced by zeros, so every lane issues its loads
// unconditionally; zero vectors with w = 0 are identity steps.
__device__ __forceinline__ void load_sub(SubLoad& d, const Inputs& in, int64_t tok0, int64_t t_end,
                                         int64_t tstride, int64_t hoff, int lane) {
  const int64_t tok = tok0 + (lane & 15);
  const bool valid = tok < t_end;
  const int64_t io = (valid ? tok : t_end - 1) * tstride + hoff + 16 * (lane >> 4);
  load_vec(d.r, in.r, io, valid);
  load_vec(d.w, in.w, io, valid);
  load_vec(d.k, in.k, io, valid);
  load_vec(d.v, in.v, io, valid);
  load_vec(d.a, in.a, io, valid);
  load_vec(d.b, in.b, io, valid);
}

// element e (0..15) of a 16-wide bf16 vector held as 2 x uint4
__device__ __forceinline__ float elem(const uint4 (&x)[2], int e) {
  const uint4& q = x[e >> 3];
  const uint32_t w = (e & 6) == 0 ? q.x : (e & 6) == 2 ? q.y : (e & 6) == 4 ? q.z : q.w;
  return (e & 1) ? bf16_hi(w) : bf16_lo(w);
}
__device__ __forceinline__ uint16_t elem_bits(const uint4 (&x)[2], int e) {
  const uint4& q = x[e >> 3];
  const uint32_t w = (e & 6) == 0 ? q.x : (e & 6) == 2 ? q.y : (e & 6) == 4 ? q.z : q.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : w);
}

// Value of the lane one to the left in the DPP row; the first lane gets `first`.
__device__ __forceinline__ float row_prev(float x, float first) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(x), 0x111, 0xf, 0xf, false));
}

// Inclusive prefix sum over the 16 lanes of a DPP row (row_shr 1, 2, 4, 8).

template <int kShift>
__device__ __forceinline__ float row_shr(float x) {
  // lanes whose source falls outside the row receive 0 (the `old` operand)
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + kShift, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_prefix_sum(float x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}

template <bool kF32Out>
__global__ __launch_bounds__(kThreads) void prefill_chunked_kernel(
    float* __restrict__ wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu_seqlens, Inputs in, void* __restrict__ y,
    int64_t total_tokens, int zero_init, float scale) {
  __shared__ SubShared sh[kNumSub];
  __shared__ WaveScratch scratch[4];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int64_t seq = blockIdx.x / H;
  const int64_t head = blockIdx.x - seq * H;
  const int64_t slot = slot_ids[seq];
  if (slot < 0 || slot >= num_rows) return;  // uniform: the whole block leaves
  const int64_t t_end = min(max(int64_t(cu_seqlens[seq + 1]), int64_t(0)), total_tokens);
  const int64_t t_beg = min(max(int64_t(cu_seqlens[seq]), int64_t(0)), t_end);
  const int64_t tstride = int64_t(H) * kHead;
  const int64_t hoff = head * kHead;
  float* hbase = wkv + (slot * H + head) * (kHead * kHead);
  const int col0 = kSub * wave;  // this wave's value columns [col0, col0 + 16)

  // State columns of this wave as four 16x16 accumulator tiles (key blocks jb).
  f32x4 h[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      h[jb][rr] = zero_init ? 0.f : hbase[(16 * jb + 4 * lg + rr) * kHead + col0 + li];

  SubLoad pf;
  if (t_beg < t_end) load_sub(pf, in, t_beg + kSub * wave, t_end, tstride, hoff, lane);

  for (int64_t c0 = t_beg; c0 < t_end; c0 += kChunk) {
    // ---------------- phase I: wave `wave` builds sub-chunk `wave` ----------------
    {
      SubShared& S = sh[wave];
      auto& P1 = scratch[wave].p1;
      // lane = (token t, channel group g): log2 cumulative decay by a row scan
      const int t = lane & 15, g = lane >> 4;
      constexpr float kLog2e = 1.4426950408889634f;
      uint32_t ah[8], al[8], rh[8], rl[8], bh[8], bl[8], kh[8], kl[8];
      float gam_hi[16];
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        float ex[2], in_[2], eh[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float w2 = elem(pf.w, e + q) * kLog2e;
          const float G = row_prefix_sum(w2);  // through token t
          in_[q] = __builtin_amdgcn_exp2f(-G);
          eh[q] = __builtin_amdgcn_exp2f(G);
          ex[q] = row_prev(eh[q], 1.f);  // decay through token t-1
          gam_hi[e + q] = eh[q];
        }
        split2(elem(pf.a, e) * ex[0], elem(pf.a, e + 1) * ex[1], ah[e / 2], al[e / 2]);
        split2(elem(pf.r, e) * scale * eh[0], elem(pf.r, e + 1) * scale * eh[1], rh[e / 2], rl[e / 2]);
        split2(elem(pf.b, e) * in_[0], elem(pf.b, e + 1) * in_[1], bh[e / 2], bl[e / 2]);
        split2(elem(pf.k, e) * in_[0], elem(pf.k, e + 1) * in_[1], kh[e / 2], kl[e / 2]);
      }
      const int ro = t * kPR + 16 * g;  // row t, channels 16g.. (row layouts [t][j])
      auto st32 = [](uint16_t* dst, const uint32_t (&v)[8]) {
        reinterpret_cast<uint4*>(dst)[0] = make_uint4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<uint4*>(dst)[1] = make_uint4(v[4], v[5], v[6], v[7]);
      };
      st32(&S.A[0][ro], ah);
      st32(&S.A[1][ro], al);
      st32(&S.R[0][ro], rh);
      st32(&S.R[1][ro], rl);
      st32(&P1.Bs[0][ro], bh);
      st32(&P1.Bs[1][ro], bl);
      st32(&P1.Ks[0][ro], kh);
      st32(&P1.Ks[1][ro], kl);
      // transposed layouts [j][s]: 16 lanes of a row write 32 contiguous bytes
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int to = (16 * g + e) * kPS + t;
        const int sh16 = (e & 1) * 16;
        S.BT[0][to] = static_cast<uint16_t>(bh[e / 2] >> sh16);
        S.BT[1][to] = static_cast<uint16_t>(bl[e / 2] >> sh16);
        S.KT[0][to] = static_cast<uint16_t>(kh[e / 2] >> sh16);
        S.KT[1][to] = static_cast<uint16_t>(kl[e / 2] >> sh16);
        S.VT[to] = elem_bits(pf.v, e);
      }
      if (t == kSub - 1) {
#pragma unroll
        for (int e = 0; e < 16; e += 4)
          *reinterpret_cast<float4*>(&S.gam[16 * g + e]) =
              make_float4(gam_hi[e], gam_hi[e + 1], gam_hi[e + 2], gam_hi[e + 3]);
      }
      wave_sync();

      // scores: rows t = query token, cols s = key token, contraction over j
      f32x4 lab = {0.f, 0.f, 0.f, 0.f}, lak = lab, mrb = lab, mrk = lab;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int off = li * kPR + 32 * kb + 8 * lg;
        const uint4 ah = ld16(&S.A[0][off]), al = ld16(&S.A[1][off]);
        const uint4 rh = ld16(&S.R[0][off]), rl = ld16(&S.R[1][off]);
        const uint4 bh = ld16(&P1.Bs[0][off]), bl = ld16(&P1.Bs[1][off]);
        const uint4 kh = ld16(&P1.Ks[0][off]), kl = ld16(&P1.Ks[1][off]);
        lab = mma32x3(ah, al, bh, bl, lab);
        lak = mma32x3(ah, al, kh, kl, lak);
        mrb = mma32x3(rh, rl, bh, bl, mrb);
        mrk = mma32x3(rh, rl, kh, kl, mrk);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int tq = 4 * lg + rr, s = li;
        const int o = tq * kPS + s;
        P1.L[tq * kSub + s] = s < tq ? lab[rr] : 0.f;
        uint32_t hi, lo;
        split2(s < tq ? lak[rr] : 0.f, s <= tq ? mrb[rr] : 0.f, hi, lo);
        S.Lak[0][o] = static_cast<uint16_t>(hi);
        S.Lak[1][o] = static_cast<uint16_t>(lo);
        S.Mrb[0][o] = static_cast<uint16_t>(hi >> 16);
        S.Mrb[1][o] = static_cast<uint16_t>(lo >> 16);
        split2(s <= tq ? mrk[rr] : 0.f, 0.f, hi, lo);
        S.Mrk[0][o] = static_cast<uint16_t>(hi);
        S.Mrk[1][o] = static_cast<uint16_t>(lo);
      }
      wave_sync();

      // T = (I - L_ab)^{-1}, column c = lane, by forward substitution in fp32
      if (lane < kSub) {
        const int c = lane;
        // all of L (strictly lower, broadcast reads) into registers first
        float Lr[kSub][kSub];
#pragma unroll
        for (int tq = 1; tq < kSub; ++tq)
#pragma unroll
          for (int q = 0; q < kSub; q += 4) {
            if (q >= tq) break;
            const float4 v4 = *reinterpret_cast<const float4*>(&P1.L[tq * kSub + q]);
            Lr[tq][q] = v4.x;
            Lr[tq][q + 1] = v4.y;
            Lr[tq][q + 2] = v4.z;
            Lr[tq][q + 3] = v4.w;
          }
        float tc[kSub];
#pragma unroll
        for (int tq = 0; tq < kSub; ++tq) {
          float acc = (tq == c) ? 1.f : 0.f;
#pragma unroll
          for (int q = 0; q < tq; ++q) acc = fmaf(Lr[tq][q], tc[q], acc);
          tc[tq] = acc;
        }
#pragma unroll
        for (int tq = 0; tq < kSub; tq += 2) {
          uint32_t hi, lo;
          split2(tc[tq], tc[tq + 1], hi, lo);
          S.T[0][tq * kPS + c] = static_cast<uint16_t>(hi);
          S.T[1][tq * kPS + c] = static_cast<uint16_t>(lo);
          S.T[0][(tq + 1) * kPS + c] = static_cast<uint16_t>(hi >> 16);
          S.T[1][(tq + 1) * kPS + c] = static_cast<uint16_t>(lo >> 16);
        }
      }
    }
    __syncthreads();

    // prefetch the next chunk's sub-chunk for this wave while phase II runs
    if (c0 + kChunk < t_end)
      load_sub(pf, in, c0 + kChunk + kSub * wave, t_end, tstride, hoff, lane);

    // ---------------- phase II: wave `wave` runs its 16 columns ----------------
    {
      auto& P2 = scratch[wave].p2;
#pragma unroll 1
      for (int u = 0; u < kNumSub; ++u) {
        const SubShared& S = sh[u];
        // shared operands of this sub-chunk, all requested up front
        uint4 ah[2], al[2], rh[2], rl[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int off = li * kPR + 32 * kb + 8 * lg;
          ah[kb] = ld16(&S.A[0][off]);
          al[kb] = ld16(&S.A[1][off]);
          rh[kb] = ld16(&S.R[0][off]);
          rl[kb] = ld16(&S.R[1][off]);
        }
        const int so = li * kPS + 4 * lg;  // A operand [t = li][s = 4lg..]
        const uint2 vb = ld8(&S.VT[(col0 + li) * kPS + 4 * lg]);
        const uint2 lakh = ld8(&S.Lak[0][so]), lakl = ld8(&S.Lak[1][so]);
        const uint2 th = ld8(&S.T[0][so]), tl = ld8(&S.T[1][so]);
        const uint2 mrbh = ld8(&S.Mrb[0][so]), mrbl = ld8(&S.Mrb[1][so]);
        const uint2 mrkh = ld8(&S.Mrk[0][so]), mrkl = ld8(&S.Mrk[1][so]);
        uint2 bth[4], btl[4], kth[4], ktl[4];
        float4 gm[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int jo = (16 * jb + li) * kPS + 4 * lg;  // A operand [j = 16jb + li][s = 4lg..]
          bth[jb] = ld8(&S.BT[0][jo]);
          btl[jb] = ld8(&S.BT[1][jo]);
          kth[jb] = ld8(&S.KT[0][jo]);
          ktl[jb] = ld8(&S.KT[1][jo]);
          gm[jb] = *reinterpret_cast<const float4*>(&S.gam[16 * jb + 4 * lg]);
        }
        // stage the state columns as the B operand [i][j] (hi/lo)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          uint2 hi, lo;
          pack_split(h[jb], hi, lo);
          const int o = li * kPR + 16 * jb + 4 * lg;
          *reinterpret_cast<uint2*>(&P2.hT[0][o]) = hi;
          *reinterpret_cast<uint2*>(&P2.hT[1][o]) = lo;
        }
        wave_sync();

        f32x4 X = {0.f, 0.f, 0.f, 0.f}, Z = X;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int off = li * kPR + 32 * kb + 8 * lg;
          const uint4 hh = ld16(&P2.hT[0][off]), hl = ld16(&P2.hT[1][off]);
          X = mma32x3(ah[kb], al[kb], hh, hl, X);
          Z = mma32x3(rh[kb], rl[kb], hh, hl, Z);
        }
        X = mma16x2(lakh, lakl, vb, X);  // rhs = A^ h + L_ak V
        uint2 xh, xl;
        pack_split(X, xh, xl);
        f32x4 Pm = {0.f, 0.f, 0.f, 0.f};
        Pm = mma16x3(th, tl, xh, xl, Pm);  // P = T rhs
        uint2 ph, pl;
        pack_split(Pm, ph, pl);
        Z = mma16x3(mrbh, mrbl, ph, pl, Z);
        Z = mma16x2(mrkh, mrkl, vb, Z);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int64_t tok = c0 + kSub * u + 4 * lg + rr;
          if (tok < t_end) {
            const int64_t yo = tok * tstride + hoff + col0 + li;
            if (kF32Out)
              static_cast<float*>(y)[yo] = Z[rr];
            else
              static_cast<uint16_t*>(y)[yo] = f32_to_bf16(Z[rr]);
          }
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          h[jb] = mma16x3(bth[jb], btl[jb], ph, pl, h[jb]);
          h[jb] = mma16x2(kth[jb], ktl[jb], vb, h[jb]);
          h[jb][0] *= gm[jb].x;
          h[jb][1] *= gm[jb].y;
          h[jb][2] *= gm[jb].z;
          h[jb][3] *= gm[jb].w;
        }
        wave_sync();
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      hbase[(16 * jb + 4 * lg + rr) * kHead + col0 + li] = h[jb][rr];
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
  // inputs are read as 16-byte vectors
  const uintptr_t align = reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(w) |
                          reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                          reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
  if (align & 15u) return WKV7_ERR_SHAPE;
  if (workspace_bytes < wkv7_prefill_workspace_bytes(H, nseq, total_tokens)) return WKV7_ERR_WORKSPACE;
  (void)workspace;
  const int64_t blocks = int64_t(nseq) * H;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  const Inputs in{r, w, k, v, a, b};
  if (y_dtype == WKV7_Y_F32)
    prefill_chunked_kernel<true><<<unsigned(blocks), kThreads, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, cu_seqlens, in, y, total_tokens, zero_init, scale);
  else
    prefill_chunked_kernel<false><<<unsigned(blocks), kThreads, 0, s>>>(
        wkv_layer, num_rows, H, slot_ids, cu_seqlens, in, y, total_tokens, zero_init, scale);
  return launch_status();
}
