// Device code of the WKV7 chunked prefill (included by wkv7_prefill.hip, the
// whole-head kernel and the entry points, and by wkv7_prefill_quarter.hip,
// the quarter-head kernel for launches with few (sequence, head) pairs; two
// translation units so that neither kernel changes the other's code).
//
//
// One workgroup (16 wavefronts) walks one (sequence, head). The 64x64 fp32
// state stays in MFMA accumulator registers for the whole sequence (state
// wave q owns value columns [16q, 16q+16)) and touches HBM only to load the
// slot state at the start and store it at the end.
//
// The sequence is solved in 16-token sub-chunks. With G_t the inclusive
// cumulative log-decay inside a sub-chunk (G_{-1} = 0):
//   A^_t = a_t e^{G_{t-1}}   R^_t = scale r_t e^{G_t}   B~_s = b_s e^{-G_s}   K~_s = k_s e^{-G_s}
//   L_ab = tril(A^ B~^T, -1)  L_ak = tril(A^ K~^T, -1)  M_rb = tril(R^ B~^T)  M_rk = tril(R^ K~^T)
//   P  = (I - L_ab)^{-1} (A^ h + L_ak V)            (row t: p_t = a_t^T h_{t-1})
//   Y  = R^ h + M_rb P + M_rk V
//   h' = diag(e^{G_15}) (h + B~^T P + K~^T V)
// Sub-chunk referencing keeps every decay factor within e^{+-16 |w|}, far from
// fp32/bf16 range limits for RWKV-7's decays (|w| < 0.61 per token). Padding
// tokens past the end of a sequence enter as w = 0 (decay 1) and zero
// vectors, i.e. identity steps.
//
// Schedule: a four-deep software pipeline over sub-chunks, one workgroup
// barrier per tick. In tick k four state waves run sub-chunk k's state step
// (the products above, 16 value columns each; y goes to an LDS staging
// buffer) while twelve more waves prepare the sub-chunks further ahead:
//   inverse   (sub-chunk k+1): T = (I - L_ab)^{-1}, 4 columns per wave
//   scores    (sub-chunk k+2): L_ab, L_ak, M_rb, M_rk, one per wave; they
//                              also store sub-chunk k-1's y from the staging
//                              buffer as whole rows
//   operands  (sub-chunk k+3): decays and operand matrices, 16 key channels
//                              per wave (in the buffer path the cumulative
//                              sums G are one MFMA with a triangle of ones)
// Sub-chunk j lives in ring slot j % 4 from tick j-3 to tick j; its inputs
// are loaded two ticks before they are used, as whole 128-byte rows straight
// into an LDS staging ring of three sub-chunks (the buffer path, every batch
// whose input offsets fit 31 bits; one more fill tick) or into registers
// (larger batches).
//
// Precision: MFMA operands that are not exact bf16 inputs are split into bf16
// hi + lo parts, a product formed as hi*hi + hi*lo + lo*hi with fp32
// accumulation (~2^-16 relative per product), except two that enter as one
// bf16 each: A^ and T (solved in fp32, then rounded). Those cost ~2^-9
// relative on P only. h enters the A^ h product split as well: as one bf16
// it left a 4096-token run with no decay on half the key channels at 8e-4
// relative L2 on y and state (1.5e-4 split). Products with the exact bf16 v
// need one MFMA per term pair. Operand layouts below
// (v_mfma_f32_16x16x32_bf16, lane l, li = l%16, lg = l/16): A lane holds
// A[li][8lg..8lg+7] of a 32-wide k block, B lane holds B[8lg..8lg+7][li], the
// accumulator holds D[4lg..4lg+3][li]. Contractions over 16 tokens put
// k = 4lg..4lg+3 in elements 0..3 of both operands and zeros in 4..7; with
// that labelling a 16x16 accumulator is already the B operand of the next
// 16-token product, straight from registers, and an LDS transpose read of
// token rows 4lg..4lg+3 is the A operand B~^T / K~^T or the B operand v. Contractions over the 64 key
// rows take the k labels of a 32-row block in the order the state tiles hold
// them (key_pos below), so the state is a B operand straight from registers
// as well.
#pragma once

#include <type_traits>

#include "wkv7_common.h"

namespace wkv7 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSub = 16;
constexpr int kRing = 4;
constexpr int kOpWaves = 4;                      // operand wavefronts
constexpr int kChan = kHead / (4 * kOpWaves);  // key channels per operand lane
constexpr int kThreads = kWave * (12 + kOpWaves);  // 4 state + operand + 4 score + 4 inverse
// The row-staging reads and the decay-sum product take 4 channels per lane (one 8-byte piece).
static_assert(kChan == 4, "operand lanes hold 4 key channels");
// LDS layouts. Every operand array is [token][64 channels] with unpadded
// 128 B rows whose 16 B chunks are XOR-swizzled by the row (chunk c of row r
// sits at c ^ (r & 7)): the MFMA operand loads (16 rows x 4 chunks per
// ds_read_b128) are then free of bank conflicts on gfx950, which 144 B padded
// rows are not (measured with the LDS bank-conflict counters). The state
// waves' transposed 16-token operands come from the same arrays through the
// LDS transpose reads (ld_tr), so the operand waves store each value once, as
// 8-byte row stores (they used to store B~^T, K~^T and v^T again, transposed,
// with 2-byte stores).
constexpr int kPR = kHead;  // [row][64] arrays: 128 B rows, chunk-swizzled
// element offset of key-position element e (0..63) of row r of a [row][64] array
__device__ __forceinline__ int rk_off(int r, int e) {
  return r * kPR + ((((e >> 3) ^ r) & 7) << 3) + (e & 7);
}
constexpr int kPG = kHead + 4;     // gam rows (floats)

// Position of key row j in the [t][.] operand arrays. Key rows of the 32-row
// block kb, as the state tiles h[2kb], h[2kb+1] hold them in lane group lg,
// are 32kb + 4lg + {0..3} and 32kb + 16 + 4lg + {0..3}; they take k labels
// 8lg .. 8lg+7 of that block.
__device__ __forceinline__ int key_pos(int j) {
  const int kb = j >> 5, jj = j & 31;
  return 32 * kb + 8 * ((jj >> 2) & 3) + 4 * (jj >> 4) + (jj & 3);
}

// One sub-chunk's operands, every array row-major [token][channel]. The state
// waves read the transposed 16-token operands (B~^T, K~^T, v^T) straight from
// them with the LDS transpose reads, so nothing is stored twice.
struct __align__(16) Slot {
  uint16_t A[kSub * kPR];       // A^ as one bf16 [t][key_pos]
  uint16_t R[2][kSub * kPR];    // R^ hi/lo [t][key_pos]
  uint16_t B[2][kSub * kPR];    // B~ hi/lo [s][key_pos]
  uint16_t K[2][kSub * kPR];    // K~ hi/lo [s][key_pos]
  uint16_t V[kSub * kPR];       // v [s][value column], exact bf16 (natural order)
  uint4 M[4][kWave];            // T, L_ak, M_rb, M_rk as {hi, lo} in A-operand lane order
  float gam[kSub][kPG];         // e^{G_t}; row 15 is the sub-chunk's decay
};

// y of a sub-chunk staged for the score waves' row stores: [token][64 values]
// rows padded by 8 bytes (bf16) or 16 bytes (fp32) so the state waves' four
// lane groups write different banks.
constexpr int kYRowB = kHead * 2 + 8;   // bf16 row pitch in bytes
constexpr int kYRowF = kHead * 4 + 16;  // fp32 row pitch in bytes

struct __align__(16) Shared {
  Slot slot[kRing];
  float4 Lf[2][kWave];            // L_ab in fp32, A-operand lane order
  unsigned char ys[2][kSub * kYRowF];  // y of sub-chunks k (state waves) and k-1 (score waves)
  uint4 inb[3][6][kSub][8];  // input rows (r, w, k, v, a, b) of three sub-chunks, 128 B each
};

typedef __attribute__((address_space(3))) uint4 lds_uint4;
__device__ __forceinline__ uint32_t lds_addr(const uint4* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_uint4*)p));
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// LDS transpose read (ds_read_b64_tr_b16). Inside each 16-lane group, lane
// lam reads the 4 consecutive bf16 at its address, D[lam][0..3], and receives
// D[4 j + lam / 4][lam % 4] as element j. A lane that reads row r0 + lam / 4
// of a row-major [row][col] array at column c0 + 4 (lam % 4) therefore gets
// column c0 + lam at rows r0 .. r0 + 3: a 16-row fragment of the transpose.
__device__ __forceinline__ uint2 ld_tr(const uint16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

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

__device__ __forceinline__ f32x4 mma32(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// (The legacy 16x16x16 bf16 instruction is not used: its results read back by
// VALU came out nondeterministically wrong on gfx950 with this toolchain's
// wait-state insertion. 16-token products run on the 16x16x32 instruction
// with two terms per issue, see stage_state.)
// (ah + al)(bh + bl) without the lo*lo term, small terms first.
__device__ __forceinline__ f32x4 mma32x3(const uint4& ah, const uint4& al, const uint4& bh,
                                         const uint4& bl, f32x4 c) {
  c = mma32(al, bh, c);
  c = mma32(ah, bl, c);
  return mma32(ah, bh, c);
}

// Value of the lane one to the left in the DPP row; the first lane gets `first`.
__device__ __forceinline__ float row_prev(float x, float first) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(x), 0x111, 0xf, 0xf, false));
}

template <int kShift>
__device__ __forceinline__ float row_shr(float x) {
  // lanes whose source falls outside the row receive 0 (bound_ctrl)
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x110 + kShift, 0xf, 0xf, true));
}
// Inclusive prefix sum over the 16 lanes of a DPP row (row_shr 1, 2, 4, 8).
__device__ __forceinline__ float row_prefix_sum(float x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}

}  // namespace

// (Inputs and Runs have external linkage: prefill_quarter_launch, declared
// below and defined in the other translation unit, takes them.)
struct Inputs {
  const uint16_t *r, *w, *k, *v, *a, *b;
};

namespace {

struct SeqGeom {
  int64_t t_beg, t_end;  // token range of the sequence
  int64_t tstride;       // elements between consecutive tokens (H * 64)
  int64_t hoff;          // element offset of this head inside a token row
};

// One sub-chunk of inputs as lane (t = lane % 16, cg = lane / 16) of operand
// wave p sees it: kChan consecutive key channels starting at kChan (4p + cg)
// of token t, kChan bf16 per vector (kChan / 2 packed pairs).
struct SubIn {
  uint32_t r[kChan / 2], w[kChan / 2], k[kChan / 2], v[kChan / 2], a[kChan / 2], b[kChan / 2];
};

template <int N>
__device__ __forceinline__ void load_pairs(uint32_t (&d)[N], const uint16_t* p) {
  if constexpr (N == 2) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    d[0] = x.x;
    d[1] = x.y;
  } else {
    d[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

// Tokens past the end of the sequence load the last real token's row (always
// in bounds), so the loads are unconditional; the operand stage replaces them
// by zeros at the point of use, which keeps the loads in flight until then.
__device__ __forceinline__ void load_sub(SubIn& d, const Inputs& in, const SeqGeom& g, int64_t j,
                                         int lane, int part) {
  const int64_t tok = g.t_beg + kSub * j + (lane & 15);
  const int64_t io = (tok < g.t_end ? tok : g.t_end - 1) * g.tstride + g.hoff +
                     kChan * (4 * part + (lane >> 4));
  load_pairs(d.r, in.r + io);
  load_pairs(d.w, in.w + io);
  load_pairs(d.k, in.k + io);
  load_pairs(d.v, in.v + io);
  load_pairs(d.a, in.a + io);
  load_pairs(d.b, in.b + io);
}

// element m of packed bf16 pairs
template <int N>
__device__ __forceinline__ float elem(const uint32_t (&x)[N], int m) {
  return (m & 1) ? bf16_hi(x[m >> 1]) : bf16_lo(x[m >> 1]);
}

// kChan / 2 packed pairs -> an 8- or 4-byte LDS store
template <int N>
__device__ __forceinline__ void st_pairs(uint16_t* p, const uint32_t (&x)[N]) {
  if constexpr (N == 2)
    *reinterpret_cast<uint2*>(p) = make_uint2(x[0], x[1]);
  else
    *reinterpret_cast<uint32_t*>(p) = x[0];
}

// This lane's kChan channels of token t = lane % 16 of every input but w, and
// w transposed (channel 16 part + t at tokens 4 cg .. 4 cg + 3), from staging
// slot `slot` (rows stored with their 16-byte chunks XOR-swizzled by the
// token, see row_sources).
__device__ __forceinline__ void read_inputs(const Shared& sm, SubIn& d, int slot, int lane,
                                            int part) {
  const int t = lane & 15, cg = lane >> 4;
  const int c = 2 * part + (cg >> 1);
  const int pos = ((c ^ (t & 7)) * 16) + (cg & 1) * 8;
  auto rd = [&](uint32_t (&x)[kChan / 2], int input) {
    const uint2 v = *reinterpret_cast<const uint2*>(
        reinterpret_cast<const unsigned char*>(&sm.inb[slot][input][t][0]) + pos);
    x[0] = v.x;
    x[1] = v.y;
  };
  rd(d.r, 0);
  {
    // w transposed for the prefix-sum product of stage_operands: this lane
    // reads token 4 cg + t / 4 at channels 16 part + 4 (t % 4) and receives
    // channel 16 part + t at tokens 4 cg .. 4 cg + 3
    const int ts = 4 * cg + (t >> 2), ch = 16 * part + 4 * (t & 3);
    const int wpos = (((ch >> 3) ^ (ts & 7)) * 16) + (ch & 7) * 2;
    const uint2 v = ld_tr(reinterpret_cast<const uint16_t*>(
        reinterpret_cast<const unsigned char*>(&sm.inb[slot][1][ts][0]) + wpos));
    d.w[0] = v.x;
    d.w[1] = v.y;
  }
  rd(d.k, 2);
  rd(d.v, 3);
  rd(d.a, 4);
  rd(d.b, 5);
}

// Operands of sub-chunk j for key channels [4 kChan part, 4 kChan (part + 1)).
// kRows: the inputs come from the row-staging ring (read_inputs), where padding
// tokens are zeros already (the row loads stop at the sequence end) and w
// arrives transposed for the prefix-sum product; otherwise (registers, in
// operand layout) padding tokens arrive as copies of the last real token and
// are zeroed here. kScaled: scale != 1 (fla's default is 1, where R^ = r e^G
// needs no multiply by it).
template <bool kRows, bool kScaled>
__device__ __forceinline__ void stage_operands(Shared& sm, const SubIn& raw, int64_t j,
                                               const SeqGeom& g, int lane, int part, float scale) {
  constexpr int P = kChan / 2;
  Slot& S = sm.slot[j & (kRing - 1)];
  const int t = lane & 15, cg = lane >> 4;
  const bool valid = kRows || g.t_beg + kSub * j + t < g.t_end;
  // r and v of padding tokens only meet zero rows and columns (their k, b
  // and a are zero, and their y is not stored), so they need no masking.
  uint32_t wv[P], kv[P], av[P], bv[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    wv[i] = valid ? raw.w[i] : 0u;
    kv[i] = valid ? raw.k[i] : 0u;
    av[i] = valid ? raw.a[i] : 0u;
    bv[i] = valid ? raw.b[i] : 0u;
  }
  constexpr float kLog2e = 1.4426950408889634f;
  float A_[kChan], R_[kChan], B_[kChan], K_[kChan], eh[kChan];
  f32x4 wsum = {0.f, 0.f, 0.f, 0.f};
  if constexpr (kRows) {
    // wsum[m] = sum_{s <= t} w[s][c_m] for this lane's token t and channels
    // c_m, as the product (W^T L^T)[c][t]: A = W^T (wv holds channel 16 part + t
    // at tokens 4 cg .. 4 cg + 3) and the constant B[s][t] = [s <= t]. The
    // matrix cores take the sum off the vector ALUs, which the four wave
    // kinds share.
    const int s0 = 4 * cg;
    // On the 16x16x32 instruction with zero upper halves: results of the legacy
    // 16x16x16 one, read back by VALU, have come out wrong now and then on
    // gfx950 with this toolchain's wait-state insertion.
    const uint32_t one = 0x3f80u;  // bf16 1.0
    const uint4 lt = make_uint4((s0 <= t ? one : 0u) | (s0 + 1 <= t ? one << 16 : 0u),
                                (s0 + 2 <= t ? one : 0u) | (s0 + 3 <= t ? one << 16 : 0u), 0u, 0u);
    wsum = mma32(make_uint4(wv[0], wv[1], 0u, 0u), lt, wsum);
  }
#pragma unroll
  for (int m = 0; m < kChan; ++m) {
    // log2 decay through token t
    const float G = kRows ? wsum[m] * kLog2e : row_prefix_sum(elem(wv, m) * kLog2e);
    eh[m] = __builtin_amdgcn_exp2f(G);
    const float ex = row_prev(eh[m], 1.f);                 // decay through token t-1
    const float ie = __builtin_amdgcn_exp2f(-G);
    A_[m] = elem(av, m) * ex;
    R_[m] = kScaled ? elem(raw.r, m) * scale * eh[m] : elem(raw.r, m) * eh[m];
    B_[m] = elem(bv, m) * ie;
    K_[m] = elem(kv, m) * ie;
  }
  uint32_t ah[P], rh[P], rl[P], bh[P], bl[P], kh[P], kl[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    ah[i] = pack_bf16(A_[2 * i], A_[2 * i + 1]);
    split2(R_[2 * i], R_[2 * i + 1], rh[i], rl[i]);
    split2(B_[2 * i], B_[2 * i + 1], bh[i], bl[i]);
    split2(K_[2 * i], K_[2 * i + 1], kh[i], kl[i]);
  }

  const int c0 = kChan * (4 * part + cg);  // key channels c0 .. c0+kChan-1 (consecutive key_pos)
  const int ro = rk_off(t, key_pos(c0));  // kChan consecutive elements inside one chunk
  st_pairs(&S.A[ro], ah);
  st_pairs(&S.R[0][ro], rh);
  st_pairs(&S.R[1][ro], rl);
  st_pairs(&S.B[0][ro], bh);
  st_pairs(&S.B[1][ro], bl);
  st_pairs(&S.K[0][ro], kh);
  st_pairs(&S.K[1][ro], kl);
  st_pairs(&S.V[rk_off(t, c0)], raw.v);  // value channels c0 .. c0+kChan-1
  if constexpr (kChan == 4)
    *reinterpret_cast<float4*>(&S.gam[t][c0]) = make_float4(eh[0], eh[1], eh[2], eh[3]);
  else
    *reinterpret_cast<float2*>(&S.gam[t][c0]) = make_float2(eh[0], eh[1]);
}

// Score matrix `part` of sub-chunk j (0: L_ab, 1: L_ak, 2: M_rb, 3: M_rk) as
// the transposed product Y X^T, whose accumulator is the matrix in A-operand
// lane order. X is A^ (one bf16) for the L matrices and the split R^ for M.
template <int part>
__device__ __forceinline__ void stage_scores_of(Shared& sm, int64_t j, int lane) {
  Slot& S = sm.slot[j & (kRing - 1)];
  const int li = lane & 15, lg = lane >> 4;
  const uint16_t* Y = (part & 1) ? &S.K[0][0] : &S.B[0][0];
  constexpr int kLo = kSub * kPR;  // hi -> lo array distance
  f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int off = rk_off(li, 32 * kb + 8 * lg);
    const uint4 yh = ld16(Y + off);
    if constexpr (part < 2) {
      d = mma32(ld16(Y + kLo + off), ld16(&S.A[off]), d);  // (yh + yl) A^
      d = mma32(yh, ld16(&S.A[off]), d);
    } else {
      d = mma32x3(yh, ld16(Y + kLo + off), ld16(&S.R[0][off]), ld16(&S.R[1][off]), d);
    }
  }
  // d[r] = M[t = li][s = 4lg + r]; L_* keep s < t, M_* keep s <= t
  const int lim = li + (part >> 1);
#pragma unroll
  for (int r = 0; r < 4; ++r) d[r] = (4 * lg + r < lim) ? d[r] : 0.f;
  if constexpr (part == 0) {
    sm.Lf[j & 1][lane] = make_float4(d[0], d[1], d[2], d[3]);  // T is solved from it in fp32
  } else {
    uint2 hi, lo;
    pack_split(d, hi, lo);
    S.M[part][lane] = make_uint4(hi.x, hi.y, lo.x, lo.y);
  }
}

__device__ __forceinline__ void stage_scores(Shared& sm, int64_t j, int lane, int part) {
  switch (part) {  // wave-uniform
    case 0: stage_scores_of<0>(sm, j, lane); break;
    case 1: stage_scores_of<1>(sm, j, lane); break;
    case 2: stage_scores_of<2>(sm, j, lane); break;
    default: stage_scores_of<3>(sm, j, lane); break;
  }
}

// One forward-substitution step: every lane of a 16-lane DPP row receives
// lane Q's value (row_newbcast), i.e. T[Q][c] for the row's column c.
template <int Q>
__device__ __forceinline__ void subst_steps(float& acc, const float (&Lr)[kSub]) {
  const float tqc = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0x150 + Q, 0xf, 0xf, true));
  acc = fmaf(Lr[Q], tqc, acc);  // L[tq][Q] = 0 for Q >= tq
  if constexpr (Q + 2 < kSub) subst_steps<Q + 1>(acc, Lr);
}

// Columns 4 part .. 4 part + 3 of T = (I - L_ab)^{-1} of sub-chunk j by
// forward substitution in fp32: lane (row tq, column c) accumulates
// T[tq][c] = [tq == c] + sum_{q < tq} L[tq][q] T[q][c]; the lanes of column
// c form one DPP row, so T[q][c] is a broadcast of lane q of that row.
__device__ __forceinline__ void stage_inverse(Shared& sm, int64_t j, int lane, int part) {
  Slot& S = sm.slot[j & (kRing - 1)];
  const int tq = lane & 15, cl = lane >> 4;
  const float4* L = sm.Lf[j & 1];
  float Lr[kSub];  // row tq of L_ab
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 v4 = L[tq + 16 * g];
    Lr[4 * g] = v4.x;
    Lr[4 * g + 1] = v4.y;
    Lr[4 * g + 2] = v4.z;
    Lr[4 * g + 3] = v4.w;
  }
  float acc = (tq == 4 * part + cl) ? 1.f : 0.f;
  subst_steps<0>(acc, Lr);
  const uint16_t t16 = static_cast<uint16_t>(pack_bf16(acc, 0.f));
  // T[tq][4 part + cl] sits in lane tq + 16 part, element cl of the A operand,
  // once in each half (P = T X takes X's hi and lo halves in one product)
  uint16_t* Tm = reinterpret_cast<uint16_t*>(&S.M[0][tq + 16 * part]);
  Tm[cl] = t16;
  Tm[4 + cl] = t16;
}

// State chain of sub-chunk j for value columns [16 cb, 16 cb + 16);
// returns y of tokens 4lg .. 4lg+3 of the sub-chunk, column 16 cb + li.
// 16-token products use both halves of the 32-wide instruction for two
// terms of one sum: {mh, ml}.{v, v} = M V for an exact v, and
// {mh, ml}.{ph, ph} + {mh, ml}.{pl, 0} = mh ph + ml ph + mh pl for a split P.
__device__ __forceinline__ f32x4 stage_state(const Shared& sm, f32x4 (&h)[4], int64_t j,
                                             int lane, int cb) {
  const Slot& S = sm.slot[j & (kRing - 1)];
  const int li = lane & 15, lg = lane >> 4;
  const int col0 = kSub * cb;
  uint4 ah[2], rh[2], rl[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int off = rk_off(li, 32 * kb + 8 * lg);
    ah[kb] = ld16(&S.A[off]);
    rh[kb] = ld16(&S.R[0][off]);
    rl[kb] = ld16(&S.R[1][off]);
  }
  // Transposed 16-token operands by LDS transpose reads: this lane reads token
  // row 4 lg + li / 4 at channel 4 (li % 4) of a 16-channel block and receives
  // that block's channel li at tokens 4 lg .. 4 lg + 3.
  const int ts = 4 * lg + (li >> 2), cq = 4 * (li & 3);
  const uint2 v4 = ld_tr(&S.V[rk_off(ts, col0 + cq)]);
  const uint4 vv = make_uint4(v4.x, v4.y, v4.x, v4.y);  // {v, v}: B operand [s = 4lg..][i]
  const uint4 tm = S.M[0][lane], lak = S.M[1][lane], mrb = S.M[2][lane], mrk = S.M[3][lane];
  uint4 bt[4], kt[4];
  float4 gm[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    // A operand [j = 16jb + li][s = 4lg..4lg+3] as {hi, lo}
    const int off = rk_off(ts, key_pos(16 * jb + cq));
    const uint2 bh = ld_tr(&S.B[0][off]), bl = ld_tr(&S.B[1][off]);
    const uint2 kh = ld_tr(&S.K[0][off]), kl = ld_tr(&S.K[1][off]);
    bt[jb] = make_uint4(bh.x, bh.y, bl.x, bl.y);
    kt[jb] = make_uint4(kh.x, kh.y, kl.x, kl.y);
    gm[jb] = *reinterpret_cast<const float4*>(&S.gam[kSub - 1][16 * jb + 4 * lg]);
  }
  // the state tiles h[2kb], h[2kb+1] as the B operand of key block kb
  uint4 hbh[2], hbl[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    uint2 h0h, h0l, h1h, h1l;
    pack_split(h[2 * kb], h0h, h0l);
    pack_split(h[2 * kb + 1], h1h, h1l);
    hbh[kb] = make_uint4(h0h.x, h0h.y, h1h.x, h1h.y);
    hbl[kb] = make_uint4(h0l.x, h0l.y, h1l.x, h1l.y);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 X = mma32(lak, vv, zero);  // L_ak V
  f32x4 Z = mma32(mrk, vv, zero);  // M_rk V
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    X = mma32(ah[kb], hbl[kb], X);  // + A^ h (A^ as one bf16, h split)
    X = mma32(ah[kb], hbh[kb], X);
    Z = mma32x3(rh[kb], rl[kb], hbh[kb], hbl[kb], Z);  // + R^ h
  }
  uint2 xh, xl;
  pack_split(X, xh, xl);
  const f32x4 P = mma32(tm, make_uint4(xh.x, xh.y, xl.x, xl.y), zero);  // T xh + T xl
  uint2 ph, pl;
  pack_split(P, ph, pl);
  const uint4 pp = make_uint4(pl.x, pl.y, ph.x, ph.y);  // {pl, ph}
  const uint4 p0 = make_uint4(ph.x, ph.y, 0u, 0u);      // {ph, 0}
  Z = mma32(mrb, p0, Z);  // mh ph
  Z = mma32(mrb, pp, Z);  // + mh pl + ml ph
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    h[jb] = mma32(kt[jb], vv, h[jb]);
    h[jb] = mma32(bt[jb], p0, h[jb]);
    h[jb] = mma32(bt[jb], pp, h[jb]);
    h[jb][0] *= gm[jb].x;
    h[jb][1] *= gm[jb].y;
    h[jb][2] *= gm[jb].z;
    h[jb][3] *= gm[jb].w;
  }
  return Z;
}

// The state wave's y of sub-chunk j (tokens 4lg..4lg+3, value column
// 16 cb + li) into the staging rows, rounded as the output dtype.
template <bool kF32Out>
__device__ __forceinline__ void stage_y(Shared& sm, const f32x4& Z, int64_t j, int lane,
                                        int cb) {
  const int li = lane & 15, lg = lane >> 4;
  unsigned char* ys = sm.ys[j & 1];
  const int col = kSub * cb + li;
  if constexpr (kF32Out) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<float*>(ys + (4 * lg + r) * kYRowF + 4 * col) = Z[r];
  } else {
    const uint32_t p01 = pack_bf16(Z[0], Z[1]), p23 = pack_bf16(Z[2], Z[3]);
    *reinterpret_cast<uint16_t*>(ys + (4 * lg + 0) * kYRowB + 2 * col) = static_cast<uint16_t>(p01);
    *reinterpret_cast<uint16_t*>(ys + (4 * lg + 1) * kYRowB + 2 * col) = static_cast<uint16_t>(p01 >> 16);
    *reinterpret_cast<uint16_t*>(ys + (4 * lg + 2) * kYRowB + 2 * col) = static_cast<uint16_t>(p23);
    *reinterpret_cast<uint16_t*>(ys + (4 * lg + 3) * kYRowB + 2 * col) = static_cast<uint16_t>(p23 >> 16);
  }
}

// Score wave p stores tokens 4p..4p+3 of sub-chunk j from the staging rows:
// 16 lanes per token, whole 128-byte (bf16) or 256-byte (fp32) rows; with
// kQuarterCols only value columns [16 cb, 16 cb + 16), the ones this
// workgroup's state wave computed (four lanes per token).
template <bool kF32Out, bool kQuarterCols = false>
__device__ __forceinline__ void flush_y(const Shared& sm, void* y, int64_t j, const SeqGeom& g,
                                        int lane, int part, int cb = 0) {
  const int tt = 4 * part + (lane >> 4), c = 4 * (lane & 15);
  const int64_t tok = g.t_beg + kSub * j + tt;
  if (tok >= g.t_end) return;
  if constexpr (kQuarterCols)
    if ((c >> 4) != cb) return;
  const unsigned char* ys = sm.ys[j & 1];
  const int64_t yo = tok * g.tstride + g.hoff + c;
  if constexpr (kF32Out)
    *reinterpret_cast<float4*>(static_cast<float*>(y) + yo) =
        *reinterpret_cast<const float4*>(ys + tt * kYRowF + 4 * c);
  else
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + yo) =
        *reinterpret_cast<const uint2*>(ys + tt * kYRowB + 2 * c);
}

// Ends a pipeline tick. The scheduling fence keeps the compiler from moving
// the next tick's arithmetic above the barrier (which would make it wait for
// input loads issued only one tick earlier).
__device__ __forceinline__ void end_tick() {
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

// One tick of an operand wave: operands of sub-chunk k+3 (from `cur`, which
// is then refilled with k+5).
template <bool kScaled, class Load>
__device__ __forceinline__ void prep_tick(Shared& sm, SubIn& cur, int64_t k, const Load& load,
                                          const SeqGeom& g, int lane, int part, float scale) {
  stage_operands<false, kScaled>(sm, cur, k + 3, g, lane, part, scale);
  load(cur, k + 5);
  end_tick();
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const uint16_t* x, const SeqGeom& g,
                                                         bool empty = false) {
  const uint16_t* base = x + g.t_beg * g.tstride + g.hoff;
  // an empty range makes every load return zero (runs with k = v = 0)
  const uint32_t bytes = empty ? 0u : static_cast<uint32_t>((g.t_end - g.t_beg) * g.tstride * 2);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// Buffer-path input loads: whole 128-byte rows straight into LDS. Each input
// has one buffer resource per workgroup, based at the sequence's first token
// and sized to the sequence, so the per-tick offset is a 32-bit add and rows
// past the sequence end arrive as zeros (the padding tokens; with k = v = 0
// runs the k and v resources have an empty range). A sub-chunk is 12 loads of
// 8 tokens x 128 B (6 inputs x 2 halves), three per operand wave: lane l
// fetches token 8 half + l / 8, 16-byte chunk (l % 8) ^ (token % 8) of the
// row, so the chunks sit XOR-swizzled by the token (conflict-free reads in
// read_inputs). One request per 128-byte line instead of four 32-byte pieces.
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                               uint32_t soff, uint32_t lds_base) {
  // 16 bytes per lane into LDS at lds_base + 16 lane (M0)
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               : : "{m0}"(lds_base), "v"(voff), "s"(rs), "s"(soff) : "memory");
}

struct RowSrc {
  __amdgpu_buffer_rsrc_t rs[3];  // the input of each of this wave's loads
  uint32_t voff[3];              // this lane's byte offset of each load at sub-chunk 0
  uint32_t dst[3];               // byte offset of each load inside a staging slot
  uint32_t step;                 // bytes per sub-chunk
};

__device__ __forceinline__ RowSrc row_sources(const Inputs& in, const SeqGeom& g, int lane,
                                              int part, bool kvz) {
  RowSrc d;
  const int c = (lane & 7) ^ (lane >> 3);
  part = __builtin_amdgcn_readfirstlane(part);  // wave-uniform: the descriptors live in SGPRs
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int gi = 3 * part + i, input = gi >> 1, half = gi & 1;
    const uint16_t* p = input == 0 ? in.r : input == 1 ? in.w : input == 2 ? in.k
                      : input == 3 ? in.v : input == 4 ? in.a : in.b;
    d.rs[i] = seq_rsrc(p, g, kvz && (input == 2 || input == 3));
    d.voff[i] = 2u * (uint32_t(8 * half + (lane >> 3)) * uint32_t(g.tstride) + uint32_t(8 * c));
    d.dst[i] = uint32_t((input * kSub + 8 * half) * 128);
  }
  d.step = 2u * uint32_t(kSub) * uint32_t(g.tstride);
  return d;
}

__device__ __forceinline__ void issue_rows(Shared& sm, const RowSrc& src, int64_t j, int slot) {
  const uint32_t base = lds_addr(&sm.inb[slot][0][0][0]);
  const uint32_t soff = uint32_t(j) * src.step;
#pragma unroll
  for (int i = 0; i < 3; ++i) buf_load_lds16(src.rs[i], src.voff[i], soff, base + src.dst[i]);
}

// A tick of the row-loading operand waves ends once this wave's loads of the
// next sub-chunk have landed (only the three just issued may be in flight),
// so after the barrier every wave can read all of that sub-chunk's rows.
__device__ __forceinline__ void rows_tick_end() {
  wait_vm<3>();
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

// The row-loading operand pipeline: four fill ticks, then one tick per
// sub-chunk. Rows of sub-chunk j go to staging slot j % 3 two ticks before
// their operands are staged.
template <bool kScaled>
__device__ __forceinline__ void operand_loop_rows(Shared& sm, const Inputs& in, const SeqGeom& g,
                                                  int64_t n_sub, int lane, int part, float scale,
                                                  bool kvz) {
  SubIn d;
  const RowSrc src = row_sources(in, g, lane, part, kvz);
  issue_rows(sm, src, 0, 0);
  issue_rows(sm, src, 1, 1);
  rows_tick_end();
  read_inputs(sm, d, 0, lane, part);
  stage_operands<true, kScaled>(sm, d, 0, g, lane, part, scale);
  issue_rows(sm, src, 2, 2);
  rows_tick_end();
  read_inputs(sm, d, 1, lane, part);
  stage_operands<true, kScaled>(sm, d, 1, g, lane, part, scale);
  issue_rows(sm, src, 3, 0);
  rows_tick_end();
  read_inputs(sm, d, 2, lane, part);
  stage_operands<true, kScaled>(sm, d, 2, g, lane, part, scale);
  issue_rows(sm, src, 4, 1);
  rows_tick_end();
  // Sub-chunk k+3 is read from staging slot k % 3 and k+5 goes to slot
  // (k + 2) % 3. The loop is unrolled by three so that both slots are
  // constants in each body: the operand waves are the longest role of the
  // tick, and the slot arithmetic was scalar work on their path.
  auto tick = [&](int64_t k, auto rs, auto is) {
    read_inputs(sm, d, decltype(rs)::value, lane, part);
    stage_operands<true, kScaled>(sm, d, k + 3, g, lane, part, scale);
    issue_rows(sm, src, k + 5, decltype(is)::value);
    rows_tick_end();
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  int64_t k = 0;
  for (; k + 3 <= n_sub; k += 3) {
    tick(k, S0{}, S2{});
    tick(k + 1, S1{}, S0{});
    tick(k + 2, S2{}, S1{});
  }
  if (k < n_sub) tick(k++, S0{}, S2{});
  if (k < n_sub) tick(k++, S1{}, S0{});
  wait_vm<0>();  // no load may land in LDS after the workgroup ends
}

// The register-loading operand pipeline (64-bit input offsets): three fill
// ticks, then one tick per sub-chunk.
// Two ticks per iteration so each input buffer keeps its registers (sub-chunk
// k+3 of tick k is in p1 for even k, p0 for odd k). The loop has a single back
// edge, after the p0 refill: the compiler's memory-wait placement then knows
// that p0's loads are younger than p1's and waits for p1 alone.
template <bool kScaled, class Load>
__device__ __forceinline__ void operand_loop(Shared& sm, const Load& ld, const SeqGeom& g,
                                             int64_t n_sub, int lane, int part, float scale) {
  SubIn p0, p1;
  ld(p0, 0);
  ld(p1, 1);
  // fill ticks -3 .. -1 (stages of sub-chunks past the end, if any, work on
  // zero tokens and are never consumed)
  stage_operands<false, kScaled>(sm, p0, 0, g, lane, part, scale);
  ld(p0, 2);
  __syncthreads();
  stage_operands<false, kScaled>(sm, p1, 1, g, lane, part, scale);
  ld(p1, 3);
  __syncthreads();
  stage_operands<false, kScaled>(sm, p0, 2, g, lane, part, scale);
  ld(p0, 4);
  __syncthreads();
  int64_t k = 0;
  for (; k + 1 < n_sub; k += 2) {
    prep_tick<kScaled>(sm, p1, k, ld, g, lane, part, scale);
    prep_tick<kScaled>(sm, p0, k + 1, ld, g, lane, part, scale);
  }
  if (k < n_sub) prep_tick<kScaled>(sm, p1, k, ld, g, lane, part, scale);
}

}  // namespace

// Sixteen wavefronts in four kinds: waves 0-3 run the state chain (wave q
// owns value columns [16q, 16q+16)); waves 4-7 build operands (part p =
// wave - 4 handles key channels [16p, 16p+16)); waves 8-11 compute score
// matrix p = wave - 8; waves 12-15 solve T columns [4p, 4p+4) of the next
// sub-chunk, p = wave - 12. Each SIMD holds one wave of each kind, so the
// hardware interleaves the state chain's MFMA latencies with the other work,
// and the inverse's serial substitution chain runs beside the state chain
// instead of after it in the same wave. All kinds pass the same sequence of
// barriers: three fill ticks, then one per sub-chunk.
// Per-run options of wkv7_prefill_runs and wkv7_prefill_into (all absent for
// wkv7_prefill_varlen). Runs [0, n_primary) take their token range from
// cu_seqlens; run n_primary + i takes [ranges[2i], ranges[2i+1]). Flags select
// the initial state (slot row, zero or identity), zero k and v, and redirect y
// and the final state. With state_in set, a run that starts from a stored
// state reads it from state_in (row in_ids[run], or row `run` when in_ids is
// null) instead of its slot row.
struct Runs {
  const int32_t* flags;   // [nseq] or null
  const int32_t* cu_alt;  // [2 (nseq - n_primary)] begin/end pairs, or null
  int32_t n_primary;
  float* state_alt;       // [alt_rows, H, 64, 64]
  int64_t alt_rows;
  void* y_alt;            // like y
  const float* state_in;  // [in_rows, H, 64, 64] or null
  const int32_t* in_ids;  // [nseq] or null
  int64_t in_rows;
};

namespace {

// y = 0 for every token of a run whose state rows were rejected (as the decode
// step does for a rejected row): 16 lanes per 128-byte (bf16) or 256-byte
// (fp32) row.
template <bool kF32Out>
__device__ __forceinline__ void zero_y(void* y, const SeqGeom& g) {
  const int col = threadIdx.x & 15;
  for (int64_t t = g.t_beg + (threadIdx.x >> 4); t < g.t_end; t += kThreads / 16) {
    const int64_t o = t * g.tstride + g.hoff;
    if constexpr (kF32Out)
      reinterpret_cast<float4*>(static_cast<float*>(y) + o)[col] = make_float4(0.f, 0.f, 0.f, 0.f);
    else
      reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o)[col] = make_uint2(0u, 0u);
  }
}

}  // namespace

// Launches the quarter-head kernel (wkv7_prefill_quarter.hip): four
// workgroups per (sequence, head), each owning 16 value columns. Arguments as
// prefill_chunked_kernel's, plus the template choices.
int prefill_quarter_launch(unsigned blocks, hipStream_t stream, bool f32_out, bool buf,
                           bool scaled, float* wkv, int64_t num_rows, int H,
                           const int32_t* slot_ids, const int32_t* cu_seqlens,
                           const int32_t* seq_order, int nseq, const Inputs& in, void* y,
                           int64_t total_tokens, int zero_init, float scale, const Runs& runs);

}  // namespace wkv7
