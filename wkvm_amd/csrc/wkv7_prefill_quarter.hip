// The quarter-head prefill kernel: for launches that would leave most compute
// units idle, each (sequence, head) runs on four workgroups, each owning 16 of
// the head's 64 value columns. The per-column arithmetic is the whole-head
// kernel's (wkv7_prefill_core.h), so the results are the same bits.
#include "wkv7_prefill_core.h"

namespace wkv7 {
namespace {

// Roles of the 16 waves (wave w runs on SIMD w % 4): 0 state chain,
// 1 operands, 2 scores, 3 inverse, 4 none (passes the barriers only).
// Whole heads: waves 0-3 state (value columns 16 w), 4-7 operands, 8-11
// scores, 12-15 inverse, part = w % 4, one wave of each role per SIMD.
// Quarter heads (prefill_quarter_kernel: each of four workgroups owns value columns
// [16 q, 16 q + 16) of the head and repeats the operand, score and inverse
// work): the one state wave has SIMD 0 to itself, since its dependent chain
// sets the tick here, and the other roles share SIMDs 1-3 (instructions per
// tick: SIMD 0 state ~203; SIMD 1 operands 0, 1 + L_ak + L_ab ~365; SIMD 2
// operands 2 + M_rb + T parts 1, 2 ~320; SIMD 3 operands 3 + M_rk + T parts
// 3, 0 ~320), against ~466 for a whole head. (The state wave beside L_ab and
// T part 0 on SIMD 0 was 1.7 % slower per 512-token launch.) Packed 4 bits
// per wave.
constexpr uint64_t kQuarterRoles = 0x3324'3324'2214'1110ull;  // wave 15 .. wave 0
constexpr uint64_t kQuarterParts = 0x0200'3110'3210'3200ull;

template <bool kF32Out, bool kBuf, bool kScaled>
__global__ __launch_bounds__(kThreads) void prefill_quarter_kernel(
    float* wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ seq_order, int nseq,
    Inputs in, void* __restrict__ y, int64_t total_tokens, int zero_init, float scale, Runs runs) {
  __shared__ Shared sm;

  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; through readfirstlane the compiler knows it,
  // so the role and score-part branches are scalar branches instead of
  // exec-mask sequences over every body
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t item = int64_t(blockIdx.x >> 2);
  const int quarter = int(blockIdx.x & 3);  // this workgroup's value-column block
  const int64_t pos = item / H;
  const int64_t head = item - pos * H;
  const int64_t seq = seq_order ? int64_t(seq_order[pos]) : pos;
  if (seq < 0 || seq >= nseq) return;  // uniform: the whole block leaves
  const int fl = runs.flags ? runs.flags[seq] : 0;
  const int32_t* cu = cu_seqlens;
  int64_t ci = seq;
  if (seq >= runs.n_primary) {  // only with cu_alt (n_primary = nseq otherwise)
    cu = runs.cu_alt;
    ci = 2 * (seq - runs.n_primary);
  }
  SeqGeom g;
  g.t_end = min(max(int64_t(cu[ci + 1]), int64_t(0)), total_tokens);
  g.t_beg = min(max(int64_t(cu[ci]), int64_t(0)), g.t_end);
  g.tstride = int64_t(H) * kHead;
  g.hoff = head * kHead;
  const int64_t n_sub = (g.t_end - g.t_beg + kSub - 1) / kSub;
  void* yb = (fl & WKV7_RUN_Y_ALT) ? runs.y_alt : y;

  // State rows of this run: checked before any state access (uniform).
  const bool state_alt = fl & WKV7_RUN_STATE_ALT;
  float* out_base = state_alt ? runs.state_alt : wkv;
  const int64_t out_rows = state_alt ? runs.alt_rows : num_rows;
  const int64_t slot = slot_ids ? int64_t(slot_ids[seq]) : seq;
  const bool from_eye = fl & WKV7_RUN_INIT_IDENTITY;
  const bool from_zero = !from_eye && (zero_init || (fl & WKV7_RUN_INIT_ZERO));
  const bool from_in = !from_eye && !from_zero && runs.state_in;
  const int64_t in_row = from_in ? (runs.in_ids ? int64_t(runs.in_ids[seq]) : seq) : 0;
  const bool rows_ok = (!out_base || (slot >= 0 && slot < out_rows)) &&
                       (!from_in || (in_row >= 0 && in_row < runs.in_rows)) &&
                       (from_eye || from_zero || from_in || out_base);
  if (!rows_ok) {
    zero_y<kF32Out>(yb, g);
    return;  // uniform: the whole block leaves
  }

  // ---- state chain: value columns [16 cb, 16 cb + 16) ----
  const auto state_role = [&](int cb) {
    const int li = lane & 15, lg = lane >> 4;
    const int64_t tile = kHead * kHead;
    const float* hsrc = from_in    ? runs.state_in + (in_row * H + head) * tile
                        : out_base ? out_base + (slot * H + head) * tile
                                   : nullptr;  // not read: zero or identity start
    float* hdst = out_base ? out_base + (slot * H + head) * tile : nullptr;
    const int col0 = kSub * cb;  // this wave's value columns [col0, col0 + 16)
    // State columns of this wave as four 16x16 accumulator tiles (key blocks jb).
    f32x4 h[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int j = 16 * jb + 4 * lg + rr;
        h[jb][rr] = from_eye ? (j == col0 + li ? 1.f : 0.f)
                             : from_zero ? 0.f : hsrc[j * kHead + col0 + li];
      }
    if (n_sub > 0) {
      if constexpr (kBuf) end_tick();  // the row loads' fourth fill tick
      end_tick();  // fill ticks
      end_tick();
      end_tick();
      for (int64_t k = 0; k < n_sub; ++k) {
        const f32x4 yv = stage_state(sm, h, k, lane, cb);
        stage_y<kF32Out>(sm, yv, k, lane, cb);
        end_tick();
      }
    }
    if (hdst) {
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          hdst[(16 * jb + 4 * lg + rr) * kHead + col0 + li] = h[jb][rr];
    }
  };
  // ---- T of the next sub-chunk ----
  const auto inverse_role = [&](int part) {
    // The substitution is one serial chain of broadcast + fma steps; a raised
    // issue priority lets each step go as soon as it is ready instead of
    // queueing behind the SIMD's other waves (1.7-2.7 % faster on config 2;
    // raising the state, score or operand waves was slower).
    __builtin_amdgcn_s_setprio(2);
    if (n_sub > 0) {
      if constexpr (kBuf) end_tick();
      end_tick();
      end_tick();
      stage_inverse(sm, 0, lane, part);
      end_tick();
      for (int64_t k = 0; k < n_sub; ++k) {
        stage_inverse(sm, k + 1, lane, part);
        end_tick();
      }
    }
  };
  // ---- score matrices two sub-chunks ahead; y rows of the previous one ----
  const auto score_role = [&](int part) {
    if (n_sub > 0) {
      if constexpr (kBuf) end_tick();
      end_tick();
      stage_scores(sm, 0, lane, part);
      end_tick();
      stage_scores(sm, 1, lane, part);
      end_tick();
      for (int64_t k = 0; k < n_sub; ++k) {
        stage_scores(sm, k + 2, lane, part);
        if (k > 0) flush_y<kF32Out, true>(sm, yb, k - 1, g, lane, part, quarter);
        end_tick();
      }
      flush_y<kF32Out, true>(sm, yb, n_sub - 1, g, lane, part, quarter);
    }
  };
  // ---- operands ahead of the chain ----
  const auto operand_role = [&](int part) {
    if (n_sub == 0) return;
    if constexpr (kBuf) {
      operand_loop_rows<kScaled>(sm, in, g, n_sub, lane, part, scale, fl & WKV7_RUN_KV_ZERO);
    } else {
      const bool kvz = fl & WKV7_RUN_KV_ZERO;
      const auto ld = [&](SubIn& d, int64_t j) {
        load_sub(d, in, g, j, lane, part);
        if (kvz) {
#pragma unroll
          for (int i = 0; i < kChan / 2; ++i) d.k[i] = d.v[i] = 0u;
        }
      };
      operand_loop<kScaled>(sm, ld, g, n_sub, lane, part, scale);
    }
  };
  const int role = int((kQuarterRoles >> (4 * wave)) & 15);
  const int part = int((kQuarterParts >> (4 * wave)) & 15);
  if (role == 0)
    state_role(quarter);
  else if (role == 3)
    inverse_role(part);
  else if (role == 2)
    score_role(part);
  else if (role == 1)
    operand_role(part);
  else if (n_sub > 0)  // no work: the barriers of every tick
    for (int64_t k = 0; k < n_sub + (kBuf ? 4 : 3); ++k) end_tick();
}

}  // namespace

int prefill_quarter_launch(unsigned blocks, hipStream_t stream, bool f32_out, bool buf,
                           bool scaled, float* wkv, int64_t num_rows, int H,
                           const int32_t* slot_ids, const int32_t* cu_seqlens,
                           const int32_t* seq_order, int nseq, const Inputs& in, void* y,
                           int64_t total_tokens, int zero_init, float scale, const Runs& runs) {
  auto go = [&](auto f32, auto bufc, auto sc) {
    prefill_quarter_kernel<decltype(f32)::value, decltype(bufc)::value, decltype(sc)::value>
        <<<blocks, kThreads, 0, stream>>>(wkv, num_rows, H, slot_ids, cu_seqlens, seq_order,
                                          nseq, in, y, total_tokens, zero_init, scale, runs);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto go2 = [&](auto f32, auto bufc) {
    if (scaled) go(f32, bufc, T_{}); else go(f32, bufc, F_{});
  };
  if (f32_out) {
    if (buf) go2(T_{}, T_{}); else go2(T_{}, F_{});
  } else {
    if (buf) go2(F_{}, T_{}); else go2(F_{}, F_{});
  }
  return launch_status();
}

}  // namespace wkv7
