// Varlen WKV7 prefill over slot states: the whole-head kernel (one workgroup
// of 16 waves per (sequence, head)) and the C entry points. The algorithm,
// schedule and layouts are described in wkv7_prefill_core.h.
#include <atomic>

#include "wkv7_prefill_core.h"

namespace wkv7 {
namespace {

// wkv (with slot_ids) is where the final states go, and the initial states
// come from unless runs.state_in, zero_init or a run flag says otherwise; a
// null wkv writes no final state (slot_ids may then be null too: run s is
// row s).
template <bool kF32Out, bool kBuf, bool kScaled>
__global__ __launch_bounds__(kThreads) void prefill_chunked_kernel(
    float* wkv, int64_t num_rows, int H, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ seq_order, int nseq,
    Inputs in, void* __restrict__ y, int64_t total_tokens, int zero_init, float scale, Runs runs) {
  __shared__ Shared sm;

  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; through readfirstlane the compiler knows it,
  // so the role and score-part branches are scalar branches instead of
  // exec-mask sequences over every body
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t pos = blockIdx.x / H;
  const int64_t head = blockIdx.x - pos * H;
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

  if (wave < 4) {
    // ---- state chain ----
    const int li = lane & 15, lg = lane >> 4;
    const int64_t tile = kHead * kHead;
    const float* hsrc = from_in    ? runs.state_in + (in_row * H + head) * tile
                        : out_base ? out_base + (slot * H + head) * tile
                                   : nullptr;  // not read: zero or identity start
    float* hdst = out_base ? out_base + (slot * H + head) * tile : nullptr;
    const int col0 = kSub * wave;  // this wave's value columns [col0, col0 + 16)
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
        const f32x4 yv = stage_state(sm, h, k, lane, wave);
        stage_y<kF32Out>(sm, yv, k, lane, wave);
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
  } else if (wave >= 8 + kOpWaves) {
    // ---- T of the next sub-chunk ----
    // The substitution is one serial chain of 14 broadcast + fma steps; a
    // raised issue priority lets each step go as soon as it is ready instead
    // of queueing behind the SIMD's three other waves (1.7-2.7 % faster on
    // config 2; raising the state, score or operand waves was slower).
    __builtin_amdgcn_s_setprio(2);
    if (n_sub > 0) {
      const int part = wave - 8 - kOpWaves;
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
  } else if (wave >= 4 + kOpWaves) {
    if (n_sub > 0) {
      const int part = wave - 4 - kOpWaves;
      if constexpr (kBuf) end_tick();
      end_tick();
      stage_scores(sm, 0, lane, part);
      end_tick();
      stage_scores(sm, 1, lane, part);
      end_tick();
      for (int64_t k = 0; k < n_sub; ++k) {
        stage_scores(sm, k + 2, lane, part);
        if (k > 0) flush_y<kF32Out>(sm, yb, k - 1, g, lane, part);
        end_tick();
      }
      flush_y<kF32Out>(sm, yb, n_sub - 1, g, lane, part);
    }
  } else if (n_sub > 0) {
    // ---- operands ahead of the chain ----
    const int part = wave - 4;
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
  }
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

namespace {
// Compute units of the current device (cached per device; 256 on MI355X; 0
// when the runtime cannot say, which keeps one workgroup per (sequence, head)).
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int prefill_launch(float* wkv_layer, int64_t num_rows, int32_t H, const int32_t* slot_ids,
                   const int32_t* cu_seqlens, const int32_t* seq_order, int32_t nseq,
                   int64_t total_tokens, const Inputs& in, void* y, int32_t y_dtype,
                   int32_t zero_init, float scale, const Runs& runs, void* stream) {
  const int64_t items = int64_t(nseq) * H;
  // A launch that would leave at least three quarters of the compute units
  // idle splits each (sequence, head) over four workgroups by value columns
  // (same arithmetic per column, so the same bits; see kQuarterRoles).
  const bool quarter = 4 * items <= int64_t(device_cus());
  const int64_t blocks = quarter ? 4 * items : items;
  if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  hipStream_t s = as_stream(stream);
  // Buffer-resource input loads need every byte offset of a sequence (plus the
  // look-ahead past its end) to fit 31 bits.
  const bool buf = (total_tokens + 6 * kSub) * int64_t(H) * kHead * 2 < (int64_t(1) << 31);
  auto launch3 = [&](auto f32, auto bufc, auto sc) {
    if (quarter)
      prefill_quarter_launch(unsigned(blocks), s, decltype(f32)::value, decltype(bufc)::value,
                             decltype(sc)::value, wkv_layer, num_rows, H, slot_ids, cu_seqlens,
                             seq_order, nseq, in, y, total_tokens, zero_init, scale, runs);
    else
      prefill_chunked_kernel<decltype(f32)::value, decltype(bufc)::value, decltype(sc)::value>
          <<<unsigned(blocks), kThreads, 0, s>>>(wkv_layer, num_rows, H, slot_ids, cu_seqlens,
                                                 seq_order, nseq, in, y, total_tokens, zero_init,
                                                 scale, runs);
  };
  auto launch = [&](auto f32, auto bufc) {
    if (scale != 1.0f)
      launch3(f32, bufc, std::true_type{});
    else
      launch3(f32, bufc, std::false_type{});
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (y_dtype == WKV7_Y_F32) {
    if (buf) launch(T_{}, T_{}); else launch(T_{}, F_{});
  } else {
    if (buf) launch(F_{}, T_{}); else launch(F_{}, F_{});
  }
  return launch_status();
}

// y rows are stored as 8-byte (bf16) or 16-byte (fp32) vectors
bool y_aligned(const void* y, int32_t y_dtype) {
  return (reinterpret_cast<uintptr_t>(y) & (y_dtype == WKV7_Y_F32 ? 15u : 7u)) == 0;
}

bool inputs_aligned(const uint16_t* r, const uint16_t* w, const uint16_t* k, const uint16_t* v,
                    const uint16_t* a, const uint16_t* b) {
  // inputs are read as 16-byte vectors
  const uintptr_t align = reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(w) |
                          reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                          reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
  return (align & 15u) == 0;
}
}  // namespace

extern "C" int wkv7_prefill_varlen(float* wkv_layer, int64_t num_rows, int32_t H,
                                   const int32_t* slot_ids, const int32_t* cu_seqlens,
                                   const int32_t* seq_order, int32_t nseq, int64_t total_tokens,
                                   const uint16_t* r,
                                   const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                   const uint16_t* a, const uint16_t* b, void* y, int32_t y_dtype,
                                   int32_t zero_init, float scale, void* stream) {
  if (nseq < 0 || H < 1 || num_rows < 1 || total_tokens < 0) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (nseq == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || !cu_seqlens) return WKV7_ERR_ARG;
  if (total_tokens > 0 && (!r || !w || !k || !v || !a || !b || !y)) return WKV7_ERR_ARG;
  if (!inputs_aligned(r, w, k, v, a, b) || !y_aligned(y, y_dtype)) return WKV7_ERR_SHAPE;
  const Runs runs{nullptr, nullptr, nseq, nullptr, 0, nullptr, nullptr, nullptr, 0};
  return prefill_launch(wkv_layer, num_rows, H, slot_ids, cu_seqlens, seq_order, nseq,
                        total_tokens, Inputs{r, w, k, v, a, b}, y, y_dtype, zero_init, scale,
                        runs, stream);
}

extern "C" int wkv7_prefill_runs(float* wkv_layer, int64_t num_rows, int32_t H,
                                 const int32_t* slot_ids, const int32_t* cu_seqlens,
                                 const int32_t* seq_order, int32_t nseq, int64_t total_tokens,
                                 const uint16_t* r, const uint16_t* w, const uint16_t* k,
                                 const uint16_t* v, const uint16_t* a, const uint16_t* b, void* y,
                                 int32_t y_dtype, int32_t zero_init, float scale,
                                 const int32_t* run_flags, const int32_t* cu_alt,
                                 int32_t n_primary, float* state_alt, int64_t alt_rows,
                                 void* y_alt, const float* state_in, int64_t in_rows,
                                 const int32_t* in_ids, void* stream) {
  if (nseq < 0 || H < 1 || num_rows < 1 || total_tokens < 0 || alt_rows < 0) return WKV7_ERR_ARG;
  if (in_rows < 0 || (state_in && in_rows < 1) || (in_ids && !state_in)) return WKV7_ERR_ARG;
  if (state_in && !in_ids && in_rows < nseq) return WKV7_ERR_SHAPE;
  if (n_primary < 0 || n_primary > nseq) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if (nseq == 0) return WKV7_OK;
  if (!wkv_layer || !slot_ids || (n_primary > 0 && !cu_seqlens)) return WKV7_ERR_ARG;
  if (n_primary < nseq && !cu_alt) return WKV7_ERR_ARG;
  if (alt_rows > 0 && !state_alt) return WKV7_ERR_ARG;
  if (total_tokens > 0 && (!r || !w || !k || !v || !a || !b || !y)) return WKV7_ERR_ARG;
  if (!inputs_aligned(r, w, k, v, a, b) || !y_aligned(y, y_dtype) ||
      (y_alt && !y_aligned(y_alt, y_dtype)))
    return WKV7_ERR_SHAPE;
  const Runs runs{run_flags, cu_alt,   n_primary, state_alt, alt_rows,
                  y_alt ? y_alt : y, state_in, in_ids,    in_rows};
  return prefill_launch(wkv_layer, num_rows, H, slot_ids, cu_seqlens, seq_order, nseq,
                        total_tokens, Inputs{r, w, k, v, a, b}, y, y_dtype, zero_init, scale,
                        runs, stream);
}

extern "C" int wkv7_prefill_into(const float* state_in, int64_t in_rows, const int32_t* in_ids,
                                 float* state_out, int64_t out_rows, const int32_t* out_ids,
                                 int32_t H, const int32_t* cu_seqlens, const int32_t* seq_order,
                                 int32_t nseq, int64_t total_tokens, const uint16_t* r,
                                 const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* a, const uint16_t* b, void* y, int32_t y_dtype,
                                 float scale, void* stream) {
  if (nseq < 0 || H < 1 || total_tokens < 0 || in_rows < 0 || out_rows < 0) return WKV7_ERR_ARG;
  if (y_dtype != WKV7_Y_BF16 && y_dtype != WKV7_Y_F32) return WKV7_ERR_ARG;
  if ((in_ids && !state_in) || (out_ids && !state_out)) return WKV7_ERR_ARG;
  if (nseq == 0) return WKV7_OK;
  if (!cu_seqlens) return WKV7_ERR_ARG;
  if (total_tokens > 0 && (!r || !w || !k || !v || !a || !b || !y)) return WKV7_ERR_ARG;
  if ((state_in && !in_ids && in_rows < nseq) || (state_out && !out_ids && out_rows < nseq))
    return WKV7_ERR_SHAPE;
  if (!inputs_aligned(r, w, k, v, a, b) || !y_aligned(y, y_dtype)) return WKV7_ERR_SHAPE;
  // no state_in: zero initial state; no state_out: no final state written
  const Runs runs{nullptr, nullptr, nseq, nullptr, 0, nullptr, state_in, in_ids, in_rows};
  return prefill_launch(state_out, state_out ? out_rows : 0, H, out_ids, cu_seqlens, seq_order,
                        nseq, total_tokens, Inputs{r, w, k, v, a, b}, y, y_dtype,
                        state_in ? 0 : 1, scale, runs, stream);
}
