// Grouped projection GEMMs for few rows (RWKV-7 time-mix decode batches):
//   y_g = act_g(x_g w_g^T + bias_g),  x_g [m, k] bf16, w_g [n, k] bf16 ([out, in]).
//
// At a few hundred rows each product of the block (r, k, v, o: 2048 x 2048;
// the LoRA stages: 2048 -> 64..256 -> 2048) is a thin GEMM whose weights
// take about 1 us to stream from HBM, while a separate library launch per
// product costs 4-13 us. One launch here covers up to 8 independent products:
// the workgroups of all groups form one grid, each computing a BM x BN output
// tile over the whole k.
//
// Workgroup: 4 waves in a 2 x 2 grid, each wave a (BM/2) x (BN/2) block of
// 16 x 16 accumulator tiles on v_mfma_f32_16x16x32_bf16. Operand layout of
// that instruction (lane l, li = l % 16, lg = l / 16): A lane holds
// A[li][8lg .. 8lg+7] of a 32-wide k block, B lane holds B[8lg .. 8lg+7][li],
// the accumulator holds D[4lg .. 4lg+3][li]. With x rows and w rows both
// k-contiguous, every operand register is one 16-byte chunk of one row.
// k advances 64 per stage through a ring of S LDS stages whose 128-byte rows
// hold 8 chunks, chunk c of row r at slot c ^ (r & 7), so the 16 rows a
// fragment read touches spread over the banks. Stages are filled by direct
// global -> LDS loads (no register staging) issued S - 1 stages ahead, which
// keeps ~3 x (BM + BN) x 128 bytes in flight per workgroup: at these sizes the
// products are bound by memory latency, not by the matrix cores. One barrier
// per stage. Rows past m and columns past n load a clamped (valid) row and
// are not stored.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kProjThreads = 256;
constexpr int kChunks = 8;  // 16-byte chunks per 64-wide k stage of a row

struct ProjArgs {
  wkv7_proj_group g[WKV7_PROJ_MAX_GROUPS];
  int32_t tile_end[WKV7_PROJ_MAX_GROUPS];  // exclusive prefix sums of tiles per group
  int64_t m;
  int32_t tiles_m;
  int32_t ngroups;
};

__device__ __forceinline__ f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ int swz(int row, int chunk) { return row * kChunks + (chunk ^ (row & 7)); }

__device__ __forceinline__ float activate(float v, int act) {
  if (act == WKV7_ACT_TANH) return tanhf(v);
  if (act == WKV7_ACT_SIGMOID) return 1.f / (1.f + __expf(-v));
  return v;
}

// One stage of the LDS ring: the A rows (x) then the B rows (w) of a 64-wide
// k block, 8 swizzled 16-byte chunks per row.
template <int BM, int BN>
struct Stage {
  uint4 c[(BM + BN) * kChunks];
};

typedef __attribute__((address_space(3))) uint4 lds_uint4;

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_addr(const uint4* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_uint4*)p));
}

// Direct load: 16 bytes per lane from global memory into LDS, lane l's bytes
// at lds_base + 16 l (lds_base is wave-uniform, passed in M0; one wait state
// separates the M0 write from its use). Issued as inline assembly so that the
// compiler's wait insertion neither sees these LDS writes (it would wait for
// every pending direct load before any LDS read) nor counts them: all waits
// for them are the explicit ones of stage_barrier below.
__device__ __forceinline__ void load_lds16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_base), "v"(src)
               : "memory");
}

// Wait until at most N direct loads of this wave are pending and its LDS
// reads are done, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// stage_barrier for a run-time count of pending stages (0 .. P) of L loads.
template <int L, int P>
__device__ __forceinline__ void wait_pending(int pending) {
  if constexpr (P == 0) {
    stage_barrier<0>();
  } else {
    if (pending >= P) stage_barrier<P * L>();
    else wait_pending<L, P - 1>(pending);
  }
}

template <int BM, int BN, int S>
__global__ __launch_bounds__(kProjThreads) void proj_kernel(const ProjArgs args) {
  constexpr int WM = BM / 2, WN = BN / 2;     // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;   // accumulator tiles per wave
  // Each wave-wide direct load fills 1 KiB of a stage = 8 rows; a thread
  // issues L of them per stage.
  constexpr int kRowsPerLoad = 8;
  constexpr int L = (BM + BN) / (kRowsPerLoad * 4);
  static_assert(TM >= 1 && TN >= 1 && (BM + BN) % 32 == 0 && BM % 8 == 0, "tile shape");
  __shared__ Stage<BM, BN> ring[S];

  const int bid = blockIdx.x;
  int g = 0;
  while (g + 1 < args.ngroups && bid >= args.tile_end[g]) ++g;
  if (bid >= args.tile_end[g]) return;
  const wkv7_proj_group& G = args.g[g];
  const int local = bid - (g ? args.tile_end[g - 1] : 0);
  const int tm = local % args.tiles_m, tn = local / args.tiles_m;
  const int64_t M = args.m;
  const int N = G.n, K = G.k;
  const int64_t m0 = int64_t(tm) * BM;
  const int n0 = tn * BN;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int li = lane & 15, lg = lane >> 4;

  // Load i of this wave fills stage rows 8 j .. 8 j + 7, j = 4 i + wave; lane
  // l writes slot 8 row + q (row = 8 j + l / 8, q = l % 8), which holds
  // logical chunk q ^ (row & 7) of that row.
  const uint16_t* src[L];
  int chunk_k[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int row = kRowsPerLoad * (4 * i + wave) + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);
    chunk_k[i] = 8 * c;
    if (row < BM) {
      const int64_t m = min(m0 + row, M - 1);
      src[i] = G.x + m * G.ldx + 8 * c;
    } else {
      const int64_t n = min(int64_t(n0 + row - BM), int64_t(N - 1));
      src[i] = G.w + n * G.ldw + 8 * c;
    }
  }
  // Issue stage kt's loads into `st`. Chunks past k (the 32-wide tail of the
  // last stage) re-read a valid chunk; the tail stage never multiplies them.
  const int nk = (K + 63) / 64;
  auto issue = [&](int kt, Stage<BM, BN>& st) {
    const int k0 = kt * 64;
    const bool tail = k0 + 64 > K;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const int off = (tail && k0 + chunk_k[i] >= K) ? K - 8 - chunk_k[i] : k0;
      load_lds16(src[i] + off,
                 __builtin_amdgcn_readfirstlane(lds_addr(&st.c[64 * (4 * i + wave)])));
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Stage<BM, BN>& st, int steps) {
    for (int s = 0; s < steps; ++s) {
      uint4 af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a) af[a] = st.c[swz(wm * WM + a * 16 + li, 4 * s + lg)];
#pragma unroll
      for (int b = 0; b < TN; ++b) bf[b] = st.c[swz(BM + wn * WN + b * 16 + li, 4 * s + lg)];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = mma(af[a], bf[b], acc[a][b]);
    }
  };

  // Stages 0 .. S-2 in flight before the loop. In iteration kt the wave waits
  // until only the loads of stages kt+1 .. min(kt+S-2, nk-1) are pending, one
  // barrier publishes stage kt to every wave and retires slot (kt-1) % S,
  // whose reads all finished before it; that slot then receives stage
  // kt + S - 1.
  static_assert(S >= 2 && S <= 8, "wait ladder covers rings of 2..8 stages");
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < nk) issue(p, ring[p]);
  for (int kt = 0; kt < nk; ++kt) {
    wait_pending<L, S - 2>(min(S - 2, nk - 1 - kt));
    compute(ring[kt % S], min(2, (K - kt * 64) / 32));
    if (kt + S - 1 < nk) issue(kt + S - 1, ring[(kt + S - 1) % S]);
  }

  const int act = G.act;
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int col = n0 + wn * WN + b * 16 + li;
    if (col >= N) continue;
    const float bias = G.bias ? bf16_to_f32(G.bias[col]) : 0.f;
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + wm * WM + a * 16 + 4 * lg + e;
        if (row < M) G.y[row * G.ldy + col] = f32_to_bf16(activate(acc[a][b][e] + bias, act));
      }
    }
  }
}

struct TileShape {
  int bm, bn;
};

// Tile shapes, largest first (fewest re-reads of x and w).
constexpr TileShape kShapes[] = {{128, 64}, {64, 64}, {64, 32}};

int64_t count_tiles(int64_t m, const wkv7_proj_group* gs, int ng, TileShape sh) {
  int64_t tiles = 0;
  const int64_t tm = (m + sh.bm - 1) / sh.bm;
  for (int i = 0; i < ng; ++i) tiles += tm * ((gs[i].n + sh.bn - 1) / sh.bn);
  return tiles;
}

template <int BM, int BN, int S>
int launch(int64_t m, const wkv7_proj_group* gs, int ng, hipStream_t s) {
  ProjArgs args{};
  args.m = m;
  args.ngroups = ng;
  const int64_t tiles_m = (m + BM - 1) / BM;
  int64_t end = 0;
  for (int i = 0; i < ng; ++i) {
    args.g[i] = gs[i];
    end += tiles_m * ((gs[i].n + BN - 1) / BN);
    if (end > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
    args.tile_end[i] = int32_t(end);
  }
  args.tiles_m = int32_t(tiles_m);
  proj_kernel<BM, BN, S><<<unsigned(end), kProjThreads, 0, s>>>(args);
  return launch_status();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_proj_grouped(int64_t m, const wkv7_proj_group* groups, int32_t ngroups,
                                 void* stream) {
  if (m < 0 || !groups || ngroups < 1 || ngroups > WKV7_PROJ_MAX_GROUPS) return WKV7_ERR_ARG;
  if (m > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
  for (int i = 0; i < ngroups; ++i) {
    const wkv7_proj_group& g = groups[i];
    if (!g.x || !g.w || !g.y || g.n < 1 || g.k < 32 || g.k % 32 != 0) return WKV7_ERR_ARG;
    if (g.act != WKV7_ACT_NONE && g.act != WKV7_ACT_TANH && g.act != WKV7_ACT_SIGMOID)
      return WKV7_ERR_ARG;
    if (g.ldx < g.k || g.ldw < g.k || g.ldy < g.n) return WKV7_ERR_SHAPE;
    if (g.ldx % 8 || g.ldw % 8 || !aligned16(g.x) || !aligned16(g.w)) return WKV7_ERR_SHAPE;
  }
  if (m == 0) return WKV7_OK;
  int cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return launch_status();
  // The largest tile that still gives most compute units a workgroup; with
  // short k (LoRA up-projections: a few stages per workgroup) aim for two
  // workgroups per unit.
  int kmax = 0;
  for (int i = 0; i < ngroups; ++i) kmax = max(kmax, groups[i].k);
  const int64_t target = kmax <= 256 ? 2 * int64_t(cus) : int64_t(cus) * 4 / 5;
  int pick = 2;
  for (int i = 0; i < 3; ++i)
    if (count_tiles(m, groups, ngroups, kShapes[i]) >= target) {
      pick = i;
      break;
    }
  hipStream_t s = as_stream(stream);
  switch (pick) {
    case 0: return launch<128, 64, 4>(m, groups, ngroups, s);
    case 1: return launch<64, 64, 4>(m, groups, ngroups, s);
    default: return launch<64, 32, 4>(m, groups, ngroups, s);
  }
}
