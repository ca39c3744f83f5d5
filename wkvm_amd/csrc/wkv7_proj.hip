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
// Workgroup: GM x GN waves (4 or 8), each a (BM/GM) x (BN/GN) block of
// 16 x 16 accumulator tiles on v_mfma_f32_16x16x32_bf16. Operand layout of
// that instruction (lane l, li = l % 16, lg = l / 16): A lane holds
// A[li][8lg .. 8lg+7] of a 32-wide k block, B lane holds B[8lg .. 8lg+7][li],
// the accumulator holds D[4lg .. 4lg+3][li]. With x rows and w rows both
// k-contiguous, every operand register is one 16-byte chunk of one row.
// k advances BK (64 or 128) per stage through a ring of S LDS stages whose
// rows hold KC = BK / 8 chunks of 16 bytes, chunk c of row r at slot
// c ^ (r & (KC - 1)), so the 16 rows a fragment read touches spread over the
// banks. Stages are filled by direct global -> LDS loads (no register
// staging) issued S - 1 stages ahead and spread between the MFMAs of the
// stage being multiplied. One barrier per stage. Rows past m and columns past
// n load a clamped (valid) row and are not stored. Tiles are dealt to the
// XCDs in contiguous runs so that each XCD's L2 keeps the x rows it
// re-reads. With few tiles and long k, k can be split over several
// workgroups per tile (fp32 partials in a caller-provided workspace, summed
// in part order by proj_reduce_kernel).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "wkv7_common.h"

namespace wkv7 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));


constexpr int kXcds = 8;  // MI355X: workgroups are dealt round-robin over 8 XCDs

struct ProjArgs {
  wkv7_proj_group g[WKV7_PROJ_MAX_GROUPS];
  int32_t tile_end[WKV7_PROJ_MAX_GROUPS];  // exclusive prefix sums of work items per group
  int64_t ws_off[WKV7_PROJ_MAX_GROUPS];    // split k: group's partials, [parts][m][n] fp32
  int64_t elem_end[WKV7_PROJ_MAX_GROUPS];  // split k: prefix sums of m * n
  float* ws;
  int64_t m;
  int32_t tiles_m;
  int32_t ngroups;
  int32_t xcd_span;  // work items per XCD: ceil(items / kXcds)
  int32_t parts;     // k parts per output tile (1: the tile's workgroup covers all of k)
};

__device__ __forceinline__ f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int KC>
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * KC + (chunk ^ (row & (KC - 1)));
}

__device__ __forceinline__ float activate(float v, int act) {
  if (act == WKV7_ACT_TANH) return tanhf(v);
  if (act == WKV7_ACT_SIGMOID) return 1.f / (1.f + __expf(-v));
  return v;
}

// One stage of the LDS ring: the A rows (x) then the B rows (w) of a
// (8 KC)-wide k block, KC swizzled 16-byte chunks per row.
template <int BM, int BN, int KC>
struct Stage {
  uint4 c[(BM + BN) * KC];
};

typedef __attribute__((address_space(3))) uint4 lds_uint4;

// LDS byte address of a __shared__ location.
__device__ __forceinline__ uint32_t lds_addr(const uint4* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_uint4*)p));
}

// Direct load: 16 bytes per lane from global memory into LDS, lane l's bytes
// at lds_base + 16 l (lds_base is wave-uniform and bound to M0 as an input
// operand, so the compiler writes M0 itself and knows its value; one wait
// state separates that write from its use). Issued as inline assembly so that the
// compiler's wait insertion neither sees these LDS writes (it would wait for
// every pending direct load before any LDS read) nor counts them: all waits
// for them are the explicit ones of stage_barrier below.
__device__ __forceinline__ void load_lds16(const void* src, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "{m0}"(lds_base), "v"(src)
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

template <int BM, int BN, int S, int GM, int GN, int BK, bool kSplit>
__global__ __launch_bounds__(64 * GM * GN) void proj_kernel(const ProjArgs args) {
  constexpr int NW = GM * GN;                 // waves, a GM x GN grid
  constexpr int WM = BM / GM, WN = BN / GN;   // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;   // accumulator tiles per wave
  // k per stage BK = 64 or 128: KC chunks of 16 bytes per row. Each
  // wave-wide direct load fills 1 KiB of a stage = 64 / KC rows; a thread
  // issues L of them per stage.
  constexpr int KC = BK / 8, kStepsFull = BK / 32;
  static_assert(BK == 64 || BK == 128, "stage depth");
  constexpr int kRowsPerLoad = 64 / KC;
  constexpr int L = (BM + BN) / (kRowsPerLoad * NW);
  static_assert(TM >= 1 && TN >= 1 && (BM + BN) % (kRowsPerLoad * NW) == 0 && BM % 8 == 0,
                "tile shape");
  __shared__ Stage<BM, BN, KC> ring[S];

  // Workgroup b runs on XCD b % 8; XCD x takes the x-th contiguous run of
  // tiles (ordered by group, then output columns, then rows), so each XCD's
  // L2 holds the x rows of one or two groups instead of all of them.
  const int bid = int(blockIdx.x % kXcds) * args.xcd_span + int(blockIdx.x / kXcds);
  int g = 0;
  while (g + 1 < args.ngroups && bid >= args.tile_end[g]) ++g;
  if (bid >= args.tile_end[g]) return;
  const wkv7_proj_group& G = args.g[g];
  const int item = bid - (g ? args.tile_end[g - 1] : 0);
  const int part = kSplit ? item % args.parts : 0;
  const int local = kSplit ? item / args.parts : item;
  const int tm = local % args.tiles_m, tn = local / args.tiles_m;
  const int64_t M = args.m;
  const int N = G.n, K = G.k;
  const int64_t m0 = int64_t(tm) * BM;
  const int n0 = tn * BN;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave % GM, wn = wave / GM;
  const int li = lane & 15, lg = lane >> 4;
  // LDS destinations are wave-uniform: computed in scalar registers.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t ring_base = lds_addr(&ring[0].c[0]) + 1024u * wave_s;
  constexpr uint32_t kStageBytes = sizeof(Stage<BM, BN, KC>);

  // Load i of this wave fills stage rows R j .. R j + R - 1 (R = 64 / KC,
  // j = NW i + wave); lane l writes slot KC row + q (row = R j + l / KC,
  // q = l % KC), which holds logical chunk q ^ (row & (KC - 1)) of that row.
  const uint16_t* src[L];
  int chunk_k[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int row = kRowsPerLoad * (NW * i + wave) + lane / KC;
    const int c = (lane % KC) ^ (row & (KC - 1));
    chunk_k[i] = 8 * c;
    if (row < BM) {
      const int64_t m = min(m0 + row, M - 1);
      src[i] = G.x + m * G.ldx + 8 * c;
    } else {
      const int64_t n = min(int64_t(n0 + row - BM), int64_t(N - 1));
      src[i] = G.w + n * G.ldw + 8 * c;
    }
  }
  // Issue stage kt's loads into ring slot `slot`. In a partial tail stage
  // (k % BK != 0) chunks past k re-read a valid chunk; nothing multiplies
  // them.
  // This workgroup's k stages: [kb, kb + nk) of the product's nk_all, all
  // of them unless k is split over `parts` workgroups.
  const int nk_all = (K + BK - 1) / BK;
  const int spp = kSplit ? (nk_all + args.parts - 1) / args.parts : nk_all;
  const int kb = kSplit ? min(part * spp, nk_all) : 0;
  const int nk = kSplit ? min(nk_all, kb + spp) - kb : nk_all;
  const bool has_tail = (K % BK) && kb + nk == nk_all;  // the partial stage is ours
  auto issue = [&](int kt, int slot) {
    const int k0 = (kb + kt) * BK;
    const uint32_t base = ring_base + kStageBytes * slot;
    if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < L; ++i) load_lds16(src[i] + k0, base + 1024u * NW * i);
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i)
        load_lds16(src[i] + (k0 + chunk_k[i] >= K ? K - 8 - chunk_k[i] : k0),
                   base + 1024u * NW * i);
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A stage: all fragment reads first, then its MFMAs with the next stage's
  // loads (when kIssue) spread between them, so the matrix core works while
  // a load waits for the load pipe. Inline-assembly loads are scheduling
  // boundaries, which keeps that placement.
  auto stage = [&](int kt, auto steps_c, auto issue_c) {
    constexpr int kSteps = decltype(steps_c)::value;
    constexpr bool kIssue = decltype(issue_c)::value;
    constexpr int kMfma = kSteps * TM * TN;
    const Stage<BM, BN, KC>& st = ring[kt % S];
    // (kt counts this workgroup's stages; k offsets add kb)
    uint4 af[kSteps][TM], bf[kSteps][TN];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
#pragma unroll
      for (int a = 0; a < TM; ++a) af[s][a] = st.c[swz<KC>(wm * WM + a * 16 + li, 4 * s + lg)];
#pragma unroll
      for (int b = 0; b < TN; ++b)
        bf[s][b] = st.c[swz<KC>(BM + wn * WN + b * 16 + li, 4 * s + lg)];
    }
    const int k1 = (kb + kt + S - 1) * BK;
    const uint32_t base = ring_base + kStageBytes * ((kt + S - 1) % S);
    int issued = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
          acc[a][b] = mma(af[s][a], bf[s][b], acc[a][b]);
          if constexpr (kIssue) {
            // load i goes after MFMA number ((i + 1) * kMfma) / (L + 1)
            const int m = (s * TM + a) * TN + b + 1;
#pragma unroll
            for (int i = 0; i < L; ++i)
              if (m == ((i + 1) * kMfma) / (L + 1) && issued == i) {
                load_lds16(src[i] + k1, base + 1024u * NW * i);
                ++issued;
              }
          }
        }
    if constexpr (kIssue) {
#pragma unroll
      for (int i = 0; i < L; ++i)
        if (issued == i) {
          load_lds16(src[i] + k1, base + 1024u * NW * i);
          ++issued;
        }
    }
  };

  // Stages 0 .. S-2 in flight before the loop. In iteration kt the wave waits
  // until only the loads of stages kt+1 .. min(kt+S-2, nk-1) are pending and
  // its LDS reads are done; one barrier publishes stage kt to every wave and
  // retires slot (kt-1) % S, which receives stage kt + S - 1 while stage kt
  // is multiplied. Only the last stage can be partial (32, 64 or 96 wide),
  // and nothing is issued after it.
  static_assert(S >= 2 && S <= 8, "wait ladder covers rings of 2..8 stages");
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < nk) issue(p, p);
  for (int kt = 0; kt < nk; ++kt) {
    wait_pending<L, S - 2>(min(S - 2, nk - 1 - kt));
    if (kt + S - 1 < nk) {
      if (kt + S - 1 == nk - 1 && has_tail) {
        issue(kt + S - 1, (kt + S - 1) % S);  // the tail stage's clamped loads
        stage(kt, std::integral_constant<int, kStepsFull>{}, std::false_type{});
      } else {
        stage(kt, std::integral_constant<int, kStepsFull>{}, std::true_type{});
      }
    } else if ((kb + kt) * BK + BK <= K) {
      stage(kt, std::integral_constant<int, kStepsFull>{}, std::false_type{});
    } else {
      const int steps = (K - (kb + kt) * BK) / 32;  // 1 .. kStepsFull - 1
      if (steps == 1) {
        stage(kt, std::integral_constant<int, 1>{}, std::false_type{});
      } else if constexpr (kStepsFull > 2) {
        if (steps == 2)
          stage(kt, std::integral_constant<int, 2>{}, std::false_type{});
        else
          stage(kt, std::integral_constant<int, 3>{}, std::false_type{});
      }
    }
  }

  if constexpr (kSplit) {  // fp32 partial tile; proj_reduce_kernel finishes the sum
    float* wsp = args.ws + args.ws_off[g] + int64_t(part) * M * N;
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int col = n0 + wn * WN + b * 16 + li;
      if (col >= N) continue;
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t row = m0 + wm * WM + a * 16 + 4 * lg + e;
          if (row < M) wsp[row * N + col] = acc[a][b][e];
        }
    }
    return;
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

// Split k: y = act(sum of the k parts' partials, in part order, + bias), one
// thread per output element.
__global__ __launch_bounds__(256) void proj_reduce_kernel(const ProjArgs args) {
  const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
  int g = 0;
  while (g + 1 < args.ngroups && e >= args.elem_end[g]) ++g;
  if (e >= args.elem_end[g]) return;
  const wkv7_proj_group& G = args.g[g];
  const int64_t local = e - (g ? args.elem_end[g - 1] : 0);
  const int64_t row = local / G.n;
  const int col = int(local - row * G.n);
  const int64_t plane = args.m * G.n;
  const float* src = args.ws + args.ws_off[g] + local;
  float sum = 0.f;
  for (int p = 0; p < args.parts; ++p) sum += src[p * plane];
  const float bias = G.bias ? bf16_to_f32(G.bias[col]) : 0.f;
  G.y[row * G.ldy + col] = f32_to_bf16(activate(sum + bias, G.act));
}

struct TileShape {
  int bm, bn;
};

// Tile shapes (fewer re-reads of x and w per output the larger the tile);
// measured on the MI355X inside HIP graphs.
constexpr TileShape kShapes[] = {{64, 64}, {32, 32}, {128, 64}, {64, 32}};

int64_t count_tiles(int64_t m, const wkv7_proj_group* gs, int ng, TileShape sh) {
  int64_t tiles = 0;
  const int64_t tm = (m + sh.bm - 1) / sh.bm;
  for (int i = 0; i < ng; ++i) tiles += tm * ((gs[i].n + sh.bn - 1) / sh.bn);
  return tiles;
}

template <int BM, int BN, int S, int GM = 2, int GN = 2, int BK = 64>
int launch(int64_t m, const wkv7_proj_group* gs, int ng, int parts, float* ws, hipStream_t s) {
  ProjArgs args{};
  args.m = m;
  args.ngroups = ng;
  args.parts = parts;
  args.ws = ws;
  const int64_t tiles_m = (m + BM - 1) / BM;
  int64_t end = 0, elems = 0;
  for (int i = 0; i < ng; ++i) {
    args.g[i] = gs[i];
    end += tiles_m * ((gs[i].n + BN - 1) / BN) * parts;
    if (end > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
    args.tile_end[i] = int32_t(end);
    args.ws_off[i] = elems * parts;
    elems += m * gs[i].n;
    args.elem_end[i] = elems;
  }
  args.tiles_m = int32_t(tiles_m);
  args.xcd_span = int32_t((end + kXcds - 1) / kXcds);
  const unsigned grid = unsigned(args.xcd_span) * kXcds;
  if (parts == 1) {
    proj_kernel<BM, BN, S, GM, GN, BK, false><<<grid, 64 * GM * GN, 0, s>>>(args);
  } else {
    proj_kernel<BM, BN, S, GM, GN, BK, true><<<grid, 64 * GM * GN, 0, s>>>(args);
    const int rc = launch_status();
    if (rc != WKV7_OK) return rc;
    const int64_t blocks = (elems + 255) / 256;
    if (blocks > int64_t(0x7fffffff)) return WKV7_ERR_ARG;
    proj_reduce_kernel<<<unsigned(blocks), 256, 0, s>>>(args);
  }
  return launch_status();
}

// Tile shape and k split for a launch (the same decision for the workspace
// query and the launch).
struct Plan {
  int shape;  // index into kShapes
  int parts;  // k parts per tile
  size_t ws_bytes;
};

Plan make_plan(int64_t m, const wkv7_proj_group* gs, int ng, int cus) {
  int kmin = gs[0].k;
  int64_t cols = 0;
  for (int i = 0; i < ng; ++i) {
    kmin = std::min(kmin, gs[i].k);
    cols += gs[i].n;
  }
  // The launch reads (BM + BN) rows of k per tile from L2, which bounds it
  // at a few hundred rows. With long k (8 stages or more), the largest tile
  // of one workgroup per compute unit that fills three quarters of the units
  // or more in one round: 128 x 64 (8 waves, 3-stage ring of 128-wide k
  // stages, 144 KiB of LDS), then 64 x 32 (4 waves, 4-stage ring, 96 KiB).
  // A unit then reads 192 or 96 rows instead of twice 128 or 64 (the 1.5B
  // first stage at 256 rows: 20.1 against 22.7 us; o_proj 10.6 against 11.3).
  // Else 64 x 64 tiles (8 waves, 2-stage ring) when they give every unit
  // about 1.5 workgroups or more; else 32 x 32 tiles (4 waves, 4-stage ring).
  Plan p{1, 1, 0};
  int64_t tiles = count_tiles(m, gs, ng, kShapes[1]);
  auto fills = [&](int64_t t) { return t * 4 >= int64_t(cus) * 3 && t <= int64_t(cus); };
  const int64_t t128 = count_tiles(m, gs, ng, kShapes[2]);
  const int64_t t6432 = count_tiles(m, gs, ng, kShapes[3]);
  if (kmin >= 1024 && fills(t128)) {
    p.shape = 2;
    tiles = t128;
  } else if (kmin >= 1024 && fills(t6432)) {
    p.shape = 3;
    tiles = t6432;
  } else if (count_tiles(m, gs, ng, kShapes[0]) * 2 >= int64_t(cus) * 3) {
    p.shape = 0;
    tiles = count_tiles(m, gs, ng, kShapes[0]);
  }
  // At most one workgroup per two units and long k: split k so that about two
  // workgroups per unit each walk at least 8 stages. (With more tiles the
  // partials' extra traffic and second launch cost more than they save.)
  const int nk = (kmin + 63) / 64;
  if (tiles * 2 <= int64_t(cus) && nk >= 16) {
    int64_t parts = (2 * int64_t(cus) + tiles / 2) / tiles;
    parts = std::min<int64_t>(parts, std::min(8, nk / 8));
    if (parts >= 2) {
      p.parts = int(parts);
      p.ws_bytes = size_t(parts) * size_t(m) * size_t(cols) * sizeof(float);
    }
  }
  return p;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wkv7

using namespace wkv7;

namespace wkv7 {
namespace {

int validate(int64_t m, const wkv7_proj_group* groups, int32_t ngroups) {
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
  return WKV7_OK;
}

int device_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return launch_status();
  return WKV7_OK;
}

}  // namespace
}  // namespace wkv7

namespace wkv7 {
namespace {

// Split-k partials of wkv7_proj_grouped_noalloc: a library-owned device array,
// one per GPU (each device holds its own copy until the process ends). Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in symbol); it passes the device address hipGetSymbolAddress returns
// for the current device, looked up once per device and kept below.
static __device__ __align__(256) float scratch[WKV7_PROJ_STATIC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call made
// with that device current).
int scratch_address(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return WKV7_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return WKV7_ERR_WORKSPACE;
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return WKV7_OK;
}

}  // namespace
}  // namespace wkv7

extern "C" size_t wkv7_proj_workspace_bytes(int64_t m, const wkv7_proj_group* groups,
                                            int32_t ngroups) {
  if (validate(m, groups, ngroups) != WKV7_OK || m == 0) return 0;
  int cus = 0;
  if (device_cus(&cus) != WKV7_OK) return 0;
  return make_plan(m, groups, ngroups, cus).ws_bytes;
}

extern "C" int wkv7_proj_grouped(int64_t m, const wkv7_proj_group* groups, int32_t ngroups,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = validate(m, groups, ngroups);
  if (rc != WKV7_OK) return rc;
  if (m == 0) return WKV7_OK;
  int cus = 0;
  const int drc = device_cus(&cus);
  if (drc != WKV7_OK) return drc;
  Plan p = make_plan(m, groups, ngroups, cus);
  // without (enough) workspace every tile's workgroup covers all of k
  if (p.parts > 1 && (!workspace || workspace_bytes < p.ws_bytes || !aligned16(workspace)))
    p.parts = 1;
  float* ws = static_cast<float*>(workspace);
  hipStream_t s = as_stream(stream);
  if (p.shape == 0) return launch<64, 64, 2, 2, 4, 128>(m, groups, ngroups, p.parts, ws, s);
  if (p.shape == 2) return launch<128, 64, 3, 2, 4, 128>(m, groups, ngroups, p.parts, ws, s);
  if (p.shape == 3) return launch<64, 32, 4, 2, 2, 128>(m, groups, ngroups, p.parts, ws, s);
  return launch<32, 32, 4, 2, 2, 128>(m, groups, ngroups, p.parts, ws, s);
}

extern "C" int wkv7_proj_grouped_noalloc(int64_t m, const wkv7_proj_group* groups,
                                         int32_t ngroups, void* stream) {
  const int rc = validate(m, groups, ngroups);
  if (rc != WKV7_OK) return rc;
  if (m == 0) return WKV7_OK;
  int cus = 0;
  const int drc = device_cus(&cus);
  if (drc != WKV7_OK) return drc;
  const Plan p = make_plan(m, groups, ngroups, cus);
  float* ws = nullptr;
  if (p.parts > 1) {
    // the split needs more partials than the static buffer holds
    if (p.ws_bytes > WKV7_PROJ_STATIC_SCRATCH_BYTES) return WKV7_ERR_WORKSPACE;
    const int src = scratch_address(&ws);
    if (src != WKV7_OK) return src;
  }
  hipStream_t s = as_stream(stream);
  if (p.shape == 0) return launch<64, 64, 2, 2, 4, 128>(m, groups, ngroups, p.parts, ws, s);
  if (p.shape == 2) return launch<128, 64, 3, 2, 4, 128>(m, groups, ngroups, p.parts, ws, s);
  if (p.shape == 3) return launch<64, 32, 4, 2, 2, 128>(m, groups, ngroups, p.parts, ws, s);
  return launch<32, 32, 4, 2, 2, 128>(m, groups, ngroups, p.parts, ws, s);
}
