// Slot-row copy / zero kernels: fork, snapshot, gather and scatter of pool rows.
//
// The pool tensors are layer-major ([L, S+1, ...] for wkv, [L, 2, S+1, D] for
// the token-shift family), so one slot is `outer` strided rows of `row_bytes`
// contiguous bytes. Work is cut into 16 KiB tiles of one row; each of a block's
// 512 threads moves 2 vectors of the widest type the pointers, strides and row
// size allow. Pure HBM streaming: no LDS, loads of one tile are all issued
// before its stores, and both carry non-temporal hints (5 % faster than plain
// accesses when forking 128 slots of the 7B shape). On that fork 512 x 2 runs
// 3 % faster than 256 x 4; deeper unrolling, 768- or 1024-thread blocks and a
// persistent grid are all slower.
#include "wkv7_common.h"

namespace wkv7 {
namespace {

constexpr int kCopyThreads = 512;
constexpr int kCopyUnroll = 2;

struct RowMap {
  char* dst;
  int64_t dst_outer, dst_slot, dst_rows;
  const int32_t* dst_ids;
  const char* src;
  int64_t src_outer, src_slot, src_rows;
  const int32_t* src_ids;
  int64_t outer;
};

// Native vector types for the non-temporal builtins (HIP's uint4/uint2 are structs).
template <typename V> struct NativeVec { using type = V; };
template <> struct NativeVec<uint4> { typedef unsigned type __attribute__((ext_vector_type(4))); };
template <> struct NativeVec<uint2> { typedef unsigned type __attribute__((ext_vector_type(2))); };

template <typename V>
__global__ __launch_bounds__(kCopyThreads) void slot_copy_kernel(RowMap m, int64_t row_elems,
                                                                 int64_t tiles_per_row,
                                                                 int64_t total_tiles) {
  constexpr int64_t kTile = int64_t(kCopyThreads) * kCopyUnroll;
  for (int64_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    const int64_t in_row = tile % tiles_per_row;
    const int64_t po = tile / tiles_per_row;
    const int64_t o = po % m.outer;
    const int64_t p = po / m.outer;
    const int64_t d = m.dst_ids ? int64_t(m.dst_ids[p]) : p;
    const int64_t s = m.src_ids ? int64_t(m.src_ids[p]) : p;
    if (d < 0 || d >= m.dst_rows || s < 0 || s >= m.src_rows) continue;  // uniform per block
    using N = typename NativeVec<V>::type;
    const N* sp = reinterpret_cast<const N*>(m.src + o * m.src_outer + s * m.src_slot);
    N* dp = reinterpret_cast<N*>(m.dst + o * m.dst_outer + d * m.dst_slot);
    const int64_t base = in_row * kTile + threadIdx.x;
    N tmp[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t idx = base + int64_t(u) * kCopyThreads;
      if (idx < row_elems) tmp[u] = __builtin_nontemporal_load(sp + idx);
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t idx = base + int64_t(u) * kCopyThreads;
      if (idx < row_elems) __builtin_nontemporal_store(tmp[u], dp + idx);
    }
  }
}

template <typename V>
__global__ __launch_bounds__(kCopyThreads) void slot_zero_kernel(RowMap m, int64_t row_elems,
                                                                 int64_t tiles_per_row,
                                                                 int64_t total_tiles) {
  constexpr int64_t kTile = int64_t(kCopyThreads) * kCopyUnroll;
  for (int64_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    const int64_t in_row = tile % tiles_per_row;
    const int64_t po = tile / tiles_per_row;
    const int64_t o = po % m.outer;
    const int64_t p = po / m.outer;
    const int64_t d = m.dst_ids ? int64_t(m.dst_ids[p]) : p;
    if (d < 0 || d >= m.dst_rows) continue;
    V* dp = reinterpret_cast<V*>(m.dst + o * m.dst_outer + d * m.dst_slot);
    const int64_t base = in_row * kTile + threadIdx.x;
    V zero{};
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t idx = base + int64_t(u) * kCopyThreads;
      if (idx < row_elems) dp[idx] = zero;
    }
  }
}

// Widest power-of-two vector (<= 16 bytes) dividing every address term.
int vector_bytes(uint64_t bits) {
  for (int vb = 16; vb > 1; vb >>= 1)
    if ((bits & uint64_t(vb - 1)) == 0) return vb;
  return 1;
}

template <typename V, bool kZero>
void launch_one(const RowMap& m, int64_t row_elems, int64_t tiles_per_row, int64_t total,
                unsigned grid, hipStream_t stream) {
  if (kZero)
    slot_zero_kernel<V><<<grid, kCopyThreads, 0, stream>>>(m, row_elems, tiles_per_row, total);
  else
    slot_copy_kernel<V><<<grid, kCopyThreads, 0, stream>>>(m, row_elems, tiles_per_row, total);
}

template <bool kZero>
int launch_rows(const RowMap& m, int64_t row_bytes, int32_t n, int vb, hipStream_t stream) {
  const int64_t row_elems = row_bytes / vb;
  constexpr int64_t kTile = int64_t(kCopyThreads) * kCopyUnroll;
  const int64_t tiles_per_row = (row_elems + kTile - 1) / kTile;
  const int64_t total = tiles_per_row * m.outer * int64_t(n);
  if (total == 0) return WKV7_OK;
  const int64_t cap = int64_t(1) << 30;
  const unsigned grid = static_cast<unsigned>(total < cap ? total : cap);
  switch (vb) {
    case 16: launch_one<uint4, kZero>(m, row_elems, tiles_per_row, total, grid, stream); break;
    case 8: launch_one<uint2, kZero>(m, row_elems, tiles_per_row, total, grid, stream); break;
    case 4: launch_one<uint32_t, kZero>(m, row_elems, tiles_per_row, total, grid, stream); break;
    case 2: launch_one<uint16_t, kZero>(m, row_elems, tiles_per_row, total, grid, stream); break;
    default: launch_one<uint8_t, kZero>(m, row_elems, tiles_per_row, total, grid, stream); break;
  }
  return launch_status();
}

}  // namespace
}  // namespace wkv7

using namespace wkv7;

extern "C" int wkv7_slot_copy(void* dst, int64_t dst_outer_stride, int64_t dst_slot_stride,
                              int64_t dst_rows, const int32_t* dst_ids, const void* src,
                              int64_t src_outer_stride, int64_t src_slot_stride,
                              int64_t src_rows, const int32_t* src_ids, int64_t outer,
                              int64_t row_bytes, int32_t n, void* stream) {
  if (n < 0 || outer < 0 || row_bytes < 0 || dst_rows < 0 || src_rows < 0) return WKV7_ERR_ARG;
  if (n == 0 || outer == 0 || row_bytes == 0) return WKV7_OK;
  if (!dst || !src) return WKV7_ERR_ARG;
  if (row_bytes > dst_slot_stride && dst_rows > 1) return WKV7_ERR_SHAPE;
  if (row_bytes > src_slot_stride && src_rows > 1) return WKV7_ERR_SHAPE;
  RowMap m{static_cast<char*>(dst), dst_outer_stride, dst_slot_stride, dst_rows, dst_ids,
           static_cast<const char*>(src), src_outer_stride, src_slot_stride, src_rows, src_ids,
           outer};
  const uint64_t bits = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                        uint64_t(dst_outer_stride) | uint64_t(dst_slot_stride) |
                        uint64_t(src_outer_stride) | uint64_t(src_slot_stride) |
                        uint64_t(row_bytes);
  return launch_rows<false>(m, row_bytes, n, vector_bytes(bits), as_stream(stream));
}

extern "C" int wkv7_slot_zero(void* base, int64_t outer_stride, int64_t slot_stride, int64_t rows,
                              const int32_t* ids, int64_t outer, int64_t row_bytes, int32_t n,
                              void* stream) {
  if (n < 0 || outer < 0 || row_bytes < 0 || rows < 0) return WKV7_ERR_ARG;
  if (n == 0 || outer == 0 || row_bytes == 0) return WKV7_OK;
  if (!base) return WKV7_ERR_ARG;
  if (row_bytes > slot_stride && rows > 1) return WKV7_ERR_SHAPE;
  RowMap m{static_cast<char*>(base), outer_stride, slot_stride, rows, ids,
           nullptr, 0, 0, 0, nullptr, outer};
  const uint64_t bits = reinterpret_cast<uintptr_t>(base) | uint64_t(outer_stride) |
                        uint64_t(slot_stride) | uint64_t(row_bytes);
  return launch_rows<true>(m, row_bytes, n, vector_bytes(bits), as_stream(stream));
}

extern "C" int wkv7_slot_transfer(int32_t direction, void* host, void* base, int64_t outer_stride,
                                  int64_t slot_stride, int64_t rows, int32_t slot, int64_t outer,
                                  int64_t row_bytes, void* staging, size_t staging_bytes,
                                  void* stream) {
  if (direction != WKV7_TO_HOST && direction != WKV7_FROM_HOST) return WKV7_ERR_ARG;
  if (outer < 0 || row_bytes < 0 || rows < 1 || slot < 0 || slot >= rows) return WKV7_ERR_ARG;
  if (outer == 0 || row_bytes == 0) return WKV7_OK;
  if (!host || !base) return WKV7_ERR_ARG;
  if (rows > 1 && row_bytes > slot_stride) return WKV7_ERR_SHAPE;
  if (outer > 1 && row_bytes > outer_stride) return WKV7_ERR_SHAPE;
  const size_t total = size_t(outer) * size_t(row_bytes);
  if (staging && staging_bytes < total) return WKV7_ERR_WORKSPACE;
  char* dev = static_cast<char*>(base) + int64_t(slot) * slot_stride;
  hipStream_t s = as_stream(stream);
  hipError_t e;
  if (staging) {
    // Dense device staging: the slot's strided rows <-> staging with the copy
    // kernel (HBM speed), then one contiguous DMA to or from the host.
    char* st = static_cast<char*>(staging);
    const uint64_t bits = reinterpret_cast<uintptr_t>(dev) | reinterpret_cast<uintptr_t>(st) |
                          uint64_t(outer_stride) | uint64_t(row_bytes);
    const int vb = vector_bytes(bits);
    if (direction == WKV7_TO_HOST) {
      RowMap m{st, row_bytes, 0, 1, nullptr, dev, outer_stride, 0, 1, nullptr, outer};
      const int rc = launch_rows<false>(m, row_bytes, 1, vb, s);
      if (rc != WKV7_OK) return rc;
      e = hipMemcpyAsync(host, st, total, hipMemcpyDeviceToHost, s);
    } else {
      e = hipMemcpyAsync(st, host, total, hipMemcpyHostToDevice, s);
      if (e != hipSuccess) return static_cast<int>(e);
      RowMap m{dev, outer_stride, 0, 1, nullptr, st, row_bytes, 0, 1, nullptr, outer};
      return launch_rows<false>(m, row_bytes, 1, vb, s);
    }
    return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
  }
  const size_t width = size_t(row_bytes), height = size_t(outer);
  // a single block needs no pitch; give the DMA its own width then
  const size_t dev_pitch = outer > 1 ? size_t(outer_stride) : width;
  if (direction == WKV7_TO_HOST)
    e = hipMemcpy2DAsync(host, width, dev, dev_pitch, width, height, hipMemcpyDeviceToHost, s);
  else
    e = hipMemcpy2DAsync(dev, dev_pitch, host, width, width, height, hipMemcpyHostToDevice, s);
  return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
}
