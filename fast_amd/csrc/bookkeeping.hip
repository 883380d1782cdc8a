// Segment bookkeeping kernels: exclusive scan, degree histogram, balance mask and the
// full-CSR row pointer. All integer work, bit-exact and deterministic.
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kScanItems = 8;                         // items per thread
constexpr int kScanTile = kBlock * kScanItems;        // 2048 items per workgroup

// Exclusive scan of the kBlock per-thread values `v` inside one workgroup (uint32
// arithmetic, i.e. int32 wrap-around). Returns the exclusive prefix of this thread and
// writes the workgroup total to *total.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wave_tot[kWavesPerBlock];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint32_t o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) {
    if (w < wave) before += wave_tot[w];
    all += wave_tot[w];
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

__device__ __forceinline__ uint32_t scan_item(const int32_t* in, int64_t n, int64_t i) {
  // The scanned sequence is in[0..n) followed by one 0 (n+1 items).
  return i < n ? static_cast<uint32_t>(in[i]) : 0u;
}

__global__ __launch_bounds__(kBlock) void scan_tile_sums(const int32_t* in, int64_t n,
                                                        uint32_t* tile_sum) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * kScanItems;
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) s += scan_item(in, n, base + i);
  uint32_t tot;
  block_exclusive_scan(s, &tot);
  if (threadIdx.x == 0) tile_sum[blockIdx.x] = tot;
}

// Single workgroup: exclusive scan of the tile sums, in place.
__global__ __launch_bounds__(kBlock) void scan_tile_offsets(uint32_t* tile_sum, int64_t n_tiles) {
  uint32_t carry = 0;
  for (int64_t base = 0; base < n_tiles; base += kScanTile) {
    uint32_t v[kScanItems];
    uint32_t s = 0;
    const int64_t my = base + threadIdx.x * kScanItems;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      v[i] = (my + i < n_tiles) ? tile_sum[my + i] : 0u;
      s += v[i];
    }
    uint32_t tot;
    uint32_t ex = block_exclusive_scan(s, &tot) + carry;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      if (my + i < n_tiles) tile_sum[my + i] = ex;
      ex += v[i];
    }
    carry += tot;
  }
}

__global__ __launch_bounds__(kBlock) void scan_tile_write(const int32_t* in, int64_t n,
                                                         const uint32_t* tile_off,
                                                         int32_t* out) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    v[i] = scan_item(in, n, base + i);
    s += v[i];
  }
  uint32_t tot;
  uint32_t ex = block_exclusive_scan(s, &tot) + tile_off[blockIdx.x];
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    if (base + i <= n) out[base + i] = static_cast<int32_t>(ex);
    ex += v[i];
  }
}

// Runs of equal ids among a wave's 64 consecutive ids are counted once: the first lane of a
// run adds the run's length (sorted or clustered ids, the sampler's layout, then cost one
// atomic per distinct id and wave instead of one per id; integer sums, so the result does
// not depend on the order).
__global__ __launch_bounds__(kBlock) void degree_count(const int32_t* ids, int64_t n_ids,
                                                      int32_t* deg, int64_t n_nodes) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int lane = lane_id();
  const bool in = i < n_ids;
  const int32_t v = in ? ids[i] : 0;
  const int32_t up = __shfl(v, lane > 0 ? lane - 1 : 0, kWave);
  const bool up_in = lane > 0 && i - 1 < n_ids;
  // a lane past the end starts a run of its own, which ends the last real run
  const bool head = !in || lane == 0 || !up_in || v != up;
  const uint64_t heads = __ballot(head);
  if (!in || !head || v < 0 || v >= n_nodes) return;
  const uint64_t later = lane == kWave - 1 ? 0ull : heads & (~0ull << (lane + 1));
  const int next = later ? __builtin_ctzll(later) : kWave;
  atomicAdd(deg + v, next - lane);
}

__global__ __launch_bounds__(kBlock) void balance_mask(const int32_t* ptr, int64_t n,
                                                      int32_t threshold, int32_t* mask) {
  // Entry i (< n-1) of the mask; the prefix restarts at every aligned block of 256.
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const uint32_t deg = (i < n - 1) ? static_cast<uint32_t>(ptr[i + 1]) - static_cast<uint32_t>(ptr[i]) : 0u;
  uint32_t tot;
  const uint32_t before = block_exclusive_scan(deg, &tot);
  if (i < n - 1) {
    const int32_t after_v = static_cast<int32_t>(before + deg);
    const int32_t before_v = static_cast<int32_t>(before);
    mask[i] = (after_v / threshold > before_v / threshold) ? 1 : 0;
  }
}

__global__ __launch_bounds__(kBlock) void rowptr_from_sorted(const int64_t* dst, int64_t n_edges,
                                                            int64_t n_dst, int32_t* rowptr) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (v > n_dst) return;
  int64_t lo = 0, hi = n_edges;  // first index with dst[idx] >= v
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (dst[mid] < v) lo = mid + 1; else hi = mid;
  }
  rowptr[v] = static_cast<int32_t>(lo);
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" size_t fa_exclusive_sum_scratch_bytes(int64_t n) {
  if (n < 0) return 0;
  return static_cast<size_t>(ceil_div(n + 1, kScanTile)) * sizeof(uint32_t);
}

extern "C" int fa_exclusive_sum_i32(const int32_t* in, int64_t n, int32_t* out, void* scratch,
                                    size_t scratch_bytes, hipStream_t stream) {
  if (n < 0 || out == nullptr || (n > 0 && in == nullptr)) return FA_EINVAL;
  const int64_t tiles = ceil_div(n + 1, kScanTile);
  if (scratch == nullptr || scratch_bytes < fa_exclusive_sum_scratch_bytes(n)) return FA_ESCRATCH;
  if (tiles > INT32_MAX) return FA_EUNSUPPORTED;
  uint32_t* ts = static_cast<uint32_t*>(scratch);
  hipLaunchKernelGGL(scan_tile_sums, dim3(tiles), dim3(kBlock), 0, stream, in, n, ts);
  hipLaunchKernelGGL(scan_tile_offsets, dim3(1), dim3(kBlock), 0, stream, ts, tiles);
  hipLaunchKernelGGL(scan_tile_write, dim3(tiles), dim3(kBlock), 0, stream, in, n, ts, out);
  return launch_status();
}

extern "C" int fa_degree_count_i32(const int32_t* ids, int64_t n_ids, int32_t* deg,
                                   int64_t n_nodes, hipStream_t stream) {
  if (n_ids < 0 || n_nodes < 0 || (n_ids > 0 && ids == nullptr) || (n_nodes > 0 && deg == nullptr))
    return FA_EINVAL;
  if (n_ids == 0 || n_nodes == 0) return FA_OK;
  hipLaunchKernelGGL(degree_count, dim3(ceil_div(n_ids, kBlock)), dim3(kBlock), 0, stream, ids,
                     n_ids, deg, n_nodes);
  return launch_status();
}

extern "C" int fa_balance_mask_i32(const int32_t* dense_ptr, int64_t n, int32_t threshold,
                                   int32_t* mask, hipStream_t stream) {
  if (n < 1 || dense_ptr == nullptr || threshold == 0) return FA_EINVAL;
  if (n == 1) return FA_OK;
  if (mask == nullptr) return FA_EINVAL;
  hipLaunchKernelGGL(balance_mask, dim3(ceil_div(n, kBlock)), dim3(kBlock), 0, stream, dense_ptr,
                     n, threshold, mask);
  return launch_status();
}

extern "C" int fa_rowptr_from_sorted_dst_i64(const int64_t* dst, int64_t n_edges, int64_t n_dst,
                                             int32_t* rowptr, hipStream_t stream) {
  if (n_edges < 0 || n_dst < 0 || rowptr == nullptr || (n_edges > 0 && dst == nullptr))
    return FA_EINVAL;
  if (n_edges > INT32_MAX) return FA_EUNSUPPORTED;
  hipLaunchKernelGGL(rowptr_from_sorted, dim3(ceil_div(n_dst + 1, kBlock)), dim3(kBlock), 0,
                     stream, dst, n_edges, n_dst, rowptr);
  return launch_status();
}
