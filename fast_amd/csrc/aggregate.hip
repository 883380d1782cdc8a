// Sum aggregation of source rows into destination rows: COO edge scatter (run-reduced)
// and CSR segment sum.
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kColSlots = 4;                    // columns per lane per tile
constexpr int kColTile = kWave * kColSlots;     // 256 columns per tile
constexpr int kRunChunk = 64;                   // consecutive edges per wave

__device__ __forceinline__ void flush_run(float* out, int64_t ldo, int64_t n_out, int64_t row,
                                          int col0, int dim, const float (&acc)[kColSlots]) {
  if (row < 0 || row >= n_out) return;
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < kColSlots; ++k) {
    const int c = col0 + lane + k * kWave;
    if (c < dim) atomicAdd(out + row * ldo + c, acc[k]);
  }
}

// One wave per chunk of kRunChunk consecutive edges. Consecutive edges with the same
// destination are summed in registers and flushed with one atomic add per column.
__global__ __launch_bounds__(kBlock) void edge_scatter_sum(const int64_t* dst, const int64_t* src,
                                                          int64_t n_edges, const int32_t* indptr,
                                                          int64_t n_seg, const float* x,
                                                          int64_t ldx, int64_t n_x, int dim,
                                                          float* out, int64_t ldo,
                                                          int64_t n_out) {
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  int64_t lo = 0, hi = n_edges;
  if (indptr) {  // only the edges covered by the CSR segments
    lo = indptr[0] < 0 ? 0 : indptr[0];
    hi = indptr[n_seg] < hi ? indptr[n_seg] : hi;
  }
  const int64_t e0 = wave * kRunChunk;
  if (e0 >= n_edges) return;
  int64_t e1 = e0 + kRunChunk < n_edges ? e0 + kRunChunk : n_edges;
  const int64_t eb = e0 < lo ? lo : e0;
  e1 = e1 > hi ? hi : e1;
  const int lane = lane_id();
  for (int col0 = 0; col0 < dim; col0 += kColTile) {
    float acc[kColSlots] = {0.f, 0.f, 0.f, 0.f};
    int64_t cur = -1;
    for (int64_t e = eb; e < e1; ++e) {
      const int64_t d = dst[e];
      const int64_t s = src[e];
      if (d != cur) {
        flush_run(out, ldo, n_out, cur, col0, dim, acc);
#pragma unroll
        for (int k = 0; k < kColSlots; ++k) acc[k] = 0.f;
        cur = d;
      }
      if (s >= 0 && s < n_x) {
        const float* row = x + s * ldx;
#pragma unroll
        for (int k = 0; k < kColSlots; ++k) {
          const int c = col0 + lane + k * kWave;
          if (c < dim) acc[k] += row[c];
        }
      }
    }
    flush_run(out, ldo, n_out, cur, col0, dim, acc);
  }
}

// One wave per CSR segment; the segment's destination is dst of its first edge.
__global__ __launch_bounds__(kBlock) void segment_sum(const int32_t* indptr, int64_t n_seg,
                                                     const int64_t* dst, const int64_t* src,
                                                     int64_t n_edges, const float* x, int64_t ldx,
                                                     int64_t n_x, int dim, float* out,
                                                     int64_t ldo, int64_t n_out) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (s >= n_seg) return;
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  if (le <= lb) return;
  const int64_t d = dst[lb];
  if (d < 0 || d >= n_out) return;
  const int lane = lane_id();
  for (int col0 = 0; col0 < dim; col0 += kColTile) {
    float acc[kColSlots] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t e = lb; e < le; ++e) {
      const int64_t sr = src[e];
      if (sr < 0 || sr >= n_x) continue;
      const float* row = x + sr * ldx;
#pragma unroll
      for (int k = 0; k < kColSlots; ++k) {
        const int c = col0 + lane + k * kWave;
        if (c < dim) acc[k] += row[c];
      }
    }
#pragma unroll
    for (int k = 0; k < kColSlots; ++k) {
      const int c = col0 + lane + k * kWave;
      if (c < dim) out[d * ldo + c] = acc[k];
    }
  }
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_edge_scatter_sum_f32(const int64_t* dst, const int64_t* src, int64_t n_edges,
                                       const int32_t* indptr, int64_t n_seg, const float* x,
                                       int64_t ldx, int64_t n_x, int32_t dim, float* out,
                                       int64_t ldo, int64_t n_out, hipStream_t stream) {
  if (n_edges < 0 || n_x < 0 || dim < 0 || n_out < 0 || n_seg < 0) return FA_EINVAL;
  if (n_edges == 0 || dim == 0 || n_out == 0) return FA_OK;
  if (!dst || !src || !out || (n_x > 0 && !x) || ldx < dim || ldo < dim) return FA_EINVAL;
  const int64_t waves = ceil_div(n_edges, kRunChunk);
  hipLaunchKernelGGL(edge_scatter_sum, dim3(ceil_div(waves, kWavesPerBlock)), dim3(kBlock), 0,
                     stream, dst, src, n_edges, indptr, n_seg, x, ldx, n_x, dim, out, ldo, n_out);
  return launch_status();
}

extern "C" int fa_segment_sum_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                                  const int64_t* src, int64_t n_edges, const float* x,
                                  int64_t ldx, int64_t n_x, int32_t dim, float* out, int64_t ldo,
                                  int64_t n_out, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || n_x < 0 || dim < 0 || n_out < 0) return FA_EINVAL;
  if (n_seg == 0 || dim == 0 || n_out == 0 || n_edges == 0) return FA_OK;
  if (!indptr || !dst || !src || !out || (n_x > 0 && !x) || ldx < dim || ldo < dim)
    return FA_EINVAL;
  hipLaunchKernelGGL(segment_sum, dim3(ceil_div(n_seg, kWavesPerBlock)), dim3(kBlock), 0, stream,
                     indptr, n_seg, dst, src, n_edges, x, ldx, n_x, dim, out, ldo, n_out);
  return launch_status();
}
