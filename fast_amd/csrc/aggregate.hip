// Sum aggregation of source rows into destination rows: COO edge scatter and CSR segment
// sum. The COO scatter checks on the device whether the output index is sorted; if it is,
// every output row is the sum of one run of edges and is written with plain stores by the
// run's owner (atomic-free, deterministic, every row of the output written); if not, the
// output is zero-filled and runs of equal consecutive indices are added with atomics.
//
// Rows are read through buffer descriptors sized to the row (a row id out of range has an
// empty descriptor and reads as zeros), as float4 chunks when every row start is 16-byte
// aligned and the width a multiple of 4, else dword by dword. Lane l owns chunks l, l+64,
// ... of a row (NS slots). Per-edge ids are loaded 64 at a time with one coalesced load
// and broadcast with readlane; kBatch rows are in flight per wave.
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kBatchRows = 8;   // rows in flight per wave
constexpr int kMaxSlots = 4;    // float4 slots per lane: rows up to 1024 floats

using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t row_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// AUX: cache-policy bits; kStream (non-temporal) for rows read or written once, so that they
// leave the caches first.
constexpr int kStream = 2;

template <bool VEC, int AUX = 0>
__device__ __forceinline__ float4 load_chunk(rsrc_t r, uint32_t off) {
  if (VEC) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, AUX);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
  }
  const int o = static_cast<int>(off);
  return make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o, 0, AUX)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4, 0, AUX)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 8, 0, AUX)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 12, 0, AUX)));
}

template <bool VEC, int AUX = 0>
__device__ __forceinline__ void store_chunk(rsrc_t r, uint32_t off, const float4& x) {
  if (VEC) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    u4 v;
    v[0] = __float_as_uint(x.x);
    v[1] = __float_as_uint(x.y);
    v[2] = __float_as_uint(x.z);
    v[3] = __float_as_uint(x.w);
    __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(off), 0, AUX);
    return;
  }
  const int o = static_cast<int>(off);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.x), r, o, 0, AUX);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.y), r, o + 4, 0, AUX);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.z), r, o + 8, 0, AUX);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.w), r, o + 12, 0, AUX);
}

__device__ __forceinline__ int64_t lane_i64(int64_t v, int j) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffff), j));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), j));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

struct AggParams {
  const int64_t* dst;
  const int64_t* src;
  int64_t n_edges;
  const int32_t* indptr;
  int64_t n_seg;
  const float* x; int64_t ldx; int64_t n_x;
  int dim;
  int chunks;            // ceil(dim / 4)
  float* out; int64_t ldo; int64_t n_out;
};

// Loads the rows of kBatchRows edges (ids broadcast from lanes j0.. of `ids`).
template <int NS, bool VEC, int AUX = 0>
__device__ __forceinline__ void load_batch(const AggParams& P, int64_t ids, int j0, int nb,
                                           float4 (&r)[kBatchRows][NS]) {
  const int lane = lane_id();
#pragma unroll
  for (int b = 0; b < kBatchRows; ++b) {
    if (b < nb) {
      const int64_t s = lane_i64(ids, j0 + b);
      const bool ok = s >= 0 && s < P.n_x;
      const rsrc_t rr = row_rsrc(P.x + (ok ? s : 0) * P.ldx, ok ? 4u * static_cast<uint32_t>(P.dim) : 0u);
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const int c = lane + k * kWave;
        r[b][k] = c < P.chunks ? load_chunk<VEC, AUX>(rr, 16u * static_cast<uint32_t>(c)) : f4_zero();
      }
    }
  }
}

template <int NS>
__device__ __forceinline__ void add_chunks(float4 (&acc)[NS], const float4 (&r)[NS]) {
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    acc[k].x += r[k].x;
    acc[k].y += r[k].y;
    acc[k].z += r[k].z;
    acc[k].w += r[k].w;
  }
}

// One wave per CSR segment (grid-stride); the segment's destination is dst of its first edge.
template <int NS, bool VEC>
__global__ __launch_bounds__(kBlock) void segment_sum(AggParams P) {
  const int lane = lane_id();
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       s < P.n_seg; s += total) {
    int64_t lb = P.indptr[s], le = P.indptr[s + 1];
    lb = lb < 0 ? 0 : lb;
    le = le > P.n_edges ? P.n_edges : le;
    if (le <= lb) continue;
    const int64_t d = P.dst[lb];
    if (d < 0 || d >= P.n_out) continue;
    float4 acc[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = f4_zero();
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const int cnt = static_cast<int>(le - e0 < kWave ? le - e0 : kWave);
      const int64_t ids = P.src[e0 + (lane < cnt ? lane : 0)];
      for (int j = 0; j < cnt; j += kBatchRows) {
        const int nb = cnt - j < kBatchRows ? cnt - j : kBatchRows;
        float4 r[kBatchRows][NS];
        load_batch<NS, VEC, kStream>(P, ids, j, nb, r);
#pragma unroll
        for (int b = 0; b < kBatchRows; ++b)
          if (b < nb) add_chunks<NS>(acc, r[b]);
      }
    }
    const rsrc_t orow = row_rsrc(P.out + d * P.ldo, 4u * static_cast<uint32_t>(P.dim));
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c = lane + k * kWave;
      if (c < P.chunks) store_chunk<VEC, kStream>(orow, 16u * static_cast<uint32_t>(c), acc[k]);
    }
  }
}

// The value of lane `src` (any lane, per lane).
__device__ __forceinline__ int64_t lane_i64_from(int64_t v, int src) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(v & 0xffffffff)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Rows in flight per half-wave. More (8) measured slower at 100-float rows: the registers
// they take cost occupancy that the deeper batch does not win back.
constexpr int run_rows(int) { return 4; }

template <int NS>
__device__ __forceinline__ void flush_run(const AggParams& P, int64_t row, const float4 (&acc)[NS],
                                          float* stage) {
  if (row < 0 || row >= P.n_out) return;
  atomic_add_row<NS>(P.out + row * P.ldo, P.dim, acc, stage);
}

// One wave per 64 consecutive edges. Consecutive edges with the same destination are summed
// in registers and flushed with one atomic add per column (issued lane-consecutively through
// an LDS staging row), so for destination-sorted input a
// run of at most 64 edges reaches its output row as at most two partial sums (whose sum does
// not depend on their order).
template <int NS, bool VEC>
__global__ __launch_bounds__(kBlock) void edge_scatter_sum(AggParams P, const int* flag) {
  if (flag[0] == 0) return;  // sorted: run_scatter wrote the output
  __shared__ __attribute__((aligned(16))) float stage_all[kWavesPerBlock][4 * kWave * NS];
  float* stage = stage_all[threadIdx.x / kWave];
  const int lane = lane_id();
  int64_t lo = 0, hi = P.n_edges;
  if (P.indptr) {  // only the edges covered by the CSR segments
    lo = P.indptr[0] < 0 ? 0 : P.indptr[0];
    hi = P.indptr[P.n_seg] < hi ? P.indptr[P.n_seg] : hi;
  }
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       w * kWave < P.n_edges; w += total) {
    int64_t e0 = w * kWave, e1 = e0 + kWave < P.n_edges ? e0 + kWave : P.n_edges;
    e0 = e0 < lo ? lo : e0;
    e1 = e1 > hi ? hi : e1;
    if (e1 <= e0) continue;
    const int cnt = static_cast<int>(e1 - e0);
    const int64_t my_dst = P.dst[e0 + (lane < cnt ? lane : 0)];
    const int64_t my_src = P.src[e0 + (lane < cnt ? lane : 0)];
    float4 acc[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = f4_zero();
    int64_t cur = lane_i64(my_dst, 0);
    for (int j = 0; j < cnt; j += kBatchRows) {
      const int nb = cnt - j < kBatchRows ? cnt - j : kBatchRows;
      float4 r[kBatchRows][NS];
      load_batch<NS, VEC>(P, my_src, j, nb, r);
#pragma unroll
      for (int b = 0; b < kBatchRows; ++b) {
        if (b < nb) {
          const int64_t d = lane_i64(my_dst, j + b);
          if (d != cur) {
            flush_run<NS>(P, cur, acc, stage);
#pragma unroll
            for (int k = 0; k < NS; ++k) acc[k] = f4_zero();
            cur = d;
          }
          add_chunks<NS>(acc, r[b]);
        }
      }
    }
    flush_run<NS>(P, cur, acc, stage);
  }
}

// ---------------------------------------------------------------------------------
// Sorted output index: run owners, plain stores
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void flag_clear(int* flag) {
  if (threadIdx.x == 0) flag[0] = 0;
}


// The edges taken: all, or the range the CSR segments cover (indptr[0] .. indptr[n_seg]).
__device__ __forceinline__ void edge_range(const AggParams& P, int64_t& lo, int64_t& hi) {
  lo = 0;
  hi = P.n_edges;
  if (P.indptr) {
    lo = P.indptr[0] < 0 ? 0 : P.indptr[0];
    hi = P.indptr[P.n_seg] < hi ? P.indptr[P.n_seg] : hi;
    hi = hi < lo ? lo : hi;
  }
}

// flag |= 1 when dst[e] < dst[e-1] for some lo < e < hi.
__global__ __launch_bounds__(kBlock) void check_sorted(AggParams P, int* flag) {
  int64_t lo, hi;
  edge_range(P, lo, hi);
  bool bad = false;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t e = lo + 1 + static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < hi;
       e += stride)
    bad |= P.dst[e] < P.dst[e - 1];
  const uint64_t any = __ballot(bad);
  if (any && lane_id() == __builtin_ctzll(any)) atomicOr(flag, 1);
}


// Zero rows [r0, r1) of out (clamped to [0, n_out)) by a half-wave.
template <int NS, bool VEC>
__device__ __forceinline__ void zero_rows(const AggParams& P, int64_t r0, int64_t r1, int hl) {
  r0 = r0 < 0 ? 0 : r0;
  r1 = r1 > P.n_out ? P.n_out : r1;
  for (int64_t r = r0; r < r1; ++r) {
    const rsrc_t orow = row_rsrc(P.out + r * P.ldo, 4u * static_cast<uint32_t>(P.dim));
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c = hl + k * kHalf;
      if (c < P.chunks) store_chunk<VEC, kStream>(orow, 16u * static_cast<uint32_t>(c), f4_zero());
    }
  }
}

constexpr int64_t kNoIndex = INT64_MIN;   // "no previous index"
// Rows in flight per half-wave when every run is one edge long (register budget by slots).
constexpr int copy_rows(int ns) { return ns <= 4 ? 4 : 2; }

// One wave per 64 consecutive edges of [lo, hi); the wave owns the runs (maximal ranges of
// equal output index) that start in its edges and takes them two at a time, one per
// half-wave. A run's owner sums its rows (lane hl holds chunks hl, hl+32, ...; the run's
// source ids from the tile's ids staged in LDS, or loaded 32 at a time past the tile;
// run_rows rows in flight), stores the output row, and zeroes
// the output rows between the previous run's index and its own. The rows before the first
// index and after the last are zeroed by the whole grid. Indices outside [0, n_out) are not
// written. With an unsorted index (flag set) the kernel zero-fills the output instead, for
// the atomic kernel that follows.
template <int NS, bool VEC>
__global__ __launch_bounds__(kBlock) void run_scatter(AggParams P, const int* flag) {
  constexpr int RR = run_rows(NS);
  // the source ids of the wave's current tile, read by the lanes of whichever half-wave
  // takes a run (LDS reads do not depend on the other half being active)
  __shared__ int64_t tile_src[kWavesPerBlock][kWave];
  const int wv = threadIdx.x / kWave;
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
  int64_t lo, hi;
  edge_range(P, lo, hi);
  if (flag[0] != 0 || hi <= lo) {  // unsorted, or no edge: zero-fill by half-waves
    for (int64_t r = w0 * 2 + half; r < P.n_out; r += waves * 2) zero_rows<NS, VEC>(P, r, r + 1, hl);
    return;
  }
  {  // the rows before the first index and after the last, by every half-wave of the grid
    const int64_t first = P.dst[lo], last = P.dst[hi - 1];
    const int64_t head = first < 0 ? 0 : (first > P.n_out ? P.n_out : first);
    const int64_t tail = last < 0 ? 0 : (last + 1 > P.n_out ? P.n_out : last + 1);
    for (int64_t r = w0 * 2 + half; r < head; r += waves * 2) zero_rows<NS, VEC>(P, r, r + 1, hl);
    for (int64_t r = tail + w0 * 2 + half; r < P.n_out; r += waves * 2)
      zero_rows<NS, VEC>(P, r, r + 1, hl);
  }
  for (int64_t w = w0; lo + w * kWave < hi; w += waves) {
    const int64_t e0 = lo + w * kWave;
    const int cnt = static_cast<int>(hi - e0 < kWave ? hi - e0 : kWave);
    const int64_t my = P.dst[e0 + (lane < cnt ? lane : cnt - 1)];
    const int64_t prev_tile = e0 > lo ? P.dst[e0 - 1] : kNoIndex;
    const int64_t up = lane_i64_from(my, lane > 0 ? lane - 1 : 0);
    const bool start = lane < cnt && (lane == 0 ? (e0 == lo || my != prev_tile) : my != up);
    uint64_t m = __ballot(start);
    const int64_t tsrc = P.src[e0 + (lane < cnt ? lane : cnt - 1)];
    {
      // Every edge of the tile a run of its own (the last one too) and no gap below any of
      // them: each output row is one source row, copied by half-waves, copy_rows(NS) rows in
      // flight per half.
      const uint64_t all = cnt == kWave ? ~0ull : (1ull << cnt) - 1;
      const int64_t last = lane_i64(my, cnt - 1);
      const bool has_next = e0 + cnt < hi;
      const int64_t next = has_next ? P.dst[e0 + cnt] : 0;
      const int64_t prev = lane == 0 ? (e0 == lo ? kNoIndex : prev_tile) : up;
      const bool gap = lane < cnt && prev != kNoIndex && my != kNoIndex && my - 1 > prev;
      if (m == all && __ballot(gap) == 0 && (!has_next || next != last)) {
        constexpr int R = copy_rows(NS);
        const int64_t ids = tsrc;
        for (int j = 0; j < cnt; j += 2 * R) {
          float4 r[R][NS];
#pragma unroll
          for (int q = 0; q < R; ++q) {
            const int jj = j + 2 * q + half;
            const int64_t sidx = lane_i64_from(ids, jj < cnt ? jj : 0);
            const bool ok = jj < cnt && sidx >= 0 && sidx < P.n_x;
            const rsrc_t rr = row_rsrc(P.x + (ok ? sidx : 0) * P.ldx, ok ? 4u * static_cast<uint32_t>(P.dim) : 0u);
#pragma unroll
            for (int k = 0; k < NS; ++k) {
              const int c = hl + k * kHalf;
              r[q][k] = c < P.chunks ? load_chunk<VEC>(rr, 16u * static_cast<uint32_t>(c)) : f4_zero();
            }
          }
#pragma unroll
          for (int q = 0; q < R; ++q) {
            const int jj = j + 2 * q + half;
            const int64_t row = lane_i64_from(my, jj < cnt ? jj : 0);
            if (jj < cnt && row >= 0 && row < P.n_out) {
              const rsrc_t orow = row_rsrc(P.out + row * P.ldo, 4u * static_cast<uint32_t>(P.dim));
#pragma unroll
              for (int k = 0; k < NS; ++k) {
                const int c = hl + k * kHalf;
                if (c < P.chunks) store_chunk<VEC, kStream>(orow, 16u * static_cast<uint32_t>(c), r[q][k]);
              }
            }
          }
        }
        continue;
      }
    }
    lds_sync();   // the previous tile's reads of tile_src are done
    tile_src[wv][lane] = tsrc;
    lds_sync();
    const int64_t tile_end = e0 + cnt;
    while (m) {
      // two runs: bit b0 for the first half-wave, b1 (if any) for the second
      const int b0 = __builtin_ctzll(m);
      m &= m - 1;
      const int b1 = m ? __builtin_ctzll(m) : -1;
      if (m) m &= m - 1;
      const int b = half ? b1 : b0;
      const int nb = half ? (m ? __builtin_ctzll(m) : -1) : b1;  // the next run's start bit
      // lane reads with the whole wave active (a permute from an inactive lane reads zero)
      const int bs = b < 0 ? 0 : b;
      const int64_t row = lane_i64_from(my, bs);
      const int64_t before_v = lane_i64_from(my, bs > 0 ? bs - 1 : 0);
      if (b < 0) continue;
      const int64_t before = b == 0 ? prev_tile : before_v;
      int64_t end;
      if (nb >= 0) {
        end = e0 + nb;
      } else {  // the tile's last run: scan past the tile for its end
        end = e0 + cnt;
        while (end < hi) {
          const int64_t e = end + hl;
          const int64_t v = e < hi ? P.dst[e] : row + 1;  // past the end: a different index
          const uint32_t diff = static_cast<uint32_t>(__ballot(v != row) >> (half * kHalf));
          if (diff) {
            end += __builtin_ctz(diff);
            break;
          }
          end += kHalf;
        }
        end = end > hi ? hi : end;
      }
      if (before != kNoIndex) zero_rows<NS, VEC>(P, before + 1, row, hl);  // the gap below
      if (row >= 0 && row < P.n_out) {
        float4 acc[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) acc[k] = f4_zero();
        for (int64_t eb = e0 + b; eb < end; eb += kHalf) {
          const int n = static_cast<int>(end - eb < kHalf ? end - eb : kHalf);
          // edges inside the tile take their ids from tile_src; the tile's last run, where it
          // goes on past the tile, loads this half's next 32 source ids
          const bool in_tile = eb + n <= tile_end;
          const int64_t ids = in_tile ? 0 : P.src[eb + (hl < n ? hl : 0)];
          for (int j = 0; j < n; j += RR) {
            float4 r[RR][NS];
#pragma unroll
            for (int q = 0; q < RR; ++q) {
              const int jj = j + q < n ? j + q : 0;
              const int64_t from_tile = tile_src[wv][in_tile ? static_cast<int>(eb - e0) + jj : 0];
              // permutes stay inside this half-wave, whose lanes are all active
              const int64_t from_ids = lane_i64_from(ids, half * kHalf + jj);
              const int64_t sidx = in_tile ? from_tile : from_ids;
              const bool ok = j + q < n && sidx >= 0 && sidx < P.n_x;
              const rsrc_t rr = row_rsrc(P.x + (ok ? sidx : 0) * P.ldx, ok ? 4u * static_cast<uint32_t>(P.dim) : 0u);
#pragma unroll
              for (int k = 0; k < NS; ++k) {
                const int c = hl + k * kHalf;
                r[q][k] = c < P.chunks ? load_chunk<VEC, kStream>(rr, 16u * static_cast<uint32_t>(c)) : f4_zero();
              }
            }
#pragma unroll
            for (int q = 0; q < RR; ++q)
#pragma unroll
              for (int k = 0; k < NS; ++k) {
                acc[k].x += r[q][k].x;
                acc[k].y += r[q][k].y;
                acc[k].z += r[q][k].z;
                acc[k].w += r[q][k].w;
              }
          }
        }
        const rsrc_t orow = row_rsrc(P.out + row * P.ldo, 4u * static_cast<uint32_t>(P.dim));
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          const int c = hl + k * kHalf;
          if (c < P.chunks) store_chunk<VEC, kStream>(orow, 16u * static_cast<uint32_t>(c), acc[k]);
        }
      }
    }
  }
}

constexpr int kAggMaxBlocks = 4096;

int agg_grid(int64_t waves) {
  const int64_t want = ceil_div(waves, kWavesPerBlock);
  return static_cast<int>(want < kAggMaxBlocks ? (want < 1 ? 1 : want) : kAggMaxBlocks);
}

bool vec_ok(const AggParams& P) {
  return (P.dim & 3) == 0 && (P.ldx & 3) == 0 && (P.ldo & 3) == 0 && aligned16(P.x) &&
         aligned16(P.out);
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" size_t fa_edge_scatter_sum_scratch_bytes(void) { return 16; }

extern "C" int fa_edge_scatter_sum_f32(const int64_t* dst, const int64_t* src, int64_t n_edges,
                                       const int32_t* indptr, int64_t n_seg, const float* x,
                                       int64_t ldx, int64_t n_x, int32_t dim, float* out,
                                       int64_t ldo, int64_t n_out, void* scratch,
                                       size_t scratch_bytes, hipStream_t stream) {
  if (n_edges < 0 || n_x < 0 || dim < 0 || n_out < 0 || n_seg < 0) return FA_EINVAL;
  if (dim == 0 || n_out == 0) return FA_OK;
  if (!out || ldo < dim || (n_edges > 0 && (!dst || !src || (n_x > 0 && !x) || ldx < dim)))
    return FA_EINVAL;
  if (dim > 4 * kWave * kMaxSlots) return FA_EUNSUPPORTED;
  if (!scratch || scratch_bytes < fa_edge_scatter_sum_scratch_bytes()) return FA_ESCRATCH;
  int* flag = static_cast<int*>(scratch);
  AggParams P{dst, src, n_edges, indptr, n_seg, x, ldx, n_x, dim, static_cast<int>(ceil_div(dim, 4)),
              out, ldo, n_out};
  const dim3 grid(agg_grid(ceil_div(n_edges > 0 ? n_edges : 1, kWave)));
  const int ns = static_cast<int>(ceil_div(P.chunks, kWave));
  const int ns_half = static_cast<int>(ceil_div(P.chunks, kHalf));
  const bool vec = vec_ok(P);
  hipLaunchKernelGGL(flag_clear, dim3(1), dim3(64), 0, stream, flag);
  if (n_edges > 1)
    hipLaunchKernelGGL(check_sorted, grid, dim3(kBlock), 0, stream, P, flag);
#define FA_RUN_LAUNCH(NSV)                                                                       \
  if (vec) hipLaunchKernelGGL((run_scatter<NSV, true>), grid, dim3(kBlock), 0, stream, P,        \
                              static_cast<const int*>(flag));                                    \
  else hipLaunchKernelGGL((run_scatter<NSV, false>), grid, dim3(kBlock), 0, stream, P,           \
                          static_cast<const int*>(flag));
  switch (ns_half) {
    case 1: FA_RUN_LAUNCH(1) break;
    case 2: FA_RUN_LAUNCH(2) break;
    case 3: FA_RUN_LAUNCH(3) break;
    case 4: FA_RUN_LAUNCH(4) break;
    case 5: case 6: FA_RUN_LAUNCH(6) break;
    default: FA_RUN_LAUNCH(8) break;
  }
#undef FA_RUN_LAUNCH
  if (n_edges > 0) {
#define FA_AGG_LAUNCH(NSV)                                                                       \
    if (vec) hipLaunchKernelGGL((edge_scatter_sum<NSV, true>), grid, dim3(kBlock), 0, stream, P,  \
                                static_cast<const int*>(flag));                                  \
    else hipLaunchKernelGGL((edge_scatter_sum<NSV, false>), grid, dim3(kBlock), 0, stream, P,     \
                            static_cast<const int*>(flag));
    switch (ns) {
      case 1: FA_AGG_LAUNCH(1) break;
      case 2: FA_AGG_LAUNCH(2) break;
      case 3: FA_AGG_LAUNCH(3) break;
      default: FA_AGG_LAUNCH(4) break;
    }
#undef FA_AGG_LAUNCH
  }
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
  if (dim > 4 * kWave * kMaxSlots) return FA_EUNSUPPORTED;
  AggParams P{dst, src, n_edges, indptr, n_seg, x, ldx, n_x, dim, static_cast<int>(ceil_div(dim, 4)),
              out, ldo, n_out};
  const dim3 grid(agg_grid(n_seg));
  const int ns = static_cast<int>(ceil_div(P.chunks, kWave));
  const bool vec = vec_ok(P);
#define FA_AGG_LAUNCH(NSV)                                                                 \
  if (vec) hipLaunchKernelGGL((segment_sum<NSV, true>), grid, dim3(kBlock), 0, stream, P); \
  else hipLaunchKernelGGL((segment_sum<NSV, false>), grid, dim3(kBlock), 0, stream, P);
  switch (ns) {
    case 1: FA_AGG_LAUNCH(1) break;
    case 2: FA_AGG_LAUNCH(2) break;
    case 3: FA_AGG_LAUNCH(3) break;
    default: FA_AGG_LAUNCH(4) break;
  }
#undef FA_AGG_LAUNCH
  return launch_status();
}
