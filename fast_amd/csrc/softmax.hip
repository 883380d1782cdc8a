// Segmented edge softmax over the incoming edges of each destination, forward and
// backward, plus the grouped ("balanced") variant keyed by a per-batch local node id.
#include <float.h>

#include "fa_common.hpp"

namespace fa {
namespace {

template <typename T> __device__ __forceinline__ T dev_exp(T x);
template <> __device__ __forceinline__ float dev_exp<float>(float x) { return expf(x); }
template <> __device__ __forceinline__ double dev_exp<double>(double x) { return exp(x); }

template <typename T> __device__ __forceinline__ T dev_max(T a, T b);
template <> __device__ __forceinline__ float dev_max<float>(float a, float b) { return fmaxf(a, b); }
template <> __device__ __forceinline__ double dev_max<double>(double a, double b) { return fmax(a, b); }

// The running maximum starts at -1e38 like the reference kernel
// (edge_softmax.cu:271); fmax ignores NaN operands.
constexpr double kMaxSeed = -1e38;

// One thread per (segment, head); edges of a segment are contiguous in x/y.
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void seg_softmax_fwd(const int32_t* indptr, int64_t n_seg,
                                                         int64_t n_edges, const T* x,
                                                         int64_t ldx, int heads, T* y,
                                                         int64_t ldy) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= n_seg * heads) return;
  const int64_t s = t / heads;
  const int h = static_cast<int>(t - s * heads);
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  T mx = static_cast<T>(kMaxSeed);
  for (int64_t e = lb; e < le; ++e) mx = dev_max<T>(mx, x[e * ldx + h]);
  T sum = 0;
  for (int64_t e = lb; e < le; ++e) sum += dev_exp<T>(x[e * ldx + h] - mx);
  if (MODE == 0) {
    const T inv = static_cast<T>(1) / sum;
    for (int64_t e = lb; e < le; ++e) y[e * ldy + h] = dev_exp<T>(x[e * ldx + h] - mx) * inv;
  } else {
    for (int64_t e = lb; e < le; ++e) y[e * ldy + h] = dev_exp<T>(x[e * ldx + h] - mx) / sum;
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void seg_softmax_bwd(const int32_t* indptr, int64_t n_seg,
                                                         int64_t n_edges, const T* dy,
                                                         int64_t lddy, const T* y, int64_t ldy,
                                                         int heads, T* dx, int64_t lddx) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= n_seg * heads) return;
  const int64_t s = t / heads;
  const int h = static_cast<int>(t - s * heads);
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  T acc = 0;
  for (int64_t e = lb; e < le; ++e) acc += y[e * ldy + h] * dy[e * lddy + h];
  for (int64_t e = lb; e < le; ++e) {
    const T yv = y[e * ldy + h];
    dx[e * lddx + h] = yv * (dy[e * lddy + h] - acc);
  }
}

// Group kernels (float32, rows of exactly `heads` values, heads in {1, 2, 4, 8, 16}): a group
// of W = max(4, heads) lanes per segment, 64 / W segments per wave in flight. A segment's
// deg*heads values are contiguous, so the group reads them coalesced: lane l takes values
// l, l+W, ... (all of head l % heads, as heads divides W), keeps the first kRowCache in
// registers, and the head's max and sum are combined across the group's lanes of that head
// by xor swizzles (a tree order rather than the reference's edge order; the results agree
// to rounding).
constexpr int kRowLanes = 16;   // widest group
constexpr int kRowCache = 4;

template <int M>
__device__ __forceinline__ float swz_xor(float v) {
  // ds_swizzle bit mode: lane' = ((lane & 0x1f) | 0) ^ M within each group of 32 lanes
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (M << 10)));
}

// Combine over the lanes of a W-lane group that share lane % H.
template <int H, int W, bool MAX>
__device__ __forceinline__ float row_reduce(float v) {
  if constexpr (W > 8 && H <= 8) v = MAX ? fmaxf(v, swz_xor<8>(v)) : v + swz_xor<8>(v);
  if constexpr (W > 4 && H <= 4) v = MAX ? fmaxf(v, swz_xor<4>(v)) : v + swz_xor<4>(v);
  if constexpr (W > 2 && H <= 2) v = MAX ? fmaxf(v, swz_xor<2>(v)) : v + swz_xor<2>(v);
  if constexpr (W > 1 && H <= 1) v = MAX ? fmaxf(v, swz_xor<1>(v)) : v + swz_xor<1>(v);
  return v;
}

constexpr int group_lanes(int H) { return H < 4 ? 4 : H; }

// Zeros in the rows before indptr[0] and from indptr[n_seg] on (`heads` values a row of
// exactly `heads`), spread over every thread of the grid.
__device__ __forceinline__ void zero_outside(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                                             int heads, float* out) {
  int64_t a = indptr[0], b = indptr[n_seg];
  a = a < 0 ? 0 : (a > n_edges ? n_edges : a);
  b = b < a ? a : (b > n_edges ? n_edges : b);
  const int64_t head = a * heads, tail = (n_edges - b) * heads;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < head + tail; i += stride)
    out[i < head ? i : i - head + b * heads] = 0.f;
}

struct RowSeg {
  int64_t base, n;  // values [base, base + n) of the segment
  bool ok;
};

__device__ __forceinline__ RowSeg row_segment(const int32_t* indptr, int64_t s, int64_t n_edges,
                                              int heads) {
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  RowSeg r{lb * heads, (le - lb) * heads, le > lb};
  return r;
}

template <int H, int MODE>
__global__ __launch_bounds__(kBlock) void seg_softmax_fwd_rows(const int32_t* indptr,
                                                              int64_t n_seg, int64_t n_edges,
                                                              const float* x, float* y) {
  constexpr int W = group_lanes(H), G = kBlock / W;
  zero_outside(indptr, n_seg, n_edges, H, y);
  const int l = threadIdx.x & (W - 1);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * G;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * G + threadIdx.x / W; s < n_seg; s += stride) {
    const RowSeg g = row_segment(indptr, s, n_edges, H);
    if (!g.ok) continue;  // the whole group skips
    const float* xs = x + g.base;
    float v[kRowCache];
    float mx = static_cast<float>(kMaxSeed);
#pragma unroll
    for (int c = 0; c < kRowCache; ++c) {
      const int64_t i = l + W * c;
      v[c] = i < g.n ? xs[i] : static_cast<float>(kMaxSeed);
      mx = fmaxf(mx, v[c]);
    }
    for (int64_t i = l + W * kRowCache; i < g.n; i += W) mx = fmaxf(mx, xs[i]);
    mx = row_reduce<H, W, true>(mx);
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < kRowCache; ++c) {   // the cached values become their exponentials
      v[c] = expf(v[c] - mx);
      if (l + W * c < g.n) sum += v[c];
    }
    for (int64_t i = l + W * kRowCache; i < g.n; i += W) sum += expf(xs[i] - mx);
    sum = row_reduce<H, W, false>(sum);
    const float inv = 1.f / sum;
    float* ys = y + g.base;
#pragma unroll
    for (int c = 0; c < kRowCache; ++c) {
      const int64_t i = l + W * c;
      if (i < g.n) ys[i] = MODE == 0 ? v[c] * inv : v[c] / sum;
    }
    for (int64_t i = l + W * kRowCache; i < g.n; i += W)
      ys[i] = MODE == 0 ? expf(xs[i] - mx) * inv : expf(xs[i] - mx) / sum;
  }
}

template <int H>
__global__ __launch_bounds__(kBlock) void seg_softmax_bwd_rows(const int32_t* indptr,
                                                              int64_t n_seg, int64_t n_edges,
                                                              const float* dy, const float* y,
                                                              float* dx) {
  constexpr int W = group_lanes(H), G = kBlock / W;
  zero_outside(indptr, n_seg, n_edges, H, dx);
  const int l = threadIdx.x & (W - 1);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * G;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * G + threadIdx.x / W; s < n_seg; s += stride) {
    const RowSeg g = row_segment(indptr, s, n_edges, H);
    if (!g.ok) continue;
    const float* ys = y + g.base;
    const float* ds = dy + g.base;
    float yv[kRowCache], gv[kRowCache];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kRowCache; ++c) {
      const int64_t i = l + W * c;
      yv[c] = i < g.n ? ys[i] : 0.f;
      gv[c] = i < g.n ? ds[i] : 0.f;
      acc += yv[c] * gv[c];
    }
    for (int64_t i = l + W * kRowCache; i < g.n; i += W) acc += ys[i] * ds[i];
    acc = row_reduce<H, W, false>(acc);
    float* xs = dx + g.base;
#pragma unroll
    for (int c = 0; c < kRowCache; ++c) {
      const int64_t i = l + W * c;
      if (i < g.n) xs[i] = yv[c] * (gv[c] - acc);
    }
    for (int64_t i = l + W * kRowCache; i < g.n; i += W) xs[i] = ys[i] * (ds[i] - acc);
  }
}

// Zeros in the first `width` values of the rows no segment covers: [0, indptr[0]) and
// [indptr[n_seg], n_edges) (every edge between the two lies in some segment, whatever the
// offsets); with indptr NULL every row. Rows are `ld` values apart.
template <typename T>
__global__ __launch_bounds__(kBlock) void zero_uncovered(const int32_t* indptr, int64_t n_seg,
                                                        int64_t n_edges, int64_t width,
                                                        int64_t ld, T* out) {
  int64_t a = n_edges, b = n_edges;
  if (indptr) {
    a = indptr[0];
    b = indptr[n_seg];
    a = a < 0 ? 0 : (a > n_edges ? n_edges : a);
    b = b < a ? a : (b > n_edges ? n_edges : b);
  }
  const int64_t head = a * width, tail = (n_edges - b) * width;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < head + tail;
       i += stride) {
    const int64_t j = i < head ? i : i - head + b * width;
    const int64_t r = j / width;
    out[r * ld + (j - r * width)] = 0;
  }
}

int row_grid(int64_t n_seg, int heads = kRowLanes) {
  const int64_t b = ceil_div(n_seg, kBlock / group_lanes(heads));
  return static_cast<int>(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

// Grouped softmax: one workgroup per batch, one thread per (edge-in-batch, head).
// Each thread scans the edges of its batch in order and keeps those with its key, so
// every member of a group computes the same max and sum in the same order.

__global__ __launch_bounds__(kBlock) void group_softmax_fwd(const int64_t* bptr, int64_t n_batch,
                                                           const int64_t* key, int64_t ld_key,
                                                           int64_t n_edges, const float* x,
                                                           int64_t ldx, int heads, float* y,
                                                           int64_t ldy) {
  const int64_t b = blockIdx.x;
  int64_t lb = bptr[b], le = bptr[b + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  const int64_t cnt = le > lb ? le - lb : 0;
  const int64_t* key_row = key + b * ld_key;
  const int64_t lim = cnt < ld_key ? cnt : ld_key;
  for (int64_t t = threadIdx.x; t < lim * heads; t += kBlock) {
    const int64_t j = t / heads;
    const int h = static_cast<int>(t - j * heads);
    const int64_t k = key_row[j];
    if (k < 0 || k >= ld_key) continue;
    float mx = static_cast<float>(kMaxSeed);
    for (int64_t i = 0; i < lim; ++i)
      if (key_row[i] == k) mx = fmaxf(mx, x[(lb + i) * ldx + h]);
    float sum = 0.f;
    for (int64_t i = 0; i < lim; ++i)
      if (key_row[i] == k) sum += expf(x[(lb + i) * ldx + h] - mx);
    y[(lb + j) * ldy + h] = expf(x[(lb + j) * ldx + h] - mx) / sum;
  }
}

__global__ __launch_bounds__(kBlock) void group_softmax_bwd(const int64_t* bptr, int64_t n_batch,
                                                           const int64_t* key, int64_t ld_key,
                                                           int64_t n_edges, const float* dy,
                                                           int64_t lddy, const float* y,
                                                           int64_t ldy, int heads, float* dx,
                                                           int64_t lddx) {
  const int64_t b = blockIdx.x;
  int64_t lb = bptr[b], le = bptr[b + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  const int64_t cnt = le > lb ? le - lb : 0;
  const int64_t* key_row = key + b * ld_key;
  const int64_t lim = cnt < ld_key ? cnt : ld_key;
  for (int64_t t = threadIdx.x; t < lim * heads; t += kBlock) {
    const int64_t j = t / heads;
    const int h = static_cast<int>(t - j * heads);
    const int64_t k = key_row[j];
    if (k < 0 || k >= ld_key) continue;
    float acc = 0.f;
    for (int64_t i = 0; i < lim; ++i)
      if (key_row[i] == k) acc += y[(lb + i) * ldy + h] * dy[(lb + i) * lddy + h];
    dx[(lb + j) * lddx + h] = y[(lb + j) * ldy + h] * (dy[(lb + j) * lddy + h] - acc);
  }
}

template <typename T>
void launch_zero_uncovered(const int32_t* indptr, int64_t n_seg, int64_t n_edges, int64_t width,
                           int64_t ld, T* out, hipStream_t stream) {
  const int blocks = indptr ? 64 : row_grid(ceil_div(n_edges * width, kRowLanes));
  hipLaunchKernelGGL((zero_uncovered<T>), dim3(blocks), dim3(kBlock), 0, stream, indptr, n_seg,
                     n_edges, width, ld, out);
}

template <int MODE>
void launch_fwd_rows(int heads, const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                     const float* x, float* y, hipStream_t stream) {
  const dim3 grid(row_grid(n_seg, heads)), block(kBlock);
  switch (heads) {
    case 1: hipLaunchKernelGGL((seg_softmax_fwd_rows<1, MODE>), grid, block, 0, stream, indptr, n_seg, n_edges, x, y); break;
    case 2: hipLaunchKernelGGL((seg_softmax_fwd_rows<2, MODE>), grid, block, 0, stream, indptr, n_seg, n_edges, x, y); break;
    case 4: hipLaunchKernelGGL((seg_softmax_fwd_rows<4, MODE>), grid, block, 0, stream, indptr, n_seg, n_edges, x, y); break;
    case 8: hipLaunchKernelGGL((seg_softmax_fwd_rows<8, MODE>), grid, block, 0, stream, indptr, n_seg, n_edges, x, y); break;
    default: hipLaunchKernelGGL((seg_softmax_fwd_rows<16, MODE>), grid, block, 0, stream, indptr, n_seg, n_edges, x, y); break;
  }
}

bool rows_fit(int heads) { return heads == 1 || heads == 2 || heads == 4 || heads == 8 || heads == 16; }

template <typename T>
int softmax_fwd(const int32_t* indptr, int64_t n_seg, int64_t n_edges, const T* x, int64_t ldx,
                int heads, T* y, int64_t ldy, int mode, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || heads < 0 || (mode != 0 && mode != 1)) return FA_EINVAL;
  if (heads == 0 || n_edges == 0) return FA_OK;
  if (!y || ldy < heads) return FA_EINVAL;
  if (n_seg == 0) {  // nothing covered: zeros
    launch_zero_uncovered<T>(nullptr, 0, n_edges, heads, ldy, y, stream);
    return launch_status();
  }
  if (!indptr || !x || ldx < heads) return FA_EINVAL;
  if constexpr (sizeof(T) == 4) {
    if (ldx == heads && ldy == heads && rows_fit(heads)) {  // the group kernels zero outside too
      if (mode == 0) launch_fwd_rows<0>(heads, indptr, n_seg, n_edges, x, y, stream);
      else launch_fwd_rows<1>(heads, indptr, n_seg, n_edges, x, y, stream);
      return launch_status();
    }
  }
  launch_zero_uncovered<T>(indptr, n_seg, n_edges, heads, ldy, y, stream);
  const int64_t threads = n_seg * heads;
  if (mode == 0)
    hipLaunchKernelGGL((seg_softmax_fwd<T, 0>), dim3(ceil_div(threads, kBlock)), dim3(kBlock), 0,
                       stream, indptr, n_seg, n_edges, x, ldx, heads, y, ldy);
  else
    hipLaunchKernelGGL((seg_softmax_fwd<T, 1>), dim3(ceil_div(threads, kBlock)), dim3(kBlock), 0,
                       stream, indptr, n_seg, n_edges, x, ldx, heads, y, ldy);
  return launch_status();
}

template <typename T>
int softmax_bwd(const int32_t* indptr, int64_t n_seg, int64_t n_edges, const T* dy, int64_t lddy,
                const T* y, int64_t ldy, int heads, T* dx, int64_t lddx, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || heads < 0) return FA_EINVAL;
  if (heads == 0 || n_edges == 0) return FA_OK;
  if (!dx || lddx < heads) return FA_EINVAL;
  if (n_seg == 0) {
    launch_zero_uncovered<T>(nullptr, 0, n_edges, heads, lddx, dx, stream);
    return launch_status();
  }
  if (!indptr || !dy || !y || lddy < heads || ldy < heads) return FA_EINVAL;
  if constexpr (sizeof(T) == 4) {
    if (lddy == heads && ldy == heads && lddx == heads && rows_fit(heads)) {
      const dim3 grid(row_grid(n_seg, heads)), block(kBlock);
      switch (heads) {
        case 1: hipLaunchKernelGGL((seg_softmax_bwd_rows<1>), grid, block, 0, stream, indptr, n_seg, n_edges, dy, y, dx); break;
        case 2: hipLaunchKernelGGL((seg_softmax_bwd_rows<2>), grid, block, 0, stream, indptr, n_seg, n_edges, dy, y, dx); break;
        case 4: hipLaunchKernelGGL((seg_softmax_bwd_rows<4>), grid, block, 0, stream, indptr, n_seg, n_edges, dy, y, dx); break;
        case 8: hipLaunchKernelGGL((seg_softmax_bwd_rows<8>), grid, block, 0, stream, indptr, n_seg, n_edges, dy, y, dx); break;
        default: hipLaunchKernelGGL((seg_softmax_bwd_rows<16>), grid, block, 0, stream, indptr, n_seg, n_edges, dy, y, dx); break;
      }
      return launch_status();
    }
  }
  launch_zero_uncovered<T>(indptr, n_seg, n_edges, heads, lddx, dx, stream);
  const int64_t threads = n_seg * heads;
  hipLaunchKernelGGL((seg_softmax_bwd<T>), dim3(ceil_div(threads, kBlock)), dim3(kBlock), 0,
                     stream, indptr, n_seg, n_edges, dy, lddy, y, ldy, heads, dx, lddx);
  return launch_status();
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_edge_softmax_fwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                                       const float* x, int64_t ldx, int32_t heads, float* y,
                                       int64_t ldy, int32_t mode, hipStream_t stream) {
  return softmax_fwd<float>(indptr, n_seg, n_edges, x, ldx, heads, y, ldy, mode, stream);
}

extern "C" int fa_edge_softmax_fwd_f64(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                                       const double* x, int64_t ldx, int32_t heads, double* y,
                                       int64_t ldy, int32_t mode, hipStream_t stream) {
  return softmax_fwd<double>(indptr, n_seg, n_edges, x, ldx, heads, y, ldy, mode, stream);
}

extern "C" int fa_edge_softmax_bwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                                       const float* dy, int64_t lddy, const float* y,
                                       int64_t ldy, int32_t heads, float* dx, int64_t lddx,
                                       hipStream_t stream) {
  return softmax_bwd<float>(indptr, n_seg, n_edges, dy, lddy, y, ldy, heads, dx, lddx, stream);
}

extern "C" int fa_edge_softmax_bwd_f64(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                                       const double* dy, int64_t lddy, const double* y,
                                       int64_t ldy, int32_t heads, double* dx, int64_t lddx,
                                       hipStream_t stream) {
  return softmax_bwd<double>(indptr, n_seg, n_edges, dy, lddy, y, ldy, heads, dx, lddx, stream);
}

extern "C" int fa_group_softmax_fwd_f32(const int64_t* batch_ptr, int64_t n_batch,
                                        const int64_t* key, int64_t ld_key, int64_t n_edges,
                                        const float* x, int64_t ldx, int32_t heads, float* y,
                                        int64_t ldy, hipStream_t stream) {
  if (n_batch < 0 || ld_key < 0 || n_edges < 0 || heads < 0) return FA_EINVAL;
  if (n_batch == 0 || heads == 0 || ld_key == 0) return FA_OK;
  if (!batch_ptr || !key || !x || !y || ldx < heads || ldy < heads) return FA_EINVAL;
  if (n_batch > INT32_MAX) return FA_EUNSUPPORTED;
  hipLaunchKernelGGL(group_softmax_fwd, dim3(n_batch), dim3(kBlock), 0, stream, batch_ptr, n_batch,
                     key, ld_key, n_edges, x, ldx, heads, y, ldy);
  return launch_status();
}

extern "C" int fa_group_softmax_bwd_f32(const int64_t* batch_ptr, int64_t n_batch,
                                        const int64_t* key, int64_t ld_key, int64_t n_edges,
                                        const float* dy, int64_t lddy, const float* y,
                                        int64_t ldy, int32_t heads, float* dx, int64_t lddx,
                                        hipStream_t stream) {
  if (n_batch < 0 || ld_key < 0 || n_edges < 0 || heads < 0) return FA_EINVAL;
  if (n_batch == 0 || heads == 0 || ld_key == 0) return FA_OK;
  if (!batch_ptr || !key || !dy || !y || !dx || lddy < heads || ldy < heads || lddx < heads)
    return FA_EINVAL;
  if (n_batch > INT32_MAX) return FA_EUNSUPPORTED;
  hipLaunchKernelGGL(group_softmax_bwd, dim3(n_batch), dim3(kBlock), 0, stream, batch_ptr,
                     n_batch, key, ld_key, n_edges, dy, lddy, y, ldy, heads, dx, lddx);
  return launch_status();
}
