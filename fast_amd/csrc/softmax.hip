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
int softmax_fwd(const int32_t* indptr, int64_t n_seg, int64_t n_edges, const T* x, int64_t ldx,
                int heads, T* y, int64_t ldy, int mode, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || heads < 0 || (mode != 0 && mode != 1)) return FA_EINVAL;
  if (n_seg == 0 || heads == 0) return FA_OK;
  if (!indptr || !x || !y || ldx < heads || ldy < heads) return FA_EINVAL;
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
  if (n_seg == 0 || heads == 0) return FA_OK;
  if (!indptr || !dy || !y || !dx || lddy < heads || ldy < heads || lddx < heads) return FA_EINVAL;
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
