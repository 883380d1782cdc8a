// Fused LeakyReLU + segment softmax + dropout + weighted aggregation over pre-computed
// per-edge scores and values (the operator pair forward/backward_fused_attn).
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kColSlots = 4;
constexpr int kColTile = kWave * kColSlots;
constexpr float kMaxSeed = -1e38f;

__device__ __forceinline__ float keep_factor(const float* mask, int64_t idx, float p) {
  // Kept entries are scaled by 1/(1-p) evaluated in double, as the reference does
  // (fused_attention.cu:285-287); dropped entries contribute 0.
  if (mask == nullptr) return 1.f;
  return mask[idx] > p ? static_cast<float>(1.0 / (1.0 - static_cast<double>(p))) : 0.f;
}

// One wave per segment. Lanes < heads hold the per-head max / sum; every lane then owns
// output columns c = col0 + lane + 64k of the destination row.
__global__ __launch_bounds__(kBlock) void fused_attn_fwd(const int32_t* indptr, int64_t n_seg,
                                                        const int64_t* dst, const int64_t* src,
                                                        int64_t n_edges, int64_t n_dst,
                                                        const float* score, const float* V,
                                                        int64_t n_v, int heads, int dh,
                                                        float slope, float p, const float* mask,
                                                        float* attn, float* out) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (s >= n_seg) return;
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  if (le <= lb) return;
  const int lane = lane_id();
  const int dim = heads * dh;
  float mx = kMaxSeed, sm = 0.f;
  if (lane < heads) {
    for (int64_t e = lb; e < le; ++e) mx = fmaxf(mx, leaky(score[e * heads + lane], slope));
    for (int64_t e = lb; e < le; ++e) sm += expf(leaky(score[e * heads + lane], slope) - mx);
    for (int64_t e = lb; e < le; ++e)
      attn[e * heads + lane] = expf(leaky(score[e * heads + lane], slope) - mx) / sm;
  }
  const int64_t d = dst[lb];
  if (d < 0 || d >= n_dst) return;
  for (int col0 = 0; col0 < dim; col0 += kColTile) {
    float acc[kColSlots] = {0.f, 0.f, 0.f, 0.f};
    int hk[kColSlots];
    float mxk[kColSlots], smk[kColSlots];
#pragma unroll
    for (int k = 0; k < kColSlots; ++k) {
      const int c = col0 + lane + k * kWave;
      hk[k] = c < dim ? c / dh : 0;
      mxk[k] = __shfl(mx, hk[k], kWave);
      smk[k] = __shfl(sm, hk[k], kWave);
    }
    for (int64_t e = lb; e < le; ++e) {
      const int64_t row = src[e] - n_dst;
      if (row < 0 || row >= n_v) continue;
#pragma unroll
      for (int k = 0; k < kColSlots; ++k) {
        const int c = col0 + lane + k * kWave;
        if (c >= dim) continue;
        const int64_t ai = e * heads + hk[k];
        const float a = expf(leaky(score[ai], slope) - mxk[k]) / smk[k];
        const float w = mask ? (keep_factor(mask, ai, p) != 0.f
                                    ? static_cast<float>(static_cast<double>(a) /
                                                         (1.0 - static_cast<double>(p)))
                                    : 0.f)
                             : a;
        acc[k] = fmaf(w, V[row * dim + c], acc[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < kColSlots; ++k) {
      const int c = col0 + lane + k * kWave;
      if (c < dim) out[d * dim + c] = acc[k];
    }
  }
}

// One wave per segment. Pass 1 scatters grad_V and records da[e,h] = keep*dout.V in
// d_act (each lane h < heads writes and later re-reads only its own entries); pass 2
// turns da into the softmax-input gradient.
__global__ __launch_bounds__(kBlock) void fused_attn_bwd(const int32_t* indptr, int64_t n_seg,
                                                        const int64_t* dst, const int64_t* src,
                                                        int64_t n_edges, int64_t n_dst,
                                                        int64_t n_src, const float* dout,
                                                        const float* V, int64_t n_v,
                                                        const float* attn, const float* mask,
                                                        int heads, int dh, float p, float* d_act,
                                                        float* grad_V) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (s >= n_seg) return;
  int64_t lb = indptr[s], le = indptr[s + 1];
  lb = lb < 0 ? 0 : lb;
  le = le > n_edges ? n_edges : le;
  if (le <= lb) return;
  const int64_t d = dst[lb];
  if (d < 0 || d >= n_dst) return;
  const int lane = lane_id();
  const int dim = heads * dh;
  float tsum = 0.f;  // lane h < heads: sum_e attn*da for head h
  for (int64_t e = lb; e < le; ++e) {
    const int64_t sr = src[e];
    const int64_t row = sr - n_dst;
    const bool valid = row >= 0 && row < n_v && sr < n_src;
    float da_mine = 0.f;
    for (int col0 = 0; col0 < dim; col0 += kColTile) {
      float part[kColSlots];
      int hk[kColSlots];
#pragma unroll
      for (int k = 0; k < kColSlots; ++k) {
        const int c = col0 + lane + k * kWave;
        part[k] = 0.f;
        hk[k] = c < dim ? c / dh : -1;
        if (c < dim && valid) {
          const int64_t ai = e * heads + hk[k];
          const float a = attn[ai];
          const float kf = keep_factor(mask, ai, p);
          const float g = dout[d * dim + c];
          atomicAdd(grad_V + row * dim + c, a * kf * g);
          part[k] = kf * g * V[row * dim + c];
        }
      }
      for (int h = 0; h < heads; ++h) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < kColSlots; ++k) v += (hk[k] == h) ? part[k] : 0.f;
        const float tot = wave_sum(v);
        if (lane == h) da_mine += tot;
      }
    }
    if (lane < heads) {
      d_act[e * heads + lane] = da_mine;
      tsum = fmaf(attn[e * heads + lane], da_mine, tsum);
    }
  }
  if (lane < heads) {
    for (int64_t e = lb; e < le; ++e) {
      const int64_t ai = e * heads + lane;
      const float da = d_act[ai];
      d_act[ai] = attn[ai] * (da - tsum);
    }
  }
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_fused_attn_fwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                                     const int64_t* src, int64_t n_edges, int64_t n_dst,
                                     const float* score, const float* V, int32_t heads,
                                     int32_t dh, float slope, float p, const float* mask,
                                     float* attn, float* out, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || n_dst < 0 || heads < 0 || dh < 0) return FA_EINVAL;
  if (heads > kWave) return FA_EUNSUPPORTED;
  if (n_seg == 0 || heads == 0) return FA_OK;
  if (!indptr || !dst || !src || !score || !attn || (dh > 0 && (!V || !out))) return FA_EINVAL;
  hipLaunchKernelGGL(fused_attn_fwd, dim3(ceil_div(n_seg, kWavesPerBlock)), dim3(kBlock), 0,
                     stream, indptr, n_seg, dst, src, n_edges, n_dst, score, V, n_edges, heads,
                     dh, slope, p, mask, attn, out);
  return launch_status();
}

extern "C" int fa_fused_attn_bwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                                     const int64_t* src, int64_t n_edges, int64_t n_dst,
                                     int64_t n_src, const float* dout, const float* V,
                                     const float* attn, const float* mask, int32_t heads,
                                     int32_t dh, float p, float* d_act, float* grad_V,
                                     hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || n_dst < 0 || heads < 0 || dh < 0) return FA_EINVAL;
  if (heads > kWave) return FA_EUNSUPPORTED;
  if (n_seg == 0 || heads == 0) return FA_OK;
  if (!indptr || !dst || !src || !attn || !d_act || (dh > 0 && (!V || !dout || !grad_V)))
    return FA_EINVAL;
  hipLaunchKernelGGL(fused_attn_bwd, dim3(ceil_div(n_seg, kWavesPerBlock)), dim3(kBlock), 0,
                     stream, indptr, n_seg, dst, src, n_edges, n_dst, n_src, dout, V, n_edges,
                     attn, mask, heads, dh, p, d_act, grad_V);
  return launch_status();
}
