// Fused epilogue of the temporal attention layer (layers.py:224-237):
//   u   = r1 + r2 + bias                (w_out([agg | h_dst]) from its two halves and bias)
//   y   = relu(dropout(u))              (counter-hash dropout, multiplier 1/(1-p) or 0)
//   out = (y - mean(y)) * rstd * gamma + beta,   rstd = 1/sqrt(var(y) + eps)   (LayerNorm)
// and its backward. One wave per row (grid-stride); lane l holds columns l, l+64, ... of the
// row (coalesced), so rows up to 64*kMaxPer columns wide are handled in registers. Row sums
// use the wave reductions of fa_common.hpp. The weight / bias gradients of the LayerNorm
// (and of the bias of u) are accumulated per wave, combined per workgroup in a fixed order
// and summed over workgroups by a second kernel (no float atomics).
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kMaxPer = 4;          // columns per lane: rows up to 256 wide
constexpr int kEpiMaxBlocks = 1024;  // grid cap (rows of the weight-gradient partials)
constexpr int kEpiRowBlocks = 2048;  // grid cap of the forward's half-wave form (8 waves per SIMD)

struct EpiParams {
  int64_t n;
  int d;
  const float* r1; int64_t ld1;
  const float* r2; int64_t ld2;     // may be null
  const float* bias;                // [d] added to u, may be null
  const float* gamma;
  const float* beta;
  float eps;
  int drop;                         // apply the hashed dropout
  uint64_t seed;
  float p, scale;
  float* out;
  float* y;                         // [n][d] saved relu(dropout(u))
  float* stats;                     // [n][2] mean, rstd
};

template <int PER>
__global__ __launch_bounds__(kBlock) void epilogue_fwd(EpiParams P) {
  const int lane = lane_id();
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const float inv_d = 1.f / static_cast<float>(P.d);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       r < P.n; r += total) {
    float v[PER];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + i * kWave;
      float u = 0.f;
      if (c < P.d) {
        u = P.r1[r * P.ld1 + c];
        if (P.r2) u += P.r2[r * P.ld2 + c];
        if (P.bias) u += P.bias[c];
        if (P.drop) u *= drop_mult(P.seed, static_cast<uint64_t>(r * P.d + c), P.p, P.scale);
        u = u > 0.f ? u : 0.f;
      }
      v[i] = u;
      s += u;
    }
    const float mean = wave_sum(s) * inv_d;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + i * kWave;
      const float dv = c < P.d ? v[i] - mean : 0.f;
      q += dv * dv;
    }
    const float rstd = 1.f / sqrtf(wave_sum(q) * inv_d + P.eps);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + i * kWave;
      if (c < P.d) {
        P.y[r * P.d + c] = v[i];
        P.out[r * P.d + c] = (v[i] - mean) * rstd * P.gamma[c] + P.beta[c];
      }
    }
    if (lane == 0) {
      P.stats[2 * r] = mean;
      P.stats[2 * r + 1] = rstd;
    }
  }
}

// Rows of whole chunks (d % 4 == 0, d <= 128, 16-byte aligned rows): a half-wave per row,
// lane l holding columns 4l .. 4l+3 as one float4; two rows per half-wave and iteration, so
// four rows' loads are in flight per wave.
constexpr int kEpiRows = 2;   // rows per half-wave and iteration

__device__ __forceinline__ float4 f4_load(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Non-temporal access for rows read or written once here and not again soon (the w_out
// products, the saved pre-norm rows, the upstream gradient), so that they leave the caches
// first; the layer output and the input gradient, read next, keep the default policy.
typedef float nt4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 f4_load_nt(const float* p) {
  const nt4 v = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void f4_store_nt(float* p, const float4& x) {
  const nt4 v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<nt4*>(p));
}

__global__ __launch_bounds__(kBlock) void epilogue_fwd_h(EpiParams P) {
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int c = 4 * hl;
  const bool on = c < P.d;
  const float inv_d = 1.f / static_cast<float>(P.d);
  const float4 gm = on ? f4_load(P.gamma + c) : f4_zero();
  const float4 bt = on ? f4_load(P.beta + c) : f4_zero();
  const float4 bs = (on && P.bias) ? f4_load(P.bias + c) : f4_zero();
  const int64_t slots = static_cast<int64_t>(gridDim.x) * kWavesPerBlock * 2;  // half-waves
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave)) * 2 + half;
  // the loop runs on the wave's first row, so both halves take every iteration (the
  // half-wave sums need the whole wave)
  for (int64_t rb = first - half; rb < P.n; rb += kEpiRows * slots) {
    const int64_t r0 = rb + half;
    float4 u[kEpiRows];
#pragma unroll
    for (int i = 0; i < kEpiRows; ++i) {
      const int64_t r = r0 + i * slots;
      float4 a = f4_zero();
      if (on && r < P.n) {
        a = f4_load_nt(P.r1 + r * P.ld1 + c);
        if (P.r2) {
          const float4 b = f4_load_nt(P.r2 + r * P.ld2 + c);
          a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
      }
      u[i] = a;
    }
#pragma unroll
    for (int i = 0; i < kEpiRows; ++i) {
      const int64_t r = r0 + i * slots;
      float4 a = u[i];
      a.x += bs.x; a.y += bs.y; a.z += bs.z; a.w += bs.w;
      if (P.drop) {
        const uint64_t e = static_cast<uint64_t>(r * P.d + c);
        a.x *= drop_mult(P.seed, e, P.p, P.scale);
        a.y *= drop_mult(P.seed, e + 1, P.p, P.scale);
        a.z *= drop_mult(P.seed, e + 2, P.p, P.scale);
        a.w *= drop_mult(P.seed, e + 3, P.p, P.scale);
      }
      a = make_float4(a.x > 0.f ? a.x : 0.f, a.y > 0.f ? a.y : 0.f, a.z > 0.f ? a.z : 0.f,
                      a.w > 0.f ? a.w : 0.f);
      if (!on) a = f4_zero();
      const float mean = half_sum(a.x + a.y + a.z + a.w) * inv_d;
      const float4 dv = on ? make_float4(a.x - mean, a.y - mean, a.z - mean, a.w - mean) : f4_zero();
      const float rstd = 1.f / sqrtf(half_sum(dv.x * dv.x + dv.y * dv.y + dv.z * dv.z + dv.w * dv.w) * inv_d + P.eps);
      if (on && r < P.n) {
        f4_store_nt(P.y + r * P.d + c, a);
        *reinterpret_cast<float4*>(P.out + r * P.d + c) =
            make_float4(dv.x * rstd * gm.x + bt.x, dv.y * rstd * gm.y + bt.y,
                        dv.z * rstd * gm.z + bt.z, dv.w * rstd * gm.w + bt.w);
      }
      if (hl == 0 && r < P.n) {
        P.stats[2 * r] = mean;
        P.stats[2 * r + 1] = rstd;
      }
    }
  }
}

struct EpiBwdParams {
  int64_t n;
  int d;
  const float* dout;
  const float* y;
  const float* stats;
  const float* gamma;
  float scale;                      // dropout multiplier of kept entries (1 without dropout)
  float* du;
  int nsum;                         // 2, or 3 with the bias gradient
  float* partial;                   // [grid][nsum][d]: sums of dout*yhat, dout (and du)
};

template <int PER>
__global__ __launch_bounds__(kBlock) void epilogue_bwd(EpiBwdParams P) {
  __shared__ float red[kWavesPerBlock][3][kMaxPer * kWave];
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const float inv_d = 1.f / static_cast<float>(P.d);
  float gg[PER], gb[PER], gu[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) gg[i] = gb[i] = gu[i] = 0.f;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave; r < P.n; r += total) {
    const float mean = P.stats[2 * r], rstd = P.stats[2 * r + 1];
    float yh[PER], g[PER], yv[PER];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + i * kWave;
      float dy = 0.f, yy = 0.f, gm = 0.f;
      if (c < P.d) {
        dy = P.dout[r * P.d + c];
        yy = P.y[r * P.d + c];
        gm = P.gamma[c];
      }
      yv[i] = yy;
      yh[i] = c < P.d ? (yy - mean) * rstd : 0.f;
      g[i] = dy * gm;
      gg[i] = fmaf(dy, yh[i], gg[i]);
      gb[i] += dy;
      s1 += g[i];
      s2 = fmaf(g[i], yh[i], s2);
    }
    const float m1 = wave_sum(s1) * inv_d;
    const float m2 = wave_sum(s2) * inv_d;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + i * kWave;
      if (c < P.d) {
        const float dyv = rstd * (g[i] - m1 - yh[i] * m2);
        // y = relu(u * mult): dy/du = mult where y > 0, else 0
        const float du = yv[i] > 0.f ? dyv * P.scale : 0.f;
        P.du[r * P.d + c] = du;
        gu[i] += du;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    red[wave][0][lane + i * kWave] = gg[i];
    red[wave][1][lane + i * kWave] = gb[i];
    red[wave][2][lane + i * kWave] = gu[i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < P.nsum * P.d; idx += kBlock) {
    const int which = idx / P.d;
    const int c = idx - which * P.d;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) s += red[w][which][c];
    P.partial[(static_cast<int64_t>(blockIdx.x) * P.nsum + which) * P.d + c] = s;
  }
}

// The backward for rows of whole chunks up to 128 wide (aligned): a half-wave per row, lane
// l holding columns 4l .. 4l+3; the column sums are kept per lane, combined over the
// workgroup's eight half-waves in a fixed order.
__global__ __launch_bounds__(kBlock) void epilogue_bwd_h(EpiBwdParams P) {
  __shared__ float4 red[2 * kWavesPerBlock][3][kHalf];
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int c = 4 * hl;
  const bool on = c < P.d;
  const float inv_d = 1.f / static_cast<float>(P.d);
  const float4 gm = on ? f4_load(P.gamma + c) : f4_zero();
  float4 gg = f4_zero(), gb = f4_zero(), gu = f4_zero();
  const int64_t slots = static_cast<int64_t>(gridDim.x) * kWavesPerBlock * 2;
  // the loop runs on the wave's first row, so both halves take every iteration
  for (int64_t rb = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave) * 2; rb < P.n; rb += slots) {
    const int64_t r = rb + half;
    const bool ok = on && r < P.n;
    const float mean = r < P.n ? P.stats[2 * r] : 0.f, rstd = r < P.n ? P.stats[2 * r + 1] : 0.f;
    const float4 dy = ok ? f4_load_nt(P.dout + r * P.d + c) : f4_zero();
    const float4 yy = ok ? f4_load_nt(P.y + r * P.d + c) : f4_zero();
    const float4 yh = ok ? make_float4((yy.x - mean) * rstd, (yy.y - mean) * rstd, (yy.z - mean) * rstd,
                                       (yy.w - mean) * rstd)
                         : f4_zero();
    const float4 g = make_float4(dy.x * gm.x, dy.y * gm.y, dy.z * gm.z, dy.w * gm.w);
    gg.x = fmaf(dy.x, yh.x, gg.x); gg.y = fmaf(dy.y, yh.y, gg.y);
    gg.z = fmaf(dy.z, yh.z, gg.z); gg.w = fmaf(dy.w, yh.w, gg.w);
    gb.x += dy.x; gb.y += dy.y; gb.z += dy.z; gb.w += dy.w;
    const float m1 = half_sum(g.x + g.y + g.z + g.w) * inv_d;
    const float m2 = half_sum(g.x * yh.x + g.y * yh.y + g.z * yh.z + g.w * yh.w) * inv_d;
    // y = relu(u * mult): dy/du = mult where y > 0, else 0
    const float4 du = make_float4(yy.x > 0.f ? rstd * (g.x - m1 - yh.x * m2) * P.scale : 0.f,
                                  yy.y > 0.f ? rstd * (g.y - m1 - yh.y * m2) * P.scale : 0.f,
                                  yy.z > 0.f ? rstd * (g.z - m1 - yh.z * m2) * P.scale : 0.f,
                                  yy.w > 0.f ? rstd * (g.w - m1 - yh.w * m2) * P.scale : 0.f);
    if (ok) {
      *reinterpret_cast<float4*>(P.du + r * P.d + c) = du;
      gu.x += du.x; gu.y += du.y; gu.z += du.z; gu.w += du.w;
    }
  }
  red[wave * 2 + half][0][hl] = gg;
  red[wave * 2 + half][1][hl] = gb;
  red[wave * 2 + half][2][hl] = gu;
  __syncthreads();
  for (int idx = threadIdx.x; idx < P.nsum * P.d; idx += kBlock) {
    const int which = idx / P.d;
    const int col = idx - which * P.d;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 2 * kWavesPerBlock; ++w) {
      const float4 v = red[w][which][col >> 2];
      s += (col & 3) == 0 ? v.x : ((col & 3) == 1 ? v.y : ((col & 3) == 2 ? v.z : v.w));
    }
    P.partial[(static_cast<int64_t>(blockIdx.x) * P.nsum + which) * P.d + col] = s;
  }
}

// out_which[c] = sum over rows r of partial[r][which][c] (which < nsum): one wave per
// output, fixed order.
__global__ __launch_bounds__(kBlock) void column_sums(const float* partial, int rows, int d,
                                                     int nsum, float* out0, float* out1,
                                                     float* out2) {
  const int o = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (o >= nsum * d) return;
  const int which = o / d;
  const int c = o - which * d;
  float s = 0.f;
  for (int r = lane_id(); r < rows; r += kWave)
    s += partial[(static_cast<int64_t>(r) * nsum + which) * d + c];
  s = wave_sum(s);
  if (lane_id() == 0) (which == 0 ? out0 : (which == 1 ? out1 : out2))[c] = s;
}

int epi_grid(int64_t n) {
  const int64_t want = ceil_div(n, kWavesPerBlock);
  return static_cast<int>(want < kEpiMaxBlocks ? (want < 1 ? 1 : want) : kEpiMaxBlocks);
}

// The same for rows of whole chunks up to 128 wide (cols % 4 == 0, 16-byte aligned rows): a
// half-wave per row, lane l multiplying columns 4l .. 4l+3; each group's products are
// summed over the half-wave in a fixed order.
__global__ __launch_bounds__(kBlock) void row_group_dots_h(int64_t n, int groups, int width,
                                                          const float* a, int64_t lda,
                                                          const float* b, int64_t ldb, float* out) {
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int cols = groups * width;
  const int c = 4 * hl;
  const bool on = c < cols;
  int gi[4];  // group of each of the lane's four columns
#pragma unroll
  for (int i = 0; i < 4; ++i) gi[i] = (c + i) / width;
  const int64_t slots = static_cast<int64_t>(gridDim.x) * kWavesPerBlock * 2;
  // the loop runs on the wave's first row, so both halves take every iteration
  for (int64_t r = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave)) * 2 + half;
       r - half < n; r += slots) {
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    if (on && r < n) {
      const float4 x = *reinterpret_cast<const float4*>(a + r * lda + c);
      const float4 y = *reinterpret_cast<const float4*>(b + r * ldb + c);
      p[0] = x.x * y.x;
      p[1] = x.y * y.y;
      p[2] = x.z * y.z;
      p[3] = x.w * y.w;
    }
    for (int g = 0; g < groups; ++g) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s += gi[i] == g ? p[i] : 0.f;
      s = half_sum(s);
      if (hl == 0 && r < n) out[r * groups + g] = s;
    }
  }
}

// out[r][g] = sum_j a[r][g*width + j] * b[r][g*width + j]: one wave per row (grid-stride),
// a fixed-order wave sum per group.
__global__ __launch_bounds__(kBlock) void row_group_dots(int64_t n, int groups, int width,
                                                        const float* a, int64_t lda,
                                                        const float* b, int64_t ldb, float* out) {
  const int lane = lane_id();
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       r < n; r += total) {
    for (int g = 0; g < groups; ++g) {
      float p = 0.f;
      for (int j = lane; j < width; j += kWave)
        p = fmaf(a[r * lda + g * width + j], b[r * ldb + g * width + j], p);
      p = wave_sum(p);
      if (lane == 0) out[r * groups + g] = p;
    }
  }
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_tgat_epilogue_fwd_f32(int64_t n, int32_t d, const float* r1, int64_t ld1,
                                        const float* r2, int64_t ld2, const float* bias,
                                        const float* gamma, const float* beta, float eps,
                                        uint64_t drop_seed, float drop_p, float* out, float* y,
                                        float* stats, hipStream_t stream) {
  if (n < 0 || d <= 0 || d > kMaxPer * kWave || !(drop_p >= 0.f && drop_p < 1.f)) return FA_EINVAL;
  if (n == 0) return FA_OK;
  if (!r1 || ld1 < d || (r2 && ld2 < d) || !gamma || !beta || !out || !y || !stats) return FA_EINVAL;
  EpiParams P;
  P.n = n; P.d = d; P.r1 = r1; P.ld1 = ld1; P.r2 = r2; P.ld2 = ld2; P.bias = bias;
  P.gamma = gamma; P.beta = beta;
  P.eps = eps; P.drop = drop_p > 0.f; P.seed = drop_seed; P.p = drop_p;
  P.scale = static_cast<float>(1.0 / (1.0 - static_cast<double>(drop_p)));
  P.out = out; P.y = y; P.stats = stats;
  const bool rows4 = !(d & 3) && d <= 4 * kHalf && aligned16(r1) && !(ld1 & 3) &&
                     (!r2 || (aligned16(r2) && !(ld2 & 3))) && (!bias || aligned16(bias)) &&
                     aligned16(gamma) && aligned16(beta) && aligned16(out) && aligned16(y);
  if (rows4) {
    const int64_t want = ceil_div(n, 2 * kWavesPerBlock * kEpiRows);
    const int g = static_cast<int>(want < kEpiRowBlocks ? want : kEpiRowBlocks);
    hipLaunchKernelGGL(epilogue_fwd_h, dim3(g), dim3(kBlock), 0, stream, P);
    return launch_status();
  }
  const dim3 grid(epi_grid(n));
  switch (static_cast<int>(ceil_div(d, kWave))) {
    case 1: hipLaunchKernelGGL(epilogue_fwd<1>, grid, dim3(kBlock), 0, stream, P); break;
    case 2: hipLaunchKernelGGL(epilogue_fwd<2>, grid, dim3(kBlock), 0, stream, P); break;
    case 3: hipLaunchKernelGGL(epilogue_fwd<3>, grid, dim3(kBlock), 0, stream, P); break;
    default: hipLaunchKernelGGL(epilogue_fwd<4>, grid, dim3(kBlock), 0, stream, P); break;
  }
  return launch_status();
}

extern "C" int fa_row_group_dots_f32(int64_t n, int32_t groups, int32_t width, const float* a,
                                     int64_t lda, const float* b, int64_t ldb, float* out,
                                     hipStream_t stream) {
  if (n < 0 || groups <= 0 || width <= 0) return FA_EINVAL;
  if (n == 0) return FA_OK;
  const int64_t cols = static_cast<int64_t>(groups) * width;
  if (!a || !b || !out || lda < cols || ldb < cols) return FA_EINVAL;
  if (!(cols & 3) && cols <= 4 * kHalf && aligned16(a) && aligned16(b) && !(lda & 3) && !(ldb & 3)) {
    const int64_t want = ceil_div(n, 2 * kWavesPerBlock);
    const int g = static_cast<int>(want < kEpiRowBlocks ? want : kEpiRowBlocks);
    hipLaunchKernelGGL(row_group_dots_h, dim3(static_cast<unsigned>(g)), dim3(kBlock), 0, stream, n,
                       groups, width, a, lda, b, ldb, out);
    return launch_status();
  }
  hipLaunchKernelGGL(row_group_dots, dim3(static_cast<unsigned>(epi_grid(n))), dim3(kBlock), 0,
                     stream, n, groups, width, a, lda, b, ldb, out);
  return launch_status();
}

extern "C" size_t fa_tgat_epilogue_bwd_scratch_bytes(int64_t n, int32_t d) {
  if (n <= 0 || d <= 0) return 0;
  return static_cast<size_t>(epi_grid(n)) * 3 * static_cast<size_t>(d) * sizeof(float);
}

extern "C" int fa_tgat_epilogue_bwd_f32(int64_t n, int32_t d, const float* dout, const float* y,
                                        const float* stats, const float* gamma, float drop_p,
                                        float* du, float* dgamma, float* dbeta, float* dbias,
                                        void* scratch, size_t scratch_bytes, hipStream_t stream) {
  if (n < 0 || d <= 0 || d > kMaxPer * kWave || !(drop_p >= 0.f && drop_p < 1.f)) return FA_EINVAL;
  if (!dgamma || !dbeta || !gamma) return FA_EINVAL;
  const int nsum = dbias ? 3 : 2;
  if (n == 0) {
    hipLaunchKernelGGL(column_sums, dim3(static_cast<unsigned>(ceil_div(nsum * d, kWavesPerBlock))),
                       dim3(kBlock), 0, stream, static_cast<const float*>(nullptr), 0, d, nsum,
                       dgamma, dbeta, dbias);
    return launch_status();
  }
  if (!dout || !y || !stats || !du) return FA_EINVAL;
  if (!scratch || scratch_bytes < fa_tgat_epilogue_bwd_scratch_bytes(n, d)) return FA_ESCRATCH;
  EpiBwdParams P;
  P.n = n; P.d = d; P.dout = dout; P.y = y; P.stats = stats; P.gamma = gamma;
  P.scale = static_cast<float>(1.0 / (1.0 - static_cast<double>(drop_p)));
  P.du = du; P.nsum = nsum; P.partial = static_cast<float*>(scratch);
  const int grid = epi_grid(n);
  const bool rows4 = !(d & 3) && d <= 4 * kHalf && aligned16(dout) && aligned16(y) &&
                     aligned16(du) && aligned16(gamma);
  if (rows4) {
    hipLaunchKernelGGL(epilogue_bwd_h, dim3(grid), dim3(kBlock), 0, stream, P);
  } else {
    switch (static_cast<int>(ceil_div(d, kWave))) {
      case 1: hipLaunchKernelGGL(epilogue_bwd<1>, dim3(grid), dim3(kBlock), 0, stream, P); break;
      case 2: hipLaunchKernelGGL(epilogue_bwd<2>, dim3(grid), dim3(kBlock), 0, stream, P); break;
      case 3: hipLaunchKernelGGL(epilogue_bwd<3>, dim3(grid), dim3(kBlock), 0, stream, P); break;
      default: hipLaunchKernelGGL(epilogue_bwd<4>, dim3(grid), dim3(kBlock), 0, stream, P); break;
    }
  }
  hipLaunchKernelGGL(column_sums, dim3(static_cast<unsigned>(ceil_div(nsum * d, kWavesPerBlock))),
                     dim3(kBlock), 0, stream, static_cast<const float*>(P.partial), grid, d, nsum,
                     dgamma, dbeta, dbias);
  return launch_status();
}
