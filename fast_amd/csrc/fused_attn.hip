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

// Generic-head fallbacks (heads not in {1, 2, 4, 8}): one wave per segment. Lanes < heads
// hold the per-head max / sum; every lane then owns output columns c = col0 + lane + 64k of
// the destination row.
__global__ __launch_bounds__(kBlock) void fused_attn_fwd_generic(const int32_t* indptr, int64_t n_seg,
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
__global__ __launch_bounds__(kBlock) void fused_attn_bwd_generic(const int32_t* indptr, int64_t n_seg,
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

// ---------------------------------------------------------------------------------
// Kernels for heads in {1, 2, 4, 8}: one wave per segment (grid-stride). Lane j holds
// edge j of a 64-edge block of the segment (score, attention and dropout factors of every
// head); V rows are read as float4 chunks (lane l owns chunks l, l+64, ...) through buffer
// descriptors sized to the row, kRows rows in flight; the head of each chunk component is
// (4c + i) / dh.
// ---------------------------------------------------------------------------------
constexpr int kRows = 8;
// Pairs of rows in flight per wave in the half-wave kernels (FA_FA_PAIR_ROWS pairs: two
// rows per load instruction).
#ifndef FA_FA_PAIR_ROWS
#define FA_FA_PAIR_ROWS 4
#endif
constexpr int kPairRows = FA_FA_PAIR_ROWS;
using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t row_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// AUX: cache-policy bits; kStream (non-temporal) for rows read or written once.
constexpr int kStream = 2;

template <bool VEC, int AUX = 0>
__device__ __forceinline__ float4 chunk_load(rsrc_t r, uint32_t off) {
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
    u4 w4;
    w4[0] = __float_as_uint(x.x);
    w4[1] = __float_as_uint(x.y);
    w4[2] = __float_as_uint(x.z);
    w4[3] = __float_as_uint(x.w);
    __builtin_amdgcn_raw_buffer_store_b128(w4, r, static_cast<int>(off), 0, AUX);
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

struct FaParams {
  const int32_t* indptr; int64_t n_seg;
  const int64_t* dst; const int64_t* src;
  int64_t n_edges, n_dst, n_src, n_v;
  const float* score; const float* V; const float* mask; const float* attn_in;
  const float* dout;
  int dh, dim, chunks;
  float slope, p;
  float* attn; float* out; float* d_act; float* grad_V;
  const int* own;   // backward: nonzero when every V row belongs to its own edge (row e)
};

// Per-lane head of each component of its NS chunks (H = number of heads).
template <int NS>
struct ChunkHeads {
  int h[NS][4];
};

template <int NS>
__device__ __forceinline__ void chunk_heads(const FaParams& P, ChunkHeads<NS>& C) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < NS; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 4 * (lane + k * kWave) + i;
      C.h[k][i] = col < P.dim ? col / P.dh : -1;
    }
}

template <int H>
__device__ __forceinline__ float pick(const float (&w)[H], int h) {
  float r = 0.f;
#pragma unroll
  for (int q = 0; q < H; ++q) r = h == q ? w[q] : r;
  return r;
}

// A kept entry's weight a/(1-p), formed in double as fused_attention.cu:285-287 does, with
// the division by 1-p taken once per kernel: a * keep with keep = 1/(1-p) in double (the two
// double results differ by at most an ulp of double, far below float's rounding).
__device__ __forceinline__ double keep_scale(float p) { return 1.0 / (1.0 - static_cast<double>(p)); }
__device__ __forceinline__ float drop_weight(float a, float m, float p, double keep) {
  return m > p ? static_cast<float>(static_cast<double>(a) * keep) : 0.f;
}

template <int H, int NS, bool VEC>
__global__ __launch_bounds__(kBlock) void fused_attn_fwd_k(FaParams P) {
  const int lane = lane_id();
  const double keep = keep_scale(P.p);
  ChunkHeads<NS> C;
  chunk_heads<NS>(P, C);
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       s < P.n_seg; s += total) {
    int64_t lb = P.indptr[s], le = P.indptr[s + 1];
    lb = lb < 0 ? 0 : lb;
    le = le > P.n_edges ? P.n_edges : le;
    if (le <= lb) continue;
    // softmax statistics per head over the whole segment (edge order within lanes)
    float mx[H], sm[H];
#pragma unroll
    for (int h = 0; h < H; ++h) { mx[h] = kMaxSeed; sm[h] = 0.f; }
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const bool in = e0 + lane < le;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const float l = in ? leaky(P.score[(e0 + lane) * H + h], P.slope) : kMaxSeed;
        mx[h] = fmaxf(mx[h], wave_max(l));
      }
    }
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const bool in = e0 + lane < le;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const float v = in ? expf(leaky(P.score[(e0 + lane) * H + h], P.slope) - mx[h]) : 0.f;
        sm[h] += wave_sum(v);
      }
    }
    const int64_t d = P.dst[lb];
    const bool write_out = d >= 0 && d < P.n_dst;
    float4 acc[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = f4_zero();
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const int cnt = static_cast<int>(le - e0 < kWave ? le - e0 : kWave);
      const bool in = lane < cnt;
      const int64_t e = e0 + (in ? lane : 0);
      float w[H];
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const float a = expf(leaky(P.score[e * H + h], P.slope) - mx[h]) / sm[h];
        if (in) P.attn[e * H + h] = a;
        w[h] = P.mask ? drop_weight(a, P.mask[e * H + h], P.p, keep) : a;
      }
      const int64_t my_src = P.src[e];
      if (!write_out || P.dim == 0) continue;
      for (int j = 0; j < cnt; j += kRows) {
        const int nb = cnt - j < kRows ? cnt - j : kRows;
        float4 r[kRows][NS];
#pragma unroll
        for (int b = 0; b < kRows; ++b) {
          if (b < nb) {
            const int64_t row = lane_i64(my_src, j + b) - P.n_dst;
            const bool ok = row >= 0 && row < P.n_v;
            const rsrc_t rr = row_rsrc(P.V + (ok ? row : 0) * P.dim, ok ? 4u * static_cast<uint32_t>(P.dim) : 0u);
#pragma unroll
            for (int k = 0; k < NS; ++k) r[b][k] = chunk_load<VEC>(rr, 16u * static_cast<uint32_t>(lane + k * kWave));
          }
        }
#pragma unroll
        for (int b = 0; b < kRows; ++b) {
          if (b < nb) {
            float wb[H];
#pragma unroll
            for (int h = 0; h < H; ++h) wb[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[h]), j + b));
#pragma unroll
            for (int k = 0; k < NS; ++k) {
              acc[k].x = fmaf(pick<H>(wb, C.h[k][0]), r[b][k].x, acc[k].x);
              acc[k].y = fmaf(pick<H>(wb, C.h[k][1]), r[b][k].y, acc[k].y);
              acc[k].z = fmaf(pick<H>(wb, C.h[k][2]), r[b][k].z, acc[k].z);
              acc[k].w = fmaf(pick<H>(wb, C.h[k][3]), r[b][k].w, acc[k].w);
            }
          }
        }
      }
    }
    if (!write_out) continue;
    float* o = P.out + d * P.dim;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c4 = 4 * (lane + k * kWave);
      if (c4 < P.dim) o[c4] = acc[k].x;
      if (c4 + 1 < P.dim) o[c4 + 1] = acc[k].y;
      if (c4 + 2 < P.dim) o[c4 + 2] = acc[k].z;
      if (c4 + 3 < P.dim) o[c4 + 3] = acc[k].w;
    }
  }
}

// Forward for rows of at most 32 float4 chunks (dim <= 128): the two half-waves take
// alternate edges of the segment and each lane one chunk of its half's V row, so one load
// instruction reads two rows (25 of each half's 32 lanes carry data at D = 100, against 25
// of 64 with one row per wave); the halves' sums are added once per segment. Statistics,
// attention and dropout weights as fused_attn_fwd_k.
template <int H, bool VEC>
__global__ __launch_bounds__(kBlock) void fused_attn_fwd_half(FaParams P) {
  const int lane = lane_id();
  const double keep = keep_scale(P.p);
  const int half = lane >> 5, hl = lane & (kHalf - 1);
  int hc[4];   // head of each component of this lane's chunk (-1 past dim)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int col = 4 * hl + i;
    hc[i] = col < P.dim ? col / P.dh : -1;
  }
  const uint32_t coff = 16u * static_cast<uint32_t>(hl);   // past the row for hl >= chunks
  static_assert(kWave % (2 * kPairRows) == 0, "pairs stay inside a 64-edge block");
  // V chunks of this half's edges of pairs j/2 .. j/2 + kPairRows - 1 of a block (entry
  // j + 2b + half; j + 2b is even, so a pair's lanes lie in the block; entries past cnt get
  // an empty descriptor)
  auto issue = [&](int64_t my_src, int j, int cnt, float4 (&r)[kPairRows]) {
#pragma unroll
    for (int b = 0; b < kPairRows; ++b) {
      const int j0 = j + 2 * b;
      const int64_t s0 = lane_i64(my_src, j0), s1 = lane_i64(my_src, j0 + 1);
      const int64_t row = (half ? s1 : s0) - P.n_dst;
      const bool ok = j0 + half < cnt && row >= 0 && row < P.n_v;
      const rsrc_t rr = row_rsrc(P.V + (ok ? row : 0) * P.dim, ok ? 4u * static_cast<uint32_t>(P.dim) : 0u);
      r[b] = chunk_load<VEC, kStream>(rr, coff);
    }
  };
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       s < P.n_seg; s += total) {
    int64_t lb = P.indptr[s], le = P.indptr[s + 1];
    lb = lb < 0 ? 0 : lb;
    le = le > P.n_edges ? P.n_edges : le;
    if (le <= lb) continue;
    const int64_t d = P.dst[lb];
    const bool write_out = d >= 0 && d < P.n_dst && P.dim > 0;
    // the first 64-edge block in registers, and its first V rows in flight while the
    // softmax statistics are formed
    const int cnt0 = static_cast<int>(le - lb < kWave ? le - lb : kWave);
    const bool in0 = lane < cnt0;
    const int64_t e00 = lb + (in0 ? lane : 0);
    float l0[H];
#pragma unroll
    for (int h = 0; h < H; ++h) l0[h] = in0 ? leaky(P.score[e00 * H + h], P.slope) : kMaxSeed;
    const int64_t src0 = P.src[e00];
    float4 r[kPairRows];
    if (write_out) issue(src0, 0, cnt0, r);
    float mx[H], sm[H], ex0[H];   // ex0: exp(l - max) of the first block, formed once
    if (le - lb <= kWave) {   // one block: the statistics from the registers
#pragma unroll
      for (int h = 0; h < H; ++h) {
        mx[h] = wave_max(l0[h]);
        ex0[h] = expf(l0[h] - mx[h]);
        sm[h] = wave_sum(in0 ? ex0[h] : 0.f);
      }
    } else {
#pragma unroll
      for (int h = 0; h < H; ++h) { mx[h] = kMaxSeed; sm[h] = 0.f; }
      for (int64_t e0 = lb; e0 < le; e0 += kWave) {
        const bool in = e0 + lane < le;
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const float l = in ? leaky(P.score[(e0 + lane) * H + h], P.slope) : kMaxSeed;
          mx[h] = fmaxf(mx[h], wave_max(l));
        }
      }
      for (int64_t e0 = lb; e0 < le; e0 += kWave) {
        const bool in = e0 + lane < le;
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const float v = in ? expf(leaky(P.score[(e0 + lane) * H + h], P.slope) - mx[h]) : 0.f;
          sm[h] += wave_sum(v);
        }
      }
#pragma unroll
      for (int h = 0; h < H; ++h) ex0[h] = expf(l0[h] - mx[h]);
    }
    float4 acc = f4_zero();
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const bool first = e0 == lb;
      const int cnt = static_cast<int>(le - e0 < kWave ? le - e0 : kWave);
      const bool in = lane < cnt;
      const int64_t e = e0 + (in ? lane : 0);
      float w[H];
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const float ex = first ? ex0[h] : expf(leaky(P.score[e * H + h], P.slope) - mx[h]);
        const float a = ex / sm[h];
        if (in) P.attn[e * H + h] = a;
        w[h] = P.mask ? drop_weight(a, P.mask[e * H + h], P.p, keep) : a;
        w[h] = in ? w[h] : 0.f;
      }
      if (!write_out) continue;
      const int64_t my_src = first ? src0 : P.src[e];
      for (int j = 0; j < cnt; j += 2 * kPairRows) {
        if (!(first && j == 0)) issue(my_src, j, cnt, r);
#pragma unroll
        for (int b = 0; b < kPairRows; ++b) {
          if (j + 2 * b >= cnt) break;
          const int j0 = j + 2 * b;
          float wb[H];
#pragma unroll
          for (int h = 0; h < H; ++h) {
            const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[h]), j0));
            const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[h]), j0 + 1));
            wb[h] = half ? w1 : w0;   // a missing entry has weight 0 and a zero row
          }
          acc.x = fmaf(pick<H>(wb, hc[0]), r[b].x, acc.x);
          acc.y = fmaf(pick<H>(wb, hc[1]), r[b].y, acc.y);
          acc.z = fmaf(pick<H>(wb, hc[2]), r[b].z, acc.z);
          acc.w = fmaf(pick<H>(wb, hc[3]), r[b].w, acc.w);
        }
      }
    }
    if (!write_out) continue;
    // the two halves' sums of each chunk (edge order within a half, then the halves)
    acc.x += __shfl_xor(acc.x, kHalf, kWave);
    acc.y += __shfl_xor(acc.y, kHalf, kWave);
    acc.z += __shfl_xor(acc.z, kHalf, kWave);
    acc.w += __shfl_xor(acc.w, kHalf, kWave);
    if (half == 0) {
      float* o = P.out + d * P.dim;
      const int c4 = 4 * hl;
      if (c4 < P.dim) o[c4] = acc.x;
      if (c4 + 1 < P.dim) o[c4 + 1] = acc.y;
      if (c4 + 2 < P.dim) o[c4 + 2] = acc.z;
      if (c4 + 3 < P.dim) o[c4 + 3] = acc.w;
    }
  }
}

template <int H, int NS, bool VEC>
__global__ __launch_bounds__(kBlock) void fused_attn_bwd_k(FaParams P) {
  __shared__ __attribute__((aligned(16))) float stage_all[kWavesPerBlock][4 * kWave * NS];
  float* stage = stage_all[threadIdx.x / kWave];
  const int lane = lane_id();
  ChunkHeads<NS> C;
  chunk_heads<NS>(P, C);
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const float keep = static_cast<float>(1.0 / (1.0 - static_cast<double>(P.p)));
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       s < P.n_seg; s += total) {
    int64_t lb = P.indptr[s], le = P.indptr[s + 1];
    lb = lb < 0 ? 0 : lb;
    le = le > P.n_edges ? P.n_edges : le;
    if (le <= lb) continue;
    const int64_t d = P.dst[lb];
    if (d < 0 || d >= P.n_dst) continue;
    // dout row of the destination, chunked like the V rows
    float4 g[NS];
    {
      const rsrc_t dr = row_rsrc(P.dout + d * P.dim, 4u * static_cast<uint32_t>(P.dim));
#pragma unroll
      for (int k = 0; k < NS; ++k) g[k] = chunk_load<VEC>(dr, 16u * static_cast<uint32_t>(lane + k * kWave));
    }
    float tsum[H];
#pragma unroll
    for (int h = 0; h < H; ++h) tsum[h] = 0.f;
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const int cnt = static_cast<int>(le - e0 < kWave ? le - e0 : kWave);
      const bool in = lane < cnt;
      const int64_t e = e0 + (in ? lane : 0);
      float a[H], kf[H], da[H];
#pragma unroll
      for (int h = 0; h < H; ++h) {
        a[h] = P.attn_in[e * H + h];
        kf[h] = P.mask ? (P.mask[e * H + h] > P.p ? keep : 0.f) : 1.f;
        da[h] = 0.f;
      }
      const int64_t my_src = P.src[e];
      for (int j = 0; j < cnt; j += kRows) {
        const int nb = cnt - j < kRows ? cnt - j : kRows;
        float4 r[kRows][NS];
        bool okb[kRows];
        int64_t rowb[kRows];
#pragma unroll
        for (int b = 0; b < kRows; ++b) {
          okb[b] = false;
          rowb[b] = 0;
          if (b < nb) {
            const int64_t sr = lane_i64(my_src, j + b);
            const int64_t row = sr - P.n_dst;
            okb[b] = row >= 0 && row < P.n_v && sr < P.n_src;
            rowb[b] = okb[b] ? row : 0;
            const rsrc_t rr = row_rsrc(P.V + rowb[b] * P.dim, okb[b] ? 4u * static_cast<uint32_t>(P.dim) : 0u);
#pragma unroll
            for (int k = 0; k < NS; ++k) r[b][k] = chunk_load<VEC>(rr, 16u * static_cast<uint32_t>(lane + k * kWave));
          }
        }
#pragma unroll
        for (int b = 0; b < kRows; ++b) {
          if (b < nb && okb[b]) {
            float ab[H], kb[H], part[H];
#pragma unroll
            for (int h = 0; h < H; ++h) {
              ab[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[h]), j + b));
              kb[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kf[h]), j + b));
              part[h] = 0.f;
            }
            float4 gvc[NS];  // this edge's grad_V row: a * keep * dout, per component head
#pragma unroll
            for (int k = 0; k < NS; ++k) {
              const float gx[4] = {g[k].x, g[k].y, g[k].z, g[k].w};
              const float vx[4] = {r[b][k].x, r[b][k].y, r[b][k].z, r[b][k].w};
              float cx[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int hh = C.h[k][i];
                cx[i] = pick<H>(ab, hh) * pick<H>(kb, hh) * gx[i];
#pragma unroll
                for (int h = 0; h < H; ++h) part[h] = hh == h ? fmaf(gx[i], vx[i], part[h]) : part[h];
              }
              gvc[k] = make_float4(cx[0], cx[1], cx[2], cx[3]);
            }
            atomic_add_row<NS>(P.grad_V + rowb[b] * P.dim, P.dim, gvc, stage);
#pragma unroll
            for (int h = 0; h < H; ++h) {
              const float v = kb[h] * wave_sum(part[h]);
              da[h] = lane == j + b ? v : da[h];
            }
          }
        }
      }
#pragma unroll
      for (int h = 0; h < H; ++h) {
        if (in) P.d_act[e * H + h] = da[h];
        tsum[h] += wave_sum(in ? a[h] * da[h] : 0.f);
      }
    }
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const int64_t e = e0 + lane;
      if (e < le) {
#pragma unroll
        for (int h = 0; h < H; ++h) P.d_act[e * H + h] = P.attn_in[e * H + h] * (P.d_act[e * H + h] - tsum[h]);
      }
    }
  }
}

// The own-rows flag: set to 1, then cleared by any edge whose V row is in range and is not
// row e (a row that two edges may add to); plain stores of a single value, any order.
__global__ __launch_bounds__(64) void own_flag_set(int* flag) {
  if (threadIdx.x == 0) flag[0] = 1;
}

// Clears the flag unless every in-range V row is its own edge's and the segment offsets
// never decrease (so no edge lies in two segments and each row has at most one writer).
__global__ __launch_bounds__(kBlock) void check_own_rows(const int64_t* src, int64_t n_edges,
                                                         int64_t n_dst, int64_t n_v,
                                                         int64_t n_src, const int32_t* indptr,
                                                         int64_t n_seg, int* flag) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < n_edges; e += stride) {
    const int64_t sr = src[e];
    const int64_t row = sr - n_dst;
    if (row >= 0 && row < n_v && sr < n_src && row != e) flag[0] = 0;
  }
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; s < n_seg; s += stride)
    if (indptr[s + 1] < indptr[s]) flag[0] = 0;
}

// The grad_V rows the backward does not store: every row when the rows are not each edge's
// own (the atomic adds then start from zeros), else the rows of the edges outside
// [indptr[0], indptr[n_seg]) (the backward stores every row inside, zeros for the edges
// that contribute nothing). `own` NULL: every row.
__global__ __launch_bounds__(kBlock) void grad_v_fill(const int* own, const int32_t* indptr,
                                                      int64_t n_seg, int64_t n_edges, int64_t n_v,
                                                      int64_t dim, float* grad_V) {
  int64_t a = 0, b = 0;   // rows [a, b) are stored by the backward
  if (own && own[0] != 0) {
    a = indptr[0];
    b = indptr[n_seg];
    a = a < 0 ? 0 : (a > n_edges ? n_edges : a);
    b = b < a ? a : (b > n_edges ? n_edges : b);
    a = a > n_v ? n_v : a;
    b = b > n_v ? n_v : b;
  }
  const int64_t head = a * dim, tail = (n_v - b) * dim;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  const bool vec = (dim & 3) == 0 && (reinterpret_cast<uintptr_t>(grad_V) & 15) == 0;
  if (vec) {
    float4* g4 = reinterpret_cast<float4*>(grad_V);
    const int64_t h4 = head / 4, t4 = tail / 4, b4 = b * dim / 4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < h4 + t4; i += stride)
      g4[i < h4 ? i : i - h4 + b4] = f4_zero();
    return;
  }
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < head + tail; i += stride)
    grad_V[i < head ? i : i - head + b * dim] = 0.f;
}

// Backward for rows of at most 32 float4 chunks, in the half-wave layout of
// fused_attn_fwd_half: the halves take alternate edges; per edge its half forms the grad_V
// chunk a*keep*dout and the partial dots keep*dout.V per head (a half-wave sum), adds the
// grad_V row with lane-consecutive atomics through its LDS staging row, and the per-edge
// dots land in the lane of their edge. A segment of at most 64 edges keeps them in
// registers and writes d_act once; longer ones finish in a second pass as fused_attn_bwd_k.
template <int H, bool VEC>
__global__ __launch_bounds__(kBlock) void fused_attn_bwd_half(FaParams P) {
  __shared__ __attribute__((aligned(16))) float stage_all[kWavesPerBlock][2][4 * kHalf];
  const int lane = lane_id();
  const int half = lane >> 5, hl = lane & (kHalf - 1);
  float* stage = stage_all[threadIdx.x / kWave][half];
  int hc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int col = 4 * hl + i;
    hc[i] = col < P.dim ? col / P.dh : -1;
  }
  const uint32_t coff = 16u * static_cast<uint32_t>(hl);
  const float keep = static_cast<float>(1.0 / (1.0 - static_cast<double>(P.p)));
  const bool own = P.own && P.own[0] != 0;
  static_assert(kWave % (2 * kPairRows) == 0, "pairs stay inside a 64-edge block");
  // this half's row of pair entry j0 (-1 when missing or out of range)
  auto row_of = [&](int64_t my_src, int j0, int cnt) -> int64_t {
    const int64_t s0 = lane_i64(my_src, j0), s1 = lane_i64(my_src, j0 + 1);
    const int64_t sr = half ? s1 : s0;
    const int64_t row = sr - P.n_dst;
    return (j0 + half < cnt && row >= 0 && row < P.n_v && sr < P.n_src) ? row : -1;
  };
  auto issue = [&](int64_t my_src, int j, int cnt, float4 (&r)[kPairRows]) {
#pragma unroll
    for (int b = 0; b < kPairRows; ++b) {
      const int64_t row = row_of(my_src, j + 2 * b, cnt);
      const rsrc_t rr = row_rsrc(P.V + (row >= 0 ? row : 0) * P.dim, row >= 0 ? 4u * static_cast<uint32_t>(P.dim) : 0u);
      r[b] = chunk_load<VEC, kStream>(rr, coff);
    }
  };
  const int64_t total = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + uniform(threadIdx.x / kWave);
       s < P.n_seg; s += total) {
    int64_t lb = P.indptr[s], le = P.indptr[s + 1];
    lb = lb < 0 ? 0 : lb;
    le = le > P.n_edges ? P.n_edges : le;
    if (le <= lb) continue;
    const int64_t d = P.dst[lb];
    if (d < 0 || d >= P.n_dst) {
      // no gradient flows through this segment; with own rows its edges' rows are zeros
      if (own)
        for (int64_t j = lb + half; j < le; j += 2) {
          const rsrc_t wr = row_rsrc(P.grad_V + (j < P.n_v ? j : 0) * P.dim,
                                     j < P.n_v ? 4u * static_cast<uint32_t>(P.dim) : 0u);
          store_chunk<VEC, kStream>(wr, coff, f4_zero());
        }
      continue;
    }
    const bool one = le - lb <= kWave;
    float4 g;   // this lane's chunk of the destination's dout row
    {
      const rsrc_t dr = row_rsrc(P.dout + d * P.dim, 4u * static_cast<uint32_t>(P.dim));
      g = chunk_load<VEC, kStream>(dr, coff);
    }
    float tsum[H];
#pragma unroll
    for (int h = 0; h < H; ++h) tsum[h] = 0.f;
    float a[H], da[H];   // lane j: entry j of the current block
    int cnt = 0;
    int64_t e = lb;
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      cnt = static_cast<int>(le - e0 < kWave ? le - e0 : kWave);
      const bool in = lane < cnt;
      e = e0 + (in ? lane : 0);
      float kf[H];
#pragma unroll
      for (int h = 0; h < H; ++h) {
        a[h] = in ? P.attn_in[e * H + h] : 0.f;
        kf[h] = P.mask ? (P.mask[e * H + h] > P.p ? keep : 0.f) : 1.f;
        da[h] = 0.f;
      }
      const int64_t my_src = P.src[e];
      float4 r[kPairRows];
      for (int j = 0; j < cnt; j += 2 * kPairRows) {
        issue(my_src, j, cnt, r);
#pragma unroll
        for (int b = 0; b < kPairRows; ++b) {
          if (j + 2 * b >= cnt) break;
          const int j0 = j + 2 * b;
          float ab[H], kb[H], part[H];
#pragma unroll
          for (int h = 0; h < H; ++h) {
            const float a0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[h]), j0));
            const float a1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[h]), j0 + 1));
            const float k0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kf[h]), j0));
            const float k1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kf[h]), j0 + 1));
            ab[h] = half ? a1 : a0;
            kb[h] = half ? k1 : k0;
            part[h] = 0.f;
          }
          const float gx[4] = {g.x, g.y, g.z, g.w};
          const float vx[4] = {r[b].x, r[b].y, r[b].z, r[b].w};
          float cx[4], ak[H];
#pragma unroll
          for (int h = 0; h < H; ++h) ak[h] = ab[h] * kb[h];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            cx[i] = pick<H>(ak, hc[i]) * gx[i];
#pragma unroll
            for (int h = 0; h < H; ++h) part[h] = hc[i] == h ? fmaf(gx[i], vx[i], part[h]) : part[h];
          }
          // the per-edge dots: half 0's into lane j0, half 1's into lane j0 + 1
#pragma unroll
          for (int h = 0; h < H; ++h) {
            const float v = kb[h] * half_sum(part[h]);
            const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
            const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kHalf));
            da[h] = lane == j0 ? v0 : (lane == j0 + 1 ? v1 : da[h]);
          }
          // grad_V row of this half's edge: stored as float4 chunks when every row is its own
          // edge's (the caller's zeros overwritten once), else added lane-consecutively with
          // atomics
          const int64_t row = row_of(my_src, j0, cnt);
          const float4 gv = make_float4(cx[0], cx[1], cx[2], cx[3]);
          if (own) {
            // an edge without a V row in range still owns grad_V row e (no other edge
            // writes it): zeros there
            const int64_t eh = e0 + j0 + half;
            const int64_t wrow = row >= 0 ? row : (j0 + half < cnt && eh < P.n_v ? eh : -1);
            const rsrc_t wr = row_rsrc(P.grad_V + (wrow >= 0 ? wrow : 0) * P.dim,
                                       wrow >= 0 ? 4u * static_cast<uint32_t>(P.dim) : 0u);
            store_chunk<VEC, kStream>(wr, coff, row >= 0 ? gv : f4_zero());
          } else {
            *reinterpret_cast<float4*>(stage + 4 * hl) = gv;
            lds_sync();
            if (row >= 0)
              for (int c = hl; c < P.dim; c += kHalf) atomicAdd(P.grad_V + row * P.dim + c, stage[c]);
            lds_sync();
          }
        }
      }
#pragma unroll
      for (int h = 0; h < H; ++h) {
        if (in && !one) P.d_act[e * H + h] = da[h];
        tsum[h] += wave_sum(in ? a[h] * da[h] : 0.f);
      }
    }
    if (one) {   // the block is still in registers
      if (lane < cnt) {
#pragma unroll
        for (int h = 0; h < H; ++h) P.d_act[e * H + h] = a[h] * (da[h] - tsum[h]);
      }
      continue;
    }
    for (int64_t e0 = lb; e0 < le; e0 += kWave) {
      const int64_t ee = e0 + lane;
      if (ee < le) {
#pragma unroll
        for (int h = 0; h < H; ++h) P.d_act[ee * H + h] = P.attn_in[ee * H + h] * (P.d_act[ee * H + h] - tsum[h]);
      }
    }
  }
}

constexpr int kFaMaxBlocks = 4096;

int fa_grid(int64_t n_seg) {
  const int64_t want = ceil_div(n_seg, kWavesPerBlock);
  return static_cast<int>(want < kFaMaxBlocks ? (want < 1 ? 1 : want) : kFaMaxBlocks);
}

template <int H>
int launch_fa(const FaParams& P, bool bwd, hipStream_t stream) {
  const int ns = static_cast<int>(ceil_div(P.chunks, kWave));
  const bool vec = (P.dim & 3) == 0 && aligned16(P.V) && (!bwd || aligned16(P.dout));
  const dim3 grid(fa_grid(P.n_seg));
#define FA_FA_LAUNCH(NSV)                                                                      \
  if (bwd) {                                                                                  \
    if (vec) hipLaunchKernelGGL((fused_attn_bwd_k<H, NSV, true>), grid, dim3(kBlock), 0, stream, P); \
    else hipLaunchKernelGGL((fused_attn_bwd_k<H, NSV, false>), grid, dim3(kBlock), 0, stream, P);    \
  } else {                                                                                    \
    if (vec) hipLaunchKernelGGL((fused_attn_fwd_k<H, NSV, true>), grid, dim3(kBlock), 0, stream, P); \
    else hipLaunchKernelGGL((fused_attn_fwd_k<H, NSV, false>), grid, dim3(kBlock), 0, stream, P);    \
  }
  if (P.chunks <= kHalf) {   // rows of at most 128 values: the half-wave kernels
    if (bwd) {
      if (vec) hipLaunchKernelGGL((fused_attn_bwd_half<H, true>), grid, dim3(kBlock), 0, stream, P);
      else hipLaunchKernelGGL((fused_attn_bwd_half<H, false>), grid, dim3(kBlock), 0, stream, P);
    } else {
      if (vec) hipLaunchKernelGGL((fused_attn_fwd_half<H, true>), grid, dim3(kBlock), 0, stream, P);
      else hipLaunchKernelGGL((fused_attn_fwd_half<H, false>), grid, dim3(kBlock), 0, stream, P);
    }
    return launch_status();
  }
  switch (ns) {
    case 0:
    case 1: FA_FA_LAUNCH(1) break;
    case 2: FA_FA_LAUNCH(2) break;
    default: FA_FA_LAUNCH(4) break;
  }
#undef FA_FA_LAUNCH
  return launch_status();
}

int launch_fa_heads(const FaParams& P, int heads, bool bwd, hipStream_t stream) {
  switch (heads) {
    case 1: return launch_fa<1>(P, bwd, stream);
    case 2: return launch_fa<2>(P, bwd, stream);
    case 4: return launch_fa<4>(P, bwd, stream);
    case 8: return launch_fa<8>(P, bwd, stream);
    default: return -1000;  // no specialised kernel
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
  if (static_cast<int64_t>(heads) * dh <= 4 * kWave * 4) {
    FaParams P{indptr, n_seg, dst, src, n_edges, n_dst, 0, n_edges, score, V, mask, nullptr,
               nullptr, dh, heads * dh, static_cast<int>(ceil_div(heads * dh, 4)), slope, p,
               attn, out, nullptr, nullptr, nullptr};
    const int st = launch_fa_heads(P, heads, false, stream);
    if (st != -1000) return st;
  }
  hipLaunchKernelGGL(fused_attn_fwd_generic, dim3(ceil_div(n_seg, kWavesPerBlock)), dim3(kBlock), 0,
                     stream, indptr, n_seg, dst, src, n_edges, n_dst, score, V, n_edges, heads,
                     dh, slope, p, mask, attn, out);
  return launch_status();
}

extern "C" size_t fa_fused_attn_bwd_scratch_bytes(void) { return 16; }

extern "C" int fa_fused_attn_bwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                                     const int64_t* src, int64_t n_edges, int64_t n_dst,
                                     int64_t n_src, const float* dout, const float* V,
                                     const float* attn, const float* mask, int32_t heads,
                                     int32_t dh, float p, float* d_act, float* grad_V,
                                     void* scratch, size_t scratch_bytes, hipStream_t stream) {
  if (n_seg < 0 || n_edges < 0 || n_dst < 0 || heads < 0 || dh < 0) return FA_EINVAL;
  if (heads > kWave) return FA_EUNSUPPORTED;
  if (scratch && scratch_bytes < fa_fused_attn_bwd_scratch_bytes()) return FA_ESCRATCH;
  if (heads == 0) return FA_OK;
  const int64_t dim = static_cast<int64_t>(heads) * dh;
  auto fill = [&](const int* own) {   // every grad_V row the kernels below do not store
    const int64_t n4 = ceil_div(n_edges * dim, 4 * kBlock);
    const unsigned grid = static_cast<unsigned>(n4 < 1 ? 1 : (n4 > 2048 ? 2048 : n4));
    hipLaunchKernelGGL(grad_v_fill, dim3(grid), dim3(kBlock), 0, stream, own, indptr, n_seg,
                       n_edges, n_edges, dim, grad_V);
  };
  if (n_seg == 0) {   // no segment: grad_V is zeros
    if (dim > 0 && n_edges > 0 && grad_V) {
      fill(nullptr);
      return launch_status();
    }
    return FA_OK;
  }
  if (!indptr || !dst || !src || !attn || !d_act || (dh > 0 && (!V || !dout || !grad_V)))
    return FA_EINVAL;
  if (dim <= 4 * kWave * 4 && (heads == 1 || heads == 2 || heads == 4 || heads == 8)) {
    int* own = nullptr;
    if (scratch && dh > 0 && dim <= 4 * kHalf) {   // the half-wave backward reads it
      own = static_cast<int*>(scratch);
      hipLaunchKernelGGL(own_flag_set, dim3(1), dim3(64), 0, stream, own);
      const int64_t want = ceil_div(n_edges > n_seg ? n_edges : n_seg, kBlock);
      const unsigned grid = static_cast<unsigned>(want < 1 ? 1 : (want > 1024 ? 1024 : want));
      hipLaunchKernelGGL(check_own_rows, dim3(grid), dim3(kBlock), 0, stream, src, n_edges, n_dst,
                         n_edges, n_src, indptr, n_seg, own);
    }
    if (dh > 0) fill(own);
    FaParams P{indptr, n_seg, dst, src, n_edges, n_dst, n_src, n_edges, nullptr, V, mask, attn,
               dout, dh, heads * dh, static_cast<int>(ceil_div(heads * dh, 4)), 0.f, p, nullptr,
               nullptr, d_act, grad_V, own};
    return launch_fa_heads(P, heads, true, stream);
  }
  if (dh > 0) fill(nullptr);
  hipLaunchKernelGGL(fused_attn_bwd_generic, dim3(ceil_div(n_seg, kWavesPerBlock)), dim3(kBlock), 0,
                     stream, indptr, n_seg, dst, src, n_edges, n_dst, n_src, dout, V, n_edges,
                     attn, mask, heads, dh, p, d_act, grad_V);
  return launch_status();
}
