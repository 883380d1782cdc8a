// Fused TGAT temporal attention over sampled temporal neighbours.
//
// For destination v with edges e in rowptr[v]..rowptr[v+1] and heads h:
//   x_e        = [node_tab[node_row(e)] | edge_tab[edge_row(e)] | cos(w*dt_e + b) | 1]
//   z[e,h]     = qt[h,v,:] . x_e                     (qt = Q_h W_k,aug[h], bias in col Kb)
//   s[e,h]     = leaky_relu(z, slope)
//   a[e,h]     = exp(s - max_v,h) / sum_v,h          (softmax over the destination's edges)
//   xbar[h,v]  = sum_e a[e,h] * drop[e,h] * x_e      (column Kb = sum_e a*drop)
//
// x_e is gathered and time-encoded on the fly and never stored. Layout of one row in
// "K-space" (float4 chunks): node chunks [0,cn), edge chunks [cn,cn+ce), time chunks
// [cn+ce, cn+ce+ct), then one bias chunk (1,0,0,0). One wavefront per destination;
// lane l owns chunks l, l+64, ... (NS slots).
#include <float.h>

#include "fa_common.hpp"

namespace fa {
namespace {

enum ChunkKind : int { kNode = 0, kEdge = 1, kTime = 2, kBias = 3, kNone = 4 };

constexpr int kBatch = 4;             // edges gathered per batch (loads in flight)
constexpr int kBwdMaxBlocks = 2048;   // backward grid cap (time-grad partial rows)

struct TgatParams {
  int64_t n_dst, n_edges;
  const int32_t* rowptr;
  const float* node_tab; int64_t ld_node; int64_t n_node; int dn; const int64_t* node_idx;
  const float* edge_tab; int64_t ld_edge; int64_t n_erow; int de; const int64_t* edge_idx;
  int node_vec, edge_vec, dnode_vec;  // rows 16-byte aligned: float4 access allowed
  const float* dt; const float* time_w; const float* time_b; int dt_dim;
  int cn, ce, ct, cp;                 // chunk counts; cp = cn+ce+ct+1
  int64_t kp;                         // row stride of qt / xbar = 4*cp
  const float* qt; int64_t qt_hs;
  float slope;
  const float* drop;
  // forward outputs
  float* xbar; int64_t xbar_hs;
  float* scores; float* stats;
  // backward
  const float* dxbar; int64_t dxbar_hs;
  float* dqt; int64_t dqt_hs;
  float* d_node; int64_t ld_dnode;
  float* partial;                     // [gridDim.x][2][dt_dim]
};

// What lane `lane` holds in slot k: kind, element offset inside its part, valid count.
struct Slot {
  int kind, off, valid;
};

__device__ __forceinline__ Slot classify(const TgatParams& P, int c) {
  Slot s;
  if (c < P.cn) {
    s.kind = kNode; s.off = 4 * c; s.valid = min(4, P.dn - s.off);
  } else if (c < P.cn + P.ce) {
    s.kind = kEdge; s.off = 4 * (c - P.cn); s.valid = min(4, P.de - s.off);
  } else if (c < P.cn + P.ce + P.ct) {
    s.kind = kTime; s.off = 4 * (c - P.cn - P.ce); s.valid = min(4, P.dt_dim - s.off);
  } else if (c == P.cn + P.ce + P.ct) {
    s.kind = kBias; s.off = 0; s.valid = 1;
  } else {
    s.kind = kNone; s.off = 0; s.valid = 0;
  }
  return s;
}

__device__ __forceinline__ int64_t clamp_edge(int64_t e, int64_t n_edges) {
  return e < 0 ? 0 : (e > n_edges ? n_edges : e);
}

__device__ __forceinline__ float4 load_row_chunk(const float* row, int off, int valid, int vec) {
  if (vec && valid == 4) return *reinterpret_cast<const float4*>(row + off);
  float4 v = f4_zero();
  if (valid > 0) v.x = row[off];
  if (valid > 1) v.y = row[off + 1];
  if (valid > 2) v.z = row[off + 2];
  if (valid > 3) v.w = row[off + 3];
  return v;
}

// Time-encoding chunk: cos(w_j * t + b_j) for the slot's (up to) 4 dims.
__device__ __forceinline__ float4 time_chunk(float t, const float4& w, const float4& b, int valid) {
  float4 v = f4_zero();
  if (valid > 0) v.x = cosf(time_arg(t, w.x, b.x));
  if (valid > 1) v.y = cosf(time_arg(t, w.y, b.y));
  if (valid > 2) v.z = cosf(time_arg(t, w.z, b.z));
  if (valid > 3) v.w = cosf(time_arg(t, w.w, b.w));
  return v;
}

// Gathers the NS chunks this lane owns of x_e for edge e.
template <int NS>
__device__ __forceinline__ void gather_x(const TgatParams& P, const Slot (&sl)[NS],
                                         const float4 (&tw)[NS], const float4 (&tb)[NS],
                                         int64_t e, float4 (&x)[NS]) {
  // Row ids are wave-uniform; out-of-range rows read as zeros.
  const int64_t nrow = P.node_idx ? P.node_idx[e] : e;
  const int64_t erow = P.edge_idx ? P.edge_idx[e] : e;
  const bool nok = nrow >= 0 && nrow < P.n_node;
  const bool eok = erow >= 0 && erow < P.n_erow;
  const float* nptr = P.node_tab + (nok ? nrow : 0) * P.ld_node;
  const float* eptr = P.edge_tab + (eok ? erow : 0) * P.ld_edge;
  const float t = P.dt_dim > 0 ? P.dt[e] : 0.f;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const Slot s = sl[k];
    if (s.kind == kNode) x[k] = nok ? load_row_chunk(nptr, s.off, s.valid, P.node_vec) : f4_zero();
    else if (s.kind == kEdge) x[k] = eok ? load_row_chunk(eptr, s.off, s.valid, P.edge_vec) : f4_zero();
    else if (s.kind == kTime) x[k] = time_chunk(t, tw[k], tb[k], s.valid);
    else if (s.kind == kBias) x[k] = make_float4(1.f, 0.f, 0.f, 0.f);
    else x[k] = f4_zero();
  }
}

template <int NS>
__device__ __forceinline__ void setup_slots(const TgatParams& P, Slot (&sl)[NS], float4 (&tw)[NS],
                                            float4 (&tb)[NS]) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int c = lane + k * kWave;
    sl[k] = classify(P, c);  // chunks past the bias chunk are kNone
    tw[k] = f4_zero();
    tb[k] = f4_zero();
    if (sl[k].kind == kTime) {
      const int o = sl[k].off, v = sl[k].valid;
      if (v > 0) { tw[k].x = P.time_w[o];     tb[k].x = P.time_b[o]; }
      if (v > 1) { tw[k].y = P.time_w[o + 1]; tb[k].y = P.time_b[o + 1]; }
      if (v > 2) { tw[k].z = P.time_w[o + 2]; tb[k].z = P.time_b[o + 2]; }
      if (v > 3) { tw[k].w = P.time_w[o + 3]; tb[k].w = P.time_b[o + 3]; }
    }
  }
}

template <int H, int NS>
__device__ __forceinline__ void load_rows(const float* base, int64_t hs, int64_t v, int64_t kp,
                                          float4 (&r)[H][NS], int cp) {
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c = lane + k * kWave;
      r[h][k] = c < cp ? *reinterpret_cast<const float4*>(base + h * hs + v * kp + 4 * c)
                       : f4_zero();
    }
}

template <int H, int NS>
__device__ __forceinline__ void store_rows(float* base, int64_t hs, int64_t v, int64_t kp,
                                           const float4 (&r)[H][NS], int cp) {
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c = lane + k * kWave;
      if (c < cp) *reinterpret_cast<float4*>(base + h * hs + v * kp + 4 * c) = r[h][k];
    }
}

template <int H, int NS>
__device__ __forceinline__ float head_dot(const float4 (&q)[H][NS], const float4 (&x)[NS], int h) {
  float p = 0.f;
#pragma unroll
  for (int k = 0; k < NS; ++k) p += dot4(q[h][k], x[k]);
  return p;
}

// ---------------------------------------------------------------------------------
// Forward: one wave per destination, online softmax over batches of kBatch edges.
// ---------------------------------------------------------------------------------
template <int H, int NS>
__global__ __launch_bounds__(kBlock) void tgat_fwd(TgatParams P) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (v >= P.n_dst) return;
  const int lane = lane_id();
  const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
  const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);

  float4 acc[H][NS];
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[h][k] = f4_zero();

  if (e1 <= e0) {  // zero-degree destination: xbar = 0
    store_rows<H, NS>(P.xbar, P.xbar_hs, v, P.kp, acc, P.cp);
    if (lane < H) {
      P.stats[(v * H + lane) * 2 + 0] = -INFINITY;
      P.stats[(v * H + lane) * 2 + 1] = 0.f;
    }
    return;
  }

  Slot sl[NS];
  float4 tw[NS], tb[NS];
  setup_slots<NS>(P, sl, tw, tb);
  float4 q[H][NS];
  load_rows<H, NS>(P.qt, P.qt_hs, v, P.kp, q, P.cp);

  float m[H], l[H];
#pragma unroll
  for (int h = 0; h < H; ++h) { m[h] = -INFINITY; l[h] = 0.f; }

  for (int64_t eb = e0; eb < e1; eb += kBatch) {
    const int nb = static_cast<int>(e1 - eb < kBatch ? e1 - eb : kBatch);
    float4 x[kBatch][NS];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (b < nb) gather_x<NS>(P, sl, tw, tb, eb + b, x[b]);
      else
#pragma unroll
        for (int k = 0; k < NS; ++k) x[b][k] = f4_zero();
    }
    float sc[kBatch][H];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int h = 0; h < H; ++h) sc[b][h] = leaky(wave_sum(head_dot<H, NS>(q, x[b], h)), P.slope);

    // Scores of this batch: lane b*H+h stores s[eb+b, h] (contiguous).
    {
      float mine = 0.f;
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
#pragma unroll
        for (int h = 0; h < H; ++h)
          if (lane == b * H + h) mine = sc[b][h];
      if (lane < nb * H) P.scores[eb * H + lane] = mine;
    }

#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (b >= nb) break;
      const int64_t e = eb + b;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const float s = sc[b][h];
        const float dr = P.drop ? P.drop[e * H + h] : 1.f;
        if (s > m[h]) {
          const float r = expf(m[h] - s);  // 0 on the first edge
          l[h] = fmaf(l[h], r, 1.f);
#pragma unroll
          for (int k = 0; k < NS; ++k) {
            scale4(acc[h][k], r);
            fma4(acc[h][k], dr, x[b][k]);
          }
          m[h] = s;
        } else {
          const float pe = expf(s - m[h]);
          l[h] += pe;
          const float w = pe * dr;
#pragma unroll
          for (int k = 0; k < NS; ++k) fma4(acc[h][k], w, x[b][k]);
        }
      }
    }
  }

#pragma unroll
  for (int h = 0; h < H; ++h) {
    const float lsum = l[h];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      acc[h][k].x /= lsum;
      acc[h][k].y /= lsum;
      acc[h][k].z /= lsum;
      acc[h][k].w /= lsum;
    }
  }
  store_rows<H, NS>(P.xbar, P.xbar_hs, v, P.kp, acc, P.cp);
  if (lane < H) {
    float mm = 0.f, ll = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h)
      if (lane == h) { mm = m[h]; ll = l[h]; }
    P.stats[(v * H + lane) * 2 + 0] = mm;
    P.stats[(v * H + lane) * 2 + 1] = ll;
  }
}

// ---------------------------------------------------------------------------------
// Backward: one wave per destination (grid-stride), two passes over the edges.
//   pass 1: da'[e,h] = dxbar[h,v] . x_e,  T_h = sum_e a*drop*da'
//   pass 2: dz = a*(drop*da' - T)*leaky'(s);  dqt += dz*x_e;
//           dx_e = sum_h a*drop*dxbar[h] + dz*qt[h]  -> node rows / time-grad partials
// ---------------------------------------------------------------------------------
template <int H, int NS>
__global__ __launch_bounds__(kBlock) void tgat_bwd(TgatParams P) {
  __shared__ float red[kWavesPerBlock][2][kWave * NS * 4];
  const int lane = lane_id();
  const int wave_in_block = threadIdx.x / kWave;

  Slot sl[NS];
  float4 tw[NS], tb[NS];
  setup_slots<NS>(P, sl, tw, tb);
  float4 gw[NS], gb[NS];  // time-grad accumulators for this lane's time chunks
#pragma unroll
  for (int k = 0; k < NS; ++k) { gw[k] = f4_zero(); gb[k] = f4_zero(); }

  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block; v < P.n_dst;
       v += total_waves) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
    float4 dq[H][NS];
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int k = 0; k < NS; ++k) dq[h][k] = f4_zero();
    if (e1 <= e0) {
      store_rows<H, NS>(P.dqt, P.dqt_hs, v, P.kp, dq, P.cp);
      continue;
    }
    float4 q[H][NS], g[H][NS];
    load_rows<H, NS>(P.qt, P.qt_hs, v, P.kp, q, P.cp);
    load_rows<H, NS>(P.dxbar, P.dxbar_hs, v, P.kp, g, P.cp);
    float mh[H], lh[H], T[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      mh[h] = P.stats[(v * H + h) * 2 + 0];
      lh[h] = P.stats[(v * H + h) * 2 + 1];
      T[h] = 0.f;
    }

    // Pass 1: T_h.
    for (int64_t eb = e0; eb < e1; eb += kBatch) {
      const int nb = static_cast<int>(e1 - eb < kBatch ? e1 - eb : kBatch);
      float4 x[kBatch][NS];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (b < nb) gather_x<NS>(P, sl, tw, tb, eb + b, x[b]);
        else
#pragma unroll
          for (int k = 0; k < NS; ++k) x[b][k] = f4_zero();
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        float dap[H];
#pragma unroll
        for (int h = 0; h < H; ++h) dap[h] = wave_sum(head_dot<H, NS>(g, x[b], h));
        if (b < nb) {
          const int64_t e = eb + b;
#pragma unroll
          for (int h = 0; h < H; ++h) {
            const float a = expf(P.scores[e * H + h] - mh[h]) / lh[h];
            const float dr = P.drop ? P.drop[e * H + h] : 1.f;
            T[h] = fmaf(a * dr, dap[h], T[h]);
          }
        }
      }
    }

    // Pass 2: dqt and dx_e.
    for (int64_t eb = e0; eb < e1; eb += kBatch) {
      const int nb = static_cast<int>(e1 - eb < kBatch ? e1 - eb : kBatch);
      float4 x[kBatch][NS];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (b < nb) gather_x<NS>(P, sl, tw, tb, eb + b, x[b]);
        else
#pragma unroll
          for (int k = 0; k < NS; ++k) x[b][k] = f4_zero();
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        float dap[H];
#pragma unroll
        for (int h = 0; h < H; ++h) dap[h] = wave_sum(head_dot<H, NS>(g, x[b], h));
        if (b >= nb) continue;
        const int64_t e = eb + b;
        float ad[H], dz[H];
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const float s = P.scores[e * H + h];
          const float a = expf(s - mh[h]) / lh[h];
          const float dr = P.drop ? P.drop[e * H + h] : 1.f;
          ad[h] = a * dr;
          dz[h] = a * (dr * dap[h] - T[h]) * (s > 0.f ? 1.f : P.slope);
#pragma unroll
          for (int k = 0; k < NS; ++k) fma4(dq[h][k], dz[h], x[b][k]);
        }
        const float t = P.dt_dim > 0 ? P.dt[e] : 0.f;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          const Slot s = sl[k];
          if (s.kind != kNode && s.kind != kTime) continue;
          if (s.kind == kNode && P.d_node == nullptr) continue;
          float4 dx = f4_zero();
#pragma unroll
          for (int h = 0; h < H; ++h) {
            fma4(dx, ad[h], g[h][k]);
            fma4(dx, dz[h], q[h][k]);
          }
          if (s.kind == kNode) {
            float* drow = P.d_node + e * P.ld_dnode + s.off;
            if (P.dnode_vec && s.valid == 4) {
              *reinterpret_cast<float4*>(drow) = dx;
            } else {
              if (s.valid > 0) drow[0] = dx.x;
              if (s.valid > 1) drow[1] = dx.y;
              if (s.valid > 2) drow[2] = dx.z;
              if (s.valid > 3) drow[3] = dx.w;
            }
          } else {
            // d cos(w t + b) = -sin(w t + b) * (t dw + db)
            float sn;
            if (s.valid > 0) { sn = -sinf(time_arg(t, tw[k].x, tb[k].x)) * dx.x; gb[k].x += sn; gw[k].x = fmaf(sn, t, gw[k].x); }
            if (s.valid > 1) { sn = -sinf(time_arg(t, tw[k].y, tb[k].y)) * dx.y; gb[k].y += sn; gw[k].y = fmaf(sn, t, gw[k].y); }
            if (s.valid > 2) { sn = -sinf(time_arg(t, tw[k].z, tb[k].z)) * dx.z; gb[k].z += sn; gw[k].z = fmaf(sn, t, gw[k].z); }
            if (s.valid > 3) { sn = -sinf(time_arg(t, tw[k].w, tb[k].w)) * dx.w; gb[k].w += sn; gw[k].w = fmaf(sn, t, gw[k].w); }
          }
        }
      }
    }
    store_rows<H, NS>(P.dqt, P.dqt_hs, v, P.kp, dq, P.cp);
  }

  // Time-grad partials of this workgroup: waves combined in a fixed order.
  if (P.dt_dim <= 0) return;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int base = (lane + k * kWave) * 4;
    red[wave_in_block][0][base + 0] = gw[k].x; red[wave_in_block][1][base + 0] = gb[k].x;
    red[wave_in_block][0][base + 1] = gw[k].y; red[wave_in_block][1][base + 1] = gb[k].y;
    red[wave_in_block][0][base + 2] = gw[k].z; red[wave_in_block][1][base + 2] = gb[k].z;
    red[wave_in_block][0][base + 3] = gw[k].w; red[wave_in_block][1][base + 3] = gb[k].w;
  }
  __syncthreads();
  // K-space column of time dim j: 4*(cn+ce) + j.
  const int tbase = 4 * (P.cn + P.ce);
  for (int idx = threadIdx.x; idx < 2 * P.dt_dim; idx += kBlock) {
    const int which = idx / P.dt_dim;
    const int j = idx - which * P.dt_dim;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) sum += red[w][which][tbase + j];
    P.partial[(static_cast<int64_t>(blockIdx.x) * 2 + which) * P.dt_dim + j] = sum;
  }
}

// Sums the per-workgroup partials: one wave per output value, fixed lane assignment.
__global__ __launch_bounds__(kBlock) void time_grad_reduce(const float* partial, int rows, int dt_dim,
                                                          float* d_w, float* d_b) {
  const int out = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (out >= 2 * dt_dim) return;
  const int which = out / dt_dim;
  const int j = out - which * dt_dim;
  float s = 0.f;
  for (int r = lane_id(); r < rows; r += kWave) s += partial[(static_cast<int64_t>(r) * 2 + which) * dt_dim + j];
  s = wave_sum(s);
  if (lane_id() == 0) (which == 0 ? d_w : d_b)[j] = s;
}

// Zero fill by a kernel rather than hipMemsetAsync, so the call is safe under graph capture.
__global__ __launch_bounds__(kBlock) void fill_zero(float* p, int64_t n) {
  for (int64_t i = threadIdx.x + static_cast<int64_t>(blockIdx.x) * kBlock; i < n;
       i += static_cast<int64_t>(gridDim.x) * kBlock)
    p[i] = 0.f;
}

__global__ __launch_bounds__(kBlock) void attn_weights(const int64_t* dst, int64_t n_edges,
                                                      int64_t n_dst, int heads,
                                                      const float* scores, const float* stats,
                                                      float* att) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n_edges * heads) return;
  const int64_t e = i / heads;
  const int h = static_cast<int>(i - e * heads);
  const int64_t v = dst[e];
  if (v < 0 || v >= n_dst) { att[i] = 0.f; return; }
  att[i] = expf(scores[i] - stats[(v * heads + h) * 2]) / stats[(v * heads + h) * 2 + 1];
}

__global__ __launch_bounds__(kBlock) void gather_rows(const float* tab, int64_t ld_tab, int64_t n_tab,
                                                     const int64_t* idx, int64_t n, int dim,
                                                     float* out, int64_t ld_out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (r >= n) return;
  const int64_t src = idx ? idx[r] : r;
  const bool ok = src >= 0 && src < n_tab;
  for (int c = lane_id(); c < dim; c += kWave) out[r * ld_out + c] = ok ? tab[src * ld_tab + c] : 0.f;
}

// ---------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------
int fill_params(const fa_tgat_graph* g, int heads, const float* qt, int64_t qt_hs, float slope,
                const float* drop, TgatParams& P) {
  if (!g || heads <= 0) return FA_EINVAL;
  if (g->n_dst < 0 || g->n_edges < 0 || g->dn < 0 || g->de < 0 || g->dt_dim < 0) return FA_EINVAL;
  if (g->n_edges > INT32_MAX) return FA_EUNSUPPORTED;
  if (!g->rowptr || !qt) return FA_EINVAL;
  if (g->n_edges > 0) {
    if (g->dn > 0 && (!g->node_tab || g->ld_node < g->dn)) return FA_EINVAL;
    if (g->de > 0 && (!g->edge_tab || g->ld_edge < g->de)) return FA_EINVAL;
    if (g->dt_dim > 0 && (!g->dt || !g->time_w || !g->time_b)) return FA_EINVAL;
  }
  P = TgatParams{};
  P.n_dst = g->n_dst; P.n_edges = g->n_edges; P.rowptr = g->rowptr;
  P.node_tab = g->node_tab; P.ld_node = g->ld_node; P.n_node = g->dn > 0 ? g->n_node : 0;
  P.dn = g->dn; P.node_idx = g->node_idx;
  P.edge_tab = g->edge_tab; P.ld_edge = g->ld_edge; P.n_erow = g->de > 0 ? g->n_edge_rows : 0;
  P.de = g->de; P.edge_idx = g->edge_idx;
  P.node_vec = aligned16(g->node_tab) && (g->ld_node & 3) == 0;
  P.edge_vec = aligned16(g->edge_tab) && (g->ld_edge & 3) == 0;
  P.dt = g->dt; P.time_w = g->time_w; P.time_b = g->time_b; P.dt_dim = g->dt_dim;
  P.cn = static_cast<int>(ceil_div(g->dn, 4));
  P.ce = static_cast<int>(ceil_div(g->de, 4));
  P.ct = static_cast<int>(ceil_div(g->dt_dim, 4));
  P.cp = P.cn + P.ce + P.ct + 1;
  P.kp = 4 * static_cast<int64_t>(P.cp);
  P.qt = qt; P.qt_hs = qt_hs; P.slope = slope; P.drop = drop;
  if (!aligned16(qt)) return FA_EALIGN;
  if (heads > 1 && ((qt_hs & 3) || qt_hs < P.kp * g->n_dst)) return FA_EINVAL;
  return FA_OK;
}

template <int H>
int launch_fwd_h(const TgatParams& P, hipStream_t stream) {
  const int ns = static_cast<int>(ceil_div(P.cp, kWave));
  const dim3 grid(static_cast<unsigned>(ceil_div(P.n_dst, kWavesPerBlock)));
  switch (ns) {
    case 1: hipLaunchKernelGGL((tgat_fwd<H, 1>), grid, dim3(kBlock), 0, stream, P); break;
    case 2: hipLaunchKernelGGL((tgat_fwd<H, 2>), grid, dim3(kBlock), 0, stream, P); break;
    case 3: hipLaunchKernelGGL((tgat_fwd<H, 3>), grid, dim3(kBlock), 0, stream, P); break;
    case 4: hipLaunchKernelGGL((tgat_fwd<H, 4>), grid, dim3(kBlock), 0, stream, P); break;
    default: return FA_EUNSUPPORTED;
  }
  return launch_status();
}

int bwd_grid(int64_t n_dst) {
  const int64_t want = ceil_div(n_dst, kWavesPerBlock);
  return static_cast<int>(want < kBwdMaxBlocks ? (want < 1 ? 1 : want) : kBwdMaxBlocks);
}

template <int H>
int launch_bwd_h(const TgatParams& P, int grid, hipStream_t stream) {
  const int ns = static_cast<int>(ceil_div(P.cp, kWave));
  switch (ns) {
    case 1: hipLaunchKernelGGL((tgat_bwd<H, 1>), dim3(grid), dim3(kBlock), 0, stream, P); break;
    case 2: hipLaunchKernelGGL((tgat_bwd<H, 2>), dim3(grid), dim3(kBlock), 0, stream, P); break;
    case 3: hipLaunchKernelGGL((tgat_bwd<H, 3>), dim3(grid), dim3(kBlock), 0, stream, P); break;
    case 4: hipLaunchKernelGGL((tgat_bwd<H, 4>), dim3(grid), dim3(kBlock), 0, stream, P); break;
    default: return FA_EUNSUPPORTED;
  }
  return launch_status();
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int64_t fa_tgat_kspace(int32_t dn, int32_t de, int32_t dt_dim) {
  if (dn < 0 || de < 0 || dt_dim < 0) return -1;
  return 4 * (ceil_div(dn, 4) + ceil_div(de, 4) + ceil_div(dt_dim, 4) + 1);
}

extern "C" int fa_tgat_attn_fwd_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                                    int64_t qt_hs, float slope, const float* drop, float* xbar,
                                    int64_t xbar_hs, float* scores, float* stats,
                                    hipStream_t stream) {
  TgatParams P;
  int st = fill_params(g, heads, qt, qt_hs, slope, drop, P);
  if (st != FA_OK) return st;
  if (P.n_dst == 0) return FA_OK;
  if (!xbar || !stats || (P.n_edges > 0 && !scores)) return FA_EINVAL;
  if (!aligned16(xbar) || (xbar_hs & 3) || (heads > 1 && xbar_hs < P.kp * P.n_dst)) return FA_EALIGN;
  P.xbar = xbar; P.xbar_hs = xbar_hs; P.scores = scores; P.stats = stats;
  if (static_cast<int64_t>(kBatch) * heads > kWave) return FA_EUNSUPPORTED;
  switch (heads) {
    case 1: return launch_fwd_h<1>(P, stream);
    case 2: return launch_fwd_h<2>(P, stream);
    case 4: return launch_fwd_h<4>(P, stream);
    case 8: return launch_fwd_h<8>(P, stream);
    default: return FA_EUNSUPPORTED;
  }
}

extern "C" int fa_tgat_attn_weights_f32(const int64_t* dst, int64_t n_edges, int64_t n_dst,
                                        int32_t heads, const float* scores, const float* stats,
                                        float* att, hipStream_t stream) {
  if (n_edges < 0 || n_dst < 0 || heads <= 0) return FA_EINVAL;
  if (n_edges == 0) return FA_OK;
  if (!dst || !scores || !stats || !att) return FA_EINVAL;
  hipLaunchKernelGGL(attn_weights, dim3(ceil_div(n_edges * heads, kBlock)), dim3(kBlock), 0, stream,
                     dst, n_edges, n_dst, heads, scores, stats, att);
  return launch_status();
}

extern "C" size_t fa_tgat_attn_bwd_scratch_bytes(int64_t n_dst, int32_t dt_dim) {
  if (n_dst < 0 || dt_dim < 0) return 0;
  return static_cast<size_t>(bwd_grid(n_dst)) * 2 * static_cast<size_t>(dt_dim) * sizeof(float);
}

extern "C" int fa_tgat_attn_bwd_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                                    int64_t qt_hs, float slope, const float* drop,
                                    const float* scores, const float* stats, const float* dxbar,
                                    int64_t dxbar_hs, float* dqt, int64_t dqt_hs, float* d_node,
                                    int64_t ld_dnode, float* d_time_w, float* d_time_b,
                                    void* scratch, size_t scratch_bytes, hipStream_t stream) {
  TgatParams P;
  int st = fill_params(g, heads, qt, qt_hs, slope, drop, P);
  if (st != FA_OK) return st;
  if (P.n_dst == 0) {
    if (P.dt_dim > 0 && d_time_w && d_time_b) {
      hipLaunchKernelGGL(fill_zero, dim3(1), dim3(kBlock), 0, stream, d_time_w, P.dt_dim);
      hipLaunchKernelGGL(fill_zero, dim3(1), dim3(kBlock), 0, stream, d_time_b, P.dt_dim);
    }
    return launch_status();
  }
  if (!dxbar || !dqt || !stats || (P.n_edges > 0 && !scores)) return FA_EINVAL;
  if (!aligned16(dxbar) || !aligned16(dqt) || (dxbar_hs & 3) || (dqt_hs & 3)) return FA_EALIGN;
  if (heads > 1 && (dxbar_hs < P.kp * P.n_dst || dqt_hs < P.kp * P.n_dst)) return FA_EALIGN;
  if (d_node && (P.dn <= 0 || ld_dnode < P.dn)) return FA_EINVAL;
  P.dnode_vec = d_node && aligned16(d_node) && (ld_dnode & 3) == 0;
  if (P.dt_dim > 0 && (!d_time_w || !d_time_b)) return FA_EINVAL;
  const int grid = bwd_grid(P.n_dst);
  if (P.dt_dim > 0 && (!scratch || scratch_bytes < fa_tgat_attn_bwd_scratch_bytes(P.n_dst, P.dt_dim)))
    return FA_ESCRATCH;
  P.dxbar = dxbar; P.dxbar_hs = dxbar_hs; P.dqt = dqt; P.dqt_hs = dqt_hs;
  P.d_node = d_node; P.ld_dnode = ld_dnode; P.scores = const_cast<float*>(scores);
  P.stats = const_cast<float*>(stats); P.partial = static_cast<float*>(scratch);
  if (static_cast<int64_t>(kBatch) * heads > kWave) return FA_EUNSUPPORTED;
  switch (heads) {
    case 1: st = launch_bwd_h<1>(P, grid, stream); break;
    case 2: st = launch_bwd_h<2>(P, grid, stream); break;
    case 4: st = launch_bwd_h<4>(P, grid, stream); break;
    case 8: st = launch_bwd_h<8>(P, grid, stream); break;
    default: return FA_EUNSUPPORTED;
  }
  if (st != FA_OK || P.dt_dim <= 0) return st;
  hipLaunchKernelGGL(time_grad_reduce, dim3(static_cast<unsigned>(ceil_div(2 * P.dt_dim, kWavesPerBlock))),
                     dim3(kBlock), 0, stream, P.partial, grid, P.dt_dim, d_time_w, d_time_b);
  return launch_status();
}

extern "C" int fa_gather_rows_f32(const float* tab, int64_t ld_tab, int64_t n_tab,
                                  const int64_t* idx, int64_t n, int32_t dim, float* out,
                                  int64_t ld_out, hipStream_t stream) {
  if (n < 0 || dim < 0 || n_tab < 0) return FA_EINVAL;
  if (n == 0 || dim == 0) return FA_OK;
  if (!tab || !out || ld_tab < dim || ld_out < dim) return FA_EINVAL;
  hipLaunchKernelGGL(gather_rows, dim3(static_cast<unsigned>(ceil_div(n, kWavesPerBlock))), dim3(kBlock), 0,
                     stream, tab, ld_tab, n_tab, idx, n, dim, out, ld_out);
  return launch_status();
}
