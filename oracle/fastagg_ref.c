/*
 * fastagg_ref.c - CPU restatement of the FAST fastAgg operators.
 *
 * TEST INFRASTRUCTURE ONLY: the checker that the gfx950 kernels are compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may load it; the product
 * never calls it.
 *
 * Each function follows the cited reference kernel with its intended semantics (every edge
 * and every head covered; see the notes on the reference's index defects). Scalar loops in
 * edge order; built with -ffp-contract=off so every float operation rounds as written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define MAX_SEED (-1e38f) /* edge_softmax.cu:271 */

static int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* exclusive_sum_cuda (getFastAgg/cuda_operators/utils.cu:16-40): the input padded with one
 * trailing 0 is exclusive-scanned, giving [0, c0, c0+c1, ..., total] (n+1 values). int32
 * arithmetic wraps. */
void ref_exclusive_sum_i32(const int32_t* in, int64_t n, int32_t* out) {
  uint32_t acc = 0;
  out[0] = 0;
  for (int64_t i = 0; i < n; ++i) {
    acc += (uint32_t)in[i];
    out[i + 1] = (int32_t)acc;
  }
}

/* cal_deg_cuda (utils.cu:42-78): deg[edges[i]] += 1; ids outside [0, n_nodes) ignored. */
void ref_degree_count_i32(const int32_t* ids, int64_t n_ids, int32_t* deg, int64_t n_nodes) {
  memset(deg, 0, sizeof(int32_t) * (size_t)n_nodes);
  for (int64_t i = 0; i < n_ids; ++i)
    if (ids[i] >= 0 && ids[i] < n_nodes) deg[ids[i]] += 1;
}

/* getBalancedPtrKernel (utils.cu:81-114): for i < n-1, deg_i = ptr[i+1]-ptr[i];
 * P_i = inclusive prefix of deg over the aligned block of 256 entries containing i;
 * mask[i] = P_i/T > (P_i - deg_i)/T with C truncating division. */
void ref_balance_mask_i32(const int32_t* ptr, int64_t n, int32_t threshold, int32_t* mask) {
  uint32_t run = 0;
  for (int64_t i = 0; i + 1 < n; ++i) {
    if (i % 256 == 0) run = 0;
    const uint32_t deg = (uint32_t)ptr[i + 1] - (uint32_t)ptr[i];
    const int32_t before = (int32_t)run;
    run += deg;
    const int32_t after = (int32_t)run;
    mask[i] = (after / threshold > before / threshold) ? 1 : 0;
  }
}

/* Full-CSR offsets of a destination-sorted edge list: rowptr[v] = #edges with dst < v. */
void ref_rowptr_from_sorted_dst(const int64_t* dst, int64_t n_edges, int64_t n_dst, int32_t* rowptr) {
  int64_t e = 0;
  for (int64_t v = 0; v <= n_dst; ++v) {
    while (e < n_edges && dst[e] < v) ++e;
    rowptr[v] = (int32_t)e;
  }
}

/* forward_edge_softmax_cuda_kernel (edge_softmax.cu:255-293) for mode 0,
 * forward_csr_edge_softmax_cuda_kernel (edge_softmax.cu:450-518) formula for mode 1
 * (division instead of reciprocal multiply), every segment edge covered. */
void ref_edge_softmax_fwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges, const float* x,
                              int64_t ldx, int32_t heads, float* y, int64_t ldy, int32_t mode) {
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t lb = clamp64(indptr[s], 0, n_edges), le = clamp64(indptr[s + 1], 0, n_edges);
    for (int h = 0; h < heads; ++h) {
      float mx = MAX_SEED;
      for (int64_t e = lb; e < le; ++e) mx = fmaxf(mx, x[e * ldx + h]);
      float sum = 0.f;
      for (int64_t e = lb; e < le; ++e) sum += expf(x[e * ldx + h] - mx);
      if (mode == 0) {
        const float inv = 1.f / sum;
        for (int64_t e = lb; e < le; ++e) y[e * ldy + h] = expf(x[e * ldx + h] - mx) * inv;
      } else {
        for (int64_t e = lb; e < le; ++e) y[e * ldy + h] = expf(x[e * ldx + h] - mx) / sum;
      }
    }
  }
}

/* backward_edge_softmax_cuda_kernel (edge_softmax.cu:295-329):
 * dx = y * (dy - sum_seg y*dy). */
void ref_edge_softmax_bwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges, const float* dy,
                              int64_t lddy, const float* y, int64_t ldy, int32_t heads, float* dx,
                              int64_t lddx) {
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t lb = clamp64(indptr[s], 0, n_edges), le = clamp64(indptr[s + 1], 0, n_edges);
    for (int h = 0; h < heads; ++h) {
      float acc = 0.f;
      for (int64_t e = lb; e < le; ++e) acc += y[e * ldy + h] * dy[e * lddy + h];
      for (int64_t e = lb; e < le; ++e) dx[e * lddx + h] = y[e * ldy + h] * (dy[e * lddy + h] - acc);
    }
  }
}

/* forward/backward_balanced_edge_softmax_cuda_kernel (edge_softmax.cu:330-448): batch b
 * covers edges bptr[b]..bptr[b+1]; its j-th edge has group key[b*ld_key+j]; softmax over
 * the edges of each (batch, key, head); j >= ld_key or key outside [0, ld_key) skipped. */
void ref_group_softmax_fwd_f32(const int64_t* bptr, int64_t n_batch, const int64_t* key,
                               int64_t ld_key, int64_t n_edges, const float* x, int64_t ldx,
                               int32_t heads, float* y, int64_t ldy) {
  for (int64_t b = 0; b < n_batch; ++b) {
    const int64_t lb = clamp64(bptr[b], 0, n_edges), le = clamp64(bptr[b + 1], 0, n_edges);
    int64_t lim = le > lb ? le - lb : 0;
    if (lim > ld_key) lim = ld_key;
    const int64_t* kr = key + b * ld_key;
    for (int64_t j = 0; j < lim; ++j) {
      const int64_t k = kr[j];
      if (k < 0 || k >= ld_key) continue;
      for (int h = 0; h < heads; ++h) {
        float mx = MAX_SEED, sum = 0.f;
        for (int64_t i = 0; i < lim; ++i)
          if (kr[i] == k) mx = fmaxf(mx, x[(lb + i) * ldx + h]);
        for (int64_t i = 0; i < lim; ++i)
          if (kr[i] == k) sum += expf(x[(lb + i) * ldx + h] - mx);
        y[(lb + j) * ldy + h] = expf(x[(lb + j) * ldx + h] - mx) / sum;
      }
    }
  }
}

void ref_group_softmax_bwd_f32(const int64_t* bptr, int64_t n_batch, const int64_t* key,
                               int64_t ld_key, int64_t n_edges, const float* dy, int64_t lddy,
                               const float* y, int64_t ldy, int32_t heads, float* dx, int64_t lddx) {
  for (int64_t b = 0; b < n_batch; ++b) {
    const int64_t lb = clamp64(bptr[b], 0, n_edges), le = clamp64(bptr[b + 1], 0, n_edges);
    int64_t lim = le > lb ? le - lb : 0;
    if (lim > ld_key) lim = ld_key;
    const int64_t* kr = key + b * ld_key;
    for (int64_t j = 0; j < lim; ++j) {
      const int64_t k = kr[j];
      if (k < 0 || k >= ld_key) continue;
      for (int h = 0; h < heads; ++h) {
        float acc = 0.f;
        for (int64_t i = 0; i < lim; ++i)
          if (kr[i] == k) acc += y[(lb + i) * ldy + h] * dy[(lb + i) * lddy + h];
        dx[(lb + j) * lddx + h] = y[(lb + j) * ldy + h] * (dy[(lb + j) * lddy + h] - acc);
      }
    }
  }
}

/* computation_aware_forward_tgat_cuda_kernel (aggregate_acc_kernel.cu:72-94) over every
 * edge: out[dst[e]] += x[src[e]]; with indptr only edges indptr[0]..indptr[n_seg]. */
void ref_edge_scatter_sum_f32(const int64_t* dst, const int64_t* src, int64_t n_edges,
                              const int32_t* indptr, int64_t n_seg, const float* x, int64_t ldx,
                              int64_t n_x, int32_t dim, float* out, int64_t ldo, int64_t n_out) {
  int64_t lo = 0, hi = n_edges;
  if (indptr) {
    lo = clamp64(indptr[0], 0, n_edges);
    hi = clamp64(indptr[n_seg], 0, n_edges);
  }
  for (int64_t e = lo; e < hi; ++e) {
    if (dst[e] < 0 || dst[e] >= n_out || src[e] < 0 || src[e] >= n_x) continue;
    for (int c = 0; c < dim; ++c) out[dst[e] * ldo + c] += x[src[e] * ldx + c];
  }
}

/* computation_aware_forward_tgat_shd_cuda_kernel (aggregate_shd_kernel.cu:161-209): the sum
 * of the segment's source rows, written to the segment's destination. */
void ref_segment_sum_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst, const int64_t* src,
                         int64_t n_edges, const float* x, int64_t ldx, int64_t n_x, int32_t dim,
                         float* out, int64_t ldo, int64_t n_out) {
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t lb = clamp64(indptr[s], 0, n_edges), le = clamp64(indptr[s + 1], 0, n_edges);
    if (le <= lb) continue;
    const int64_t d = dst[lb];
    if (d < 0 || d >= n_out) continue;
    for (int c = 0; c < dim; ++c) {
      float acc = 0.f;
      for (int64_t e = lb; e < le; ++e)
        if (src[e] >= 0 && src[e] < n_x) acc += x[src[e] * ldx + c];
      out[d * ldo + c] = acc;
    }
  }
}

static float leaky(float z, float slope) { return z > 0.f ? z : z * slope; }

/* forward_fused_attn_cuda_kernel (fused_attention.cu:203-328), intended semantics:
 * attn = softmax_seg(leaky(score)); kept (mask > p) entries scaled by 1/(1-p) evaluated in
 * double; out[dst] = sum_e w * V[src[e]-n_dst]. */
void ref_fused_attn_fwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst, const int64_t* src,
                            int64_t n_edges, int64_t n_dst, const float* score, const float* V,
                            int32_t heads, int32_t dh, float slope, float p, const float* mask,
                            float* attn, float* out) {
  const int dim = heads * dh;
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t lb = clamp64(indptr[s], 0, n_edges), le = clamp64(indptr[s + 1], 0, n_edges);
    if (le <= lb) continue;
    for (int h = 0; h < heads; ++h) {
      float mx = MAX_SEED, sm = 0.f;
      for (int64_t e = lb; e < le; ++e) mx = fmaxf(mx, leaky(score[e * heads + h], slope));
      for (int64_t e = lb; e < le; ++e) sm += expf(leaky(score[e * heads + h], slope) - mx);
      for (int64_t e = lb; e < le; ++e)
        attn[e * heads + h] = expf(leaky(score[e * heads + h], slope) - mx) / sm;
    }
    const int64_t d = dst[lb];
    if (d < 0 || d >= n_dst) continue;
    for (int c = 0; c < dim; ++c) {
      const int h = c / dh;
      float acc = 0.f;
      for (int64_t e = lb; e < le; ++e) {
        const int64_t row = src[e] - n_dst;
        if (row < 0 || row >= n_edges) continue;
        const float a = attn[e * heads + h];
        float w = a;
        if (mask) w = mask[e * heads + h] > p ? (float)((double)a / (1.0 - (double)p)) : 0.f;
        acc = fmaf(w, V[row * dim + c], acc);
      }
      out[d * dim + c] = acc;
    }
  }
}

/* backward_fused_attn_cuda_kernel (fused_attention.cu:330-446), intended semantics:
 * grad_V[row] += attn*keep*dout[dst]; da = keep * dout[dst,h].V[row,h];
 * d_act = attn*(da - sum_seg attn*da) (gradient of the LeakyReLU output). */
void ref_fused_attn_bwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst, const int64_t* src,
                            int64_t n_edges, int64_t n_dst, int64_t n_src, const float* dout,
                            const float* V, const float* attn, const float* mask, int32_t heads,
                            int32_t dh, float p, float* d_act, float* grad_V) {
  const int dim = heads * dh;
  const float keep = (float)(1.0 / (1.0 - (double)p));
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t lb = clamp64(indptr[s], 0, n_edges), le = clamp64(indptr[s + 1], 0, n_edges);
    if (le <= lb) continue;
    const int64_t d = dst[lb];
    if (d < 0 || d >= n_dst) continue;
    for (int h = 0; h < heads; ++h) {
      float tsum = 0.f;
      for (int64_t e = lb; e < le; ++e) {
        const int64_t row = src[e] - n_dst;
        float da = 0.f;
        if (row >= 0 && row < n_edges && src[e] < n_src) {
          const float kf = mask ? (mask[e * heads + h] > p ? keep : 0.f) : 1.f;
          const float a = attn[e * heads + h];
          for (int c = h * dh; c < (h + 1) * dh; ++c) {
            grad_V[row * dim + c] += a * kf * dout[d * dim + c];
            da += kf * dout[d * dim + c] * V[row * dim + c];
          }
        }
        d_act[e * heads + h] = da;
        tsum = fmaf(attn[e * heads + h], da, tsum);
      }
      for (int64_t e = lb; e < le; ++e)
        d_act[e * heads + h] = attn[e * heads + h] * (d_act[e * heads + h] - tsum);
    }
  }
}

/* Counter-based dropout multipliers of the fused TGAT kernels: entry i kept iff
 * (hash(seed, i) >> 8) / 2^24 >= p, hash = two rounds of the murmur3 32-bit finaliser. */
static uint32_t ref_mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  return x;
}

void ref_dropout_mask_f32(uint64_t seed, float p, int64_t n, float* out) {
  const float scale = (float)(1.0 / (1.0 - (double)p));
  for (int64_t i = 0; i < n; ++i) {
    uint32_t x = ref_mix32((uint32_t)i ^ (uint32_t)seed);
    x = ref_mix32(x + (uint32_t)(seed >> 32) + (uint32_t)((uint64_t)i >> 32) * 0x9e3779b9u);
    const float u = (float)(x >> 8) * (1.0f / 16777216.0f);
    out[i] = u >= p ? scale : 0.f;
  }
}
