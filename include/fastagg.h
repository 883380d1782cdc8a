/*
 * fastagg.h - C ABI of the MI355X (gfx950) temporal-attention aggregation library
 * (libfastagg_hip.so).
 *
 * Every entry point:
 *   - takes device pointers, element counts, leading dimensions (in elements) and a
 *     hipStream_t; no torch types cross this boundary;
 *   - enqueues its kernels on `stream` and returns without synchronising;
 *   - allocates nothing: scratch, when needed, is passed in by the caller and its size is
 *     given by the matching *_scratch_bytes() query;
 *   - returns FA_OK (0), a negative FA_E* argument error, or a positive hipError_t from
 *     the launch.
 *
 * Index conventions follow the FAST reference (getFastAgg/cuda_operators):
 *   indptr / CSR offsets are int32, per-edge node ids are int64, features are row-major.
 *
 * "Segment" = the run of edges that share one destination node in a CSR over edges
 * sorted by destination ("cntE" from getSamplerCore/sampler_core.cpp:384-409).
 */
#ifndef FASTAGG_H
#define FASTAGG_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FA_OK = 0,
  FA_EINVAL = -1,       /* bad size, null pointer or inconsistent dimensions */
  FA_EUNSUPPORTED = -2, /* shape outside what the kernels are built for (e.g. heads) */
  FA_EALIGN = -3,       /* pointer or leading dimension not 16-byte aligned */
  FA_ESCRATCH = -4      /* caller scratch too small */
};

/* Human-readable text for a status returned by any entry point. */
const char* fa_status_string(int status);
/* Library ABI version (major*100 + minor). */
int fa_abi_version(void);

/* ---------------------------------------------------------------------------------
 * Segment bookkeeping (bit-exact integer work)
 * ------------------------------------------------------------------------------- */

/* out[0] = 0, out[i+1] = out[i] + in[i] for i < n (int32 wrap-around), n+1 outputs.
 * Replaces exclusive_sum_cuda (getFastAgg/cuda_operators/utils.cu:16-40) and the
 * binding fastAgg.exclusive_sum (operators.cpp:580-586). */
size_t fa_exclusive_sum_scratch_bytes(int64_t n);
int fa_exclusive_sum_i32(const int32_t* in, int64_t n, int32_t* out, void* scratch,
                         size_t scratch_bytes, hipStream_t stream);

/* deg[ids[i]] += 1 for every i with 0 <= ids[i] < n_nodes; deg must be zeroed by the
 * caller. Replaces cal_deg_cuda (utils.cu:42-78) / fastAgg.cal_deg (operators.cpp:588-595). */
int fa_degree_count_i32(const int32_t* ids, int64_t n_ids, int32_t* deg, int64_t n_nodes,
                        hipStream_t stream);

/* mask[i] = (P_i / threshold > P'_i / threshold) for i < n-1 where deg_i =
 * dense_ptr[i+1]-dense_ptr[i], P_i the inclusive prefix of deg inside the aligned block of
 * 256 entries holding i, P'_i the same prefix without deg_i; C (truncating) division.
 * Replaces getBalancedPtrKernel / get_balanced_cuda (utils.cu:81-141) and
 * fastAgg.getBalancedPtr (operators.cpp:597-604). threshold must be non-zero. */
int fa_balance_mask_i32(const int32_t* dense_ptr, int64_t n, int32_t threshold, int32_t* mask,
                        hipStream_t stream);

/* rowptr[v] = first edge e with dst[e] >= v, for v = 0..n_dst (rowptr has n_dst+1 entries),
 * for dst sorted ascending. The full-CSR form of the sampler's compressed cntE: it also
 * covers zero-degree destinations. Used by the fused TGAT kernels (no reference
 * counterpart; derives the segment->destination map of layers.py:174-183). */
int fa_rowptr_from_sorted_dst_i64(const int64_t* dst, int64_t n_edges, int64_t n_dst,
                                  int32_t* rowptr, hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Segmented edge softmax (drop-in kernels of edge_softmax.cu)
 * ------------------------------------------------------------------------------- */

/* For each segment s < n_seg (edges indptr[s]..indptr[s+1]) and head h < heads:
 *   mode 0 (reciprocal): y = exp(x - max) * (1 / sum)   forward_edge_softmax
 *   mode 1 (division)  : y = exp(x - max) / sum         forward_csr_edge_softmax
 * with max seeded at -1e38. Entries of edges outside every segment are set to zero (the
 * reference's zero-initialised output). float32 rows of exactly `heads` values with heads in
 * {1, 2, 4, 8, 16} run one 16-lane row per segment (coalesced, max and sum combined in a
 * tree); other shapes and float64 one thread per (segment, head), summing in edge order.
 * Replaces forward_edge_softmax_cuda (edge_softmax.cu:55-78, 255-293) and
 * forward_csr_edge_softmax_cuda (edge_softmax.cu:178-206, 450-518). */
int fa_edge_softmax_fwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                            const float* x, int64_t ldx, int32_t heads, float* y, int64_t ldy,
                            int32_t mode, hipStream_t stream);
int fa_edge_softmax_fwd_f64(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                            const double* x, int64_t ldx, int32_t heads, double* y,
                            int64_t ldy, int32_t mode, hipStream_t stream);

/* dx = y * (dy - sum_segment(y * dy)) per segment and head h < heads; the first `heads`
 * values of rows outside every segment are set to zero (same kernels as the forward).
 * Replaces backward_edge_softmax_cuda (edge_softmax.cu:79-106, 295-329) and
 * backward_csr_edge_softmax_cuda (edge_softmax.cu:207-235, 520-577). */
int fa_edge_softmax_bwd_f32(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                            const float* dy, int64_t lddy, const float* y, int64_t ldy,
                            int32_t heads, float* dx, int64_t lddx, hipStream_t stream);
int fa_edge_softmax_bwd_f64(const int32_t* indptr, int64_t n_seg, int64_t n_edges,
                            const double* dy, int64_t lddy, const double* y, int64_t ldy,
                            int32_t heads, double* dx, int64_t lddx, hipStream_t stream);

/* Grouped ("balanced") softmax: batch b covers edges batch_ptr[b]..batch_ptr[b+1]; the
 * j-th edge of batch b belongs to group key[b*ld_key + j] (0 <= key < ld_key; edges with
 * j >= ld_key or an out-of-range key are skipped). Softmax (division form) / its gradient
 * over the edges of each (batch, key, head). Replaces
 * forward/backward_balanced_edge_softmax_cuda (edge_softmax.cu:107-176, 330-448). */
int fa_group_softmax_fwd_f32(const int64_t* batch_ptr, int64_t n_batch, const int64_t* key,
                             int64_t ld_key, int64_t n_edges, const float* x, int64_t ldx,
                             int32_t heads, float* y, int64_t ldy, hipStream_t stream);
int fa_group_softmax_bwd_f32(const int64_t* batch_ptr, int64_t n_batch, const int64_t* key,
                             int64_t ld_key, int64_t n_edges, const float* dy, int64_t lddy,
                             const float* y, int64_t ldy, int32_t heads, float* dx,
                             int64_t lddx, hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Sum aggregation over edges (drop-in kernels of aggregate_*_kernel.cu)
 * ------------------------------------------------------------------------------- */

/* out[r, :] = sum of x[src[e], :] over the edges e with dst[e] = r, for e < n_edges (COO, any
 * order; ids outside [0, n_out) / [0, n_x) are skipped; x rows outside [0, n_x) read as zero).
 * When indptr is not NULL only the edges indptr[0] <= e < indptr[n_seg] are used. Every row
 * of out (dim values) is written: rows no edge reaches get zeros. The kernels check on the
 * device whether dst is sorted (non-decreasing): if so, each output row is the sum of one run
 * of edges, summed in edge order by the run's owner and written with plain stores
 * (deterministic, no atomics); otherwise out is zero-filled and runs of equal consecutive dst
 * are added with atomics (the result may then depend on the order of the additions).
 * dim <= 1024 (FA_EUNSUPPORTED beyond). scratch: fa_edge_scatter_sum_scratch_bytes().
 * Replaces computation_aware_forward_tgat_cuda (aggregate_acc_kernel.cu:36-94), with every
 * edge covered. Also the backward of forward_tgat / forward_tgat_shd with the roles of dst
 * and src swapped (aggregate_acc_kernel.cu:97-161, aggregate_shd_kernel.cu:212-368). */
size_t fa_edge_scatter_sum_scratch_bytes(void);
int fa_edge_scatter_sum_f32(const int64_t* dst, const int64_t* src, int64_t n_edges,
                            const int32_t* indptr, int64_t n_seg, const float* x, int64_t ldx,
                            int64_t n_x, int32_t dim, float* out, int64_t ldo, int64_t n_out,
                            void* scratch, size_t scratch_bytes, hipStream_t stream);

/* CSR segment sum: for segment s, out[dst[indptr[s]], :] = sum_e x[src[e], :] over the
 * segment (edges of a segment share one destination). Rows of out outside every segment
 * are not written. dim <= 1024 (FA_EUNSUPPORTED beyond). Replaces
 * computation_aware_forward_tgat_shd_cuda (aggregate_shd_kernel.cu:37-94, 161-209). */
int fa_segment_sum_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                       const int64_t* src, int64_t n_edges, const float* x, int64_t ldx,
                       int64_t n_x, int32_t dim, float* out, int64_t ldo, int64_t n_out,
                       hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Fused LeakyReLU + segment softmax + dropout + aggregation (drop-in fused_attention.cu)
 * ------------------------------------------------------------------------------- */

/* Segment s (edges indptr[s]..indptr[s+1], destination dst[indptr[s]]):
 *   attn[e,h] = softmax_s(leaky_relu(score[e,h], slope))
 *   keep      = mask[e,h] > p ? 1/(1-p) : 0
 *   out[dst,h*dh+d] = sum_e attn[e,h]*keep*V[src[e]-n_dst, h, d]
 * out rows outside every segment are not written (caller zero-fills).
 * Replaces forward_fused_attn_cuda (fused_attention.cu:68-138, 203-328). */
int fa_fused_attn_fwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                          const int64_t* src, int64_t n_edges, int64_t n_dst,
                          const float* score, const float* V, int32_t heads, int32_t dh,
                          float slope, float p, const float* mask, float* attn, float* out,
                          hipStream_t stream);
/* Gradients of fa_fused_attn_fwd_f32 given dout [n_dst, heads*dh]:
 *   grad_V[src[e]-n_dst,h,:] = attn*keep*dout[dst,h,:]
 *   d_act[e,h] = attn*(da - sum_s attn*da), da = keep * dout[dst,h,:].V[...]
 * i.e. the gradient with respect to the LeakyReLU *output*; the caller applies
 * leaky_relu'(score). Every row of grad_V [n_edges][heads*dh] is written (it need not be
 * zeroed): rows no edge contributes to are zeros. It is accumulated with atomics after a
 * zero fill, except that with scratch (fa_fused_attn_bwd_scratch_bytes() bytes, or NULL),
 * heads in {1, 2, 4, 8} and rows of at most 128 values, a device check that every in-range
 * V row is its own edge's (src[e] - n_dst == e, the sampler's layout) and that the segment
 * offsets never decrease lets each row be stored once instead (zeros for the rows of edges
 * outside the segments, of segments whose destination is out of range and of edges whose
 * source is out of range), with no fill in front.
 * Replaces backward_fused_attn_cuda (fused_attention.cu:139-200, 330-446). */
size_t fa_fused_attn_bwd_scratch_bytes(void);
int fa_fused_attn_bwd_f32(const int32_t* indptr, int64_t n_seg, const int64_t* dst,
                          const int64_t* src, int64_t n_edges, int64_t n_dst, int64_t n_src,
                          const float* dout, const float* V, const float* attn,
                          const float* mask, int32_t heads, int32_t dh, float p,
                          float* d_act, float* grad_V, void* scratch, size_t scratch_bytes,
                          hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Fused TGAT temporal attention (the hot path of layers.py:98-240, TGAT branch)
 *
 * Per edge e the key/value input row is x_e = [h_src(e) | f(e) | cos(w*dt_e + b) | 1]
 * in "K-space": node features padded to Pn = roundup(Dn,4), edge features to
 * Pe = roundup(De,4), time encoding to Pt = roundup(Dt,4), then the constant 1 at
 * column Kb = Pn+Pe+Pt, zero-padded to Kp = roundup(Kb+1,4).
 * K and V are never formed per edge: with q~[v,h,:] = Q[v,h,:] W_k,aug[h] (bias in
 * column Kb) the score is q~.x_e, and the aggregation returns
 * xbar[v,h,:] = sum_e a'[e,h] x_e (column Kb = sum_e a'), to which the caller applies
 * W_v,aug. Destination v owns edges rowptr[v]..rowptr[v+1] (clamped to [0, n_edges]).
 * ------------------------------------------------------------------------------- */

enum { FA_F32 = 0, FA_BF16 = 1 };  /* element type of a feature table */

typedef struct fa_tgat_graph {
  int64_t n_dst;           /* destinations (including zero-degree ones) */
  int64_t n_edges;
  const int32_t* rowptr;   /* [n_dst+1] full CSR over dst-sorted edges */
  /* node part: row of edge e = node_idx ? node_idx[e] : e; rows >= n_node read as 0.
   * node_dtype FA_F32 or FA_BF16 (widened to float in registers); ld in elements. When
   * ld is a multiple of 4 and the table 16-byte (float32) / 8-byte (bf16) aligned, each row
   * may be read up to the next multiple of 4 past dn (values ignored), so the allocation
   * must cover that padding; otherwise rows are read element by element. Same for edges. */
  const void* node_tab; int64_t ld_node; int64_t n_node; int32_t dn; const int64_t* node_idx;
  int32_t node_dtype;
  /* edge part: row of edge e = edge_idx ? edge_idx[e] : e; rows >= n_edge_rows read as 0 */
  const void* edge_tab; int64_t ld_edge; int64_t n_edge_rows; int32_t de;
  const int64_t* edge_idx; int32_t edge_dtype;
  /* time part */
  const float* dt;         /* [n_edges] */
  const float* time_w;     /* [dt_dim] */
  const float* time_b;     /* [dt_dim] */
  int32_t dt_dim;
} fa_tgat_graph;

/* K-space width Kp for the given dims (all > = 0). */
int64_t fa_tgat_kspace(int32_t dn, int32_t de, int32_t dt_dim);

/* Forward. Per-destination blocks are rows of Kp floats: the qt row of destination v and
 * head h starts at qt + v*qt_rs + h*qt_hs (16-byte aligned, strides multiples of 4), so
 * (qt_rs, qt_hs) = (heads*Kp, Kp) is a [n_dst][heads][Kp] array and (Kp, n_dst*Kp) a
 * [heads][n_dst][Kp] one; xbar, dxbar and dqt below take their own strides. Inputs may
 * repeat rows (stride 0); the rows of an output must not overlap (destination-major:
 * rs >= heads*hs, hs >= Kp; or head-major: hs >= n_dst*rs, rs >= Kp).
 * Attention dropout: drop = optional explicit [n_edges][heads] multipliers (keep/(1-p) or
 * 0); when drop is NULL and drop_p > 0, entry (e,h) is kept iff the counter-based hash of
 * (drop_seed, e*heads+h) clears drop_p (see fa_dropout_mask_f32); drop_p = 0: no dropout.
 * Outputs: xbar, scores [n_edges][heads] (post-LeakyReLU),
 * stats [n_dst][heads][2] = (max, sum of exp). */
int fa_tgat_attn_fwd_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                         int64_t qt_rs, int64_t qt_hs, float slope, const float* drop,
                         uint64_t drop_seed, float drop_p, float* xbar, int64_t xbar_rs,
                         int64_t xbar_hs, float* scores, float* stats, hipStream_t stream);

/* The multipliers of the hashed attention dropout: out[i] = 1/(1-p) if
 * (hash(seed, i) >> 8) / 2^24 >= p else 0, for i < n (i = e*heads + h). */
int fa_dropout_mask_f32(uint64_t seed, float p, int64_t n, float* out, hipStream_t stream);

/* Normalised attention att[e,h] = exp(score - max[dst]) / sum[dst] (pre-dropout), for
 * callers that want the weights themselves. dst: [n_edges] int64 in [0, n_dst). */
int fa_tgat_attn_weights_f32(const int64_t* dst, int64_t n_edges, int64_t n_dst, int32_t heads,
                             const float* scores, const float* stats, float* att,
                             hipStream_t stream);

/* Backward, one pass over the edges. xbar: the forward output (its dot product with dxbar
 * gives each destination's softmax correction); tdot: that dot product itself, [n_dst][heads]
 * (may be NULL; when given, xbar is not read and may be NULL; a caller holding
 * agg = W_v xbar and its gradient has it as dagg . agg); dxbar: gradient of xbar. Outputs: dqt
 * (strides dqt_rs, dqt_hs); d_node [n_edges][ld_dnode] gradient of the
 * node-feature part of every x_e (may be NULL); d_time_w/d_time_b [dt_dim] (may be NULL
 * when dt_dim == 0). scratch: fa_tgat_attn_bwd_scratch_bytes(g->n_dst, dt_dim).
 * dt_dim <= 256, and d_node only with a float32 node table (FA_EUNSUPPORTED otherwise). */
size_t fa_tgat_attn_bwd_scratch_bytes(int64_t n_dst, int32_t dt_dim);
int fa_tgat_attn_bwd_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                         int64_t qt_rs, int64_t qt_hs, float slope, const float* drop,
                         uint64_t drop_seed, float drop_p, const float* xbar, int64_t xbar_rs,
                         int64_t xbar_hs, const float* tdot, const float* scores, const float* stats,
                         const float* dxbar, int64_t dxbar_rs, int64_t dxbar_hs, float* dqt,
                         int64_t dqt_rs, int64_t dqt_hs, float* d_node, int64_t ld_dnode,
                         float* d_time_w, float* d_time_b, void* scratch,
                         size_t scratch_bytes, hipStream_t stream);

/* The backward above without caller scratch, for callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, outputs and limits as fa_tgat_attn_bwd_f32; the time-gradient partials
 * live in a static device array of 4 MiB per GPU (held until the process ends; enough for
 * every shape the backward takes: at most 2048 workgroups x 2 x dt_dim <= 256 floats), a
 * shape needing more returns FA_ESCRATCH. It calls no hipMalloc/hipFree. The current
 * device must be the one `stream` belongs to. All calls on one GPU share its array: calls
 * that overlap in time on one GPU (different streams, no ordering) race. */
int fa_tgat_attn_bwd_noalloc_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                                 int64_t qt_rs, int64_t qt_hs, float slope, const float* drop,
                                 uint64_t drop_seed, float drop_p, const float* xbar,
                                 int64_t xbar_rs, int64_t xbar_hs, const float* tdot,
                                 const float* scores, const float* stats, const float* dxbar,
                                 int64_t dxbar_rs, int64_t dxbar_hs, float* dqt, int64_t dqt_rs,
                                 int64_t dqt_hs, float* d_node, int64_t ld_dnode,
                                 float* d_time_w, float* d_time_b, hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Per-head projections of the K-space blocks (new ops: the reference applies w_q, w_k,
 * w_v per edge as torch GEMMs, layers.py:162-169). G heads, J = dim_out/heads (<= 64),
 * C = Kp columns; W[g][j][c] = w[g*wg + j*ldw + c]. Float32 in and out, on the matrix
 * cores: where the rows allow, every operand is split into three bf16 parts (hi + mid + lo =
 * the float exactly) and the six products above 2^-16 of the whole are summed in float32
 * (the bf16 MFMA); otherwise the float32 MFMA. Either keeps float32 accuracy.
 * ------------------------------------------------------------------------------- */

/* Y[g][n][c] = sum_j X[n][j] W[g][j][c] (+ bias[g*bg + c] when bias != NULL), with
 * X[n][j] = x[n*ldx + g*xg + j] and Y[g][n][c] = y[g*yg + n*ldy + c]. */
int fa_head_proj_f32(int64_t n, int32_t j, int32_t c, int32_t groups, const float* x,
                     int64_t ldx, int64_t xg, const float* w, int64_t wg, int64_t ldw,
                     const float* bias, int64_t bg, float* y, int64_t yg, int64_t ldy,
                     hipStream_t stream);

/* Z[n][g][j] = z[n*ldz + g*zg + j] = sum_c Y[g][n][c] W[g][j][c]
 * (the transpose product of fa_head_proj_f32), Y[g][n][c] = y[g*yg + n*ldy + c].
 * W[g] is held in LDS (160 KiB): as three bf16 parts, (j+1) x (c rounded up to 64, + 8)
 * each, when Y's rows are whole 16-byte chunks (y 16-byte aligned, ldy, yg and c multiples
 * of 4); else as float32 chunks, (j+1) x (c rounded up to 64) floats. A shape that fits
 * neither returns FA_EUNSUPPORTED (e.g. j = 64 with c > 512 on unaligned rows, or
 * c > 680 on any rows); fa_head_reduce_supported tells beforehand. */
int fa_head_reduce_f32(int64_t n, int32_t j, int32_t c, int32_t groups, const float* y,
                       int64_t yg, int64_t ldy, const float* w, int64_t wg, int64_t ldw,
                       float* z, int64_t ldz, int64_t zg, hipStream_t stream);
/* Whether fa_head_reduce_f32 takes (j, c, ldy) with rows of whole 16-byte chunks (rows16 != 0)
 * or not: 2 on the split-bf16 kernel, 1 on the float32 kernel, 0 unsupported
 * (FA_EUNSUPPORTED). No device access. */
int fa_head_reduce_supported(int32_t j, int32_t c, int64_t ldy, int32_t rows16);

/* dw[g][j][c] = sum_n X[n][j] Y[g][n][c] (X, Y as in fa_head_proj_f32 / fa_head_reduce_f32),
 * [groups][j + ones][c] contiguous; with ones != 0 row j holds sum_n Y[g][n][c] (the
 * gradient of a per-column bias). Partial sums over row chunks go to scratch
 * (fa_head_wgrad_scratch_bytes) and are added in a fixed order: results are deterministic. */
size_t fa_head_wgrad_scratch_bytes(int64_t n, int32_t j, int32_t c, int32_t groups,
                                   int32_t ones);
int fa_head_wgrad_f32(int64_t n, int32_t j, int32_t c, int32_t groups, const float* x,
                      int64_t ldx, int64_t xg, const float* y, int64_t yg, int64_t ldy,
                      int32_t ones, float* dw, void* scratch, size_t scratch_bytes,
                      hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Fused layer epilogue (layers.py:224-237: w_out, dropout, ReLU, LayerNorm). New op: the
 * reference runs these as separate torch kernels.
 * ------------------------------------------------------------------------------- */

/* For each row r < n of width d (d <= 256):
 *   u = r1[r] + r2[r] + bias (r2, bias may be NULL), y = relu(u * m), m = the hashed
 *   dropout multiplier of entry r*d + c (1/(1-p) or 0, as fa_dropout_mask_f32 with
 *   drop_seed; m = 1 when drop_p = 0), out = (y - mean) * rstd * gamma + beta with
 *   rstd = 1/sqrt(var + eps) (biased variance over the row).
 * Saves y [n][d] and stats [n][2] = (mean, rstd) for the backward. */
int fa_tgat_epilogue_fwd_f32(int64_t n, int32_t d, const float* r1, int64_t ld1,
                             const float* r2, int64_t ld2, const float* bias,
                             const float* gamma, const float* beta, float eps,
                             uint64_t drop_seed, float drop_p, float* out, float* y,
                             float* stats, hipStream_t stream);
/* Gradients of fa_tgat_epilogue_fwd_f32 from dout [n][d]: du [n][d] (the gradient of r1, r2
 * and each row of bias), dgamma [d], dbeta [d] and, when dbias is not NULL,
 * dbias [d] = sum over rows of du (deterministic two-pass sums).
 * scratch: fa_tgat_epilogue_bwd_scratch_bytes(n, d). */
size_t fa_tgat_epilogue_bwd_scratch_bytes(int64_t n, int32_t d);
int fa_tgat_epilogue_bwd_f32(int64_t n, int32_t d, const float* dout, const float* y,
                             const float* stats, const float* gamma, float drop_p, float* du,
                             float* dgamma, float* dbeta, float* dbias, void* scratch,
                             size_t scratch_bytes, hipStream_t stream);

/* Per-row, per-group dot products (new op, no reference counterpart: it gives the fused
 * backward its per-destination correction in D-space, dagg . agg, instead of reading xbar):
 * out[r*groups + g] = sum_{j < width} a[r*lda + g*width + j] * b[r*ldb + g*width + j]. */
int fa_row_group_dots_f32(int64_t n, int32_t groups, int32_t width, const float* a, int64_t lda,
                          const float* b, int64_t ldb, float* out, hipStream_t stream);

/* Per-step parameter preparation of one layer (new op: the reference applies w_q, w_k, w_v,
 * w_out and the time encoding directly, layers.py:105-169; here their weights enter the
 * fused path in K-space form). d = dim_out, dn/de/dt the input widths, all row-major float32:
 * W_q [d][dn+dt] (row stride ldq), W_k, W_v [d][dn+de+dt], W_o [d][d+dn], b_t [dt].
 * Forward outputs: wq_node = W_q[:, :dn] [d][dn]; wk_aug, wv_aug [d][Kp] (= [heads][d/heads][Kp],
 * fa_tgat_kspace layout, bias at column Kp-4); qbk [heads][Kp] = qb[h-block] wk_aug[h-block] with
 * qb = b_q + W_q[:, dn:] cos(b_t); wo1 = W_o[:, :d] [d][d]; wo2 = W_o[:, d:] [d][dn].
 * Backward: the gradients of the forward's inputs from those of its outputs (each g_* may be
 * NULL for a zero gradient); d_* are written whole. dn > 0, d <= 512. scratch: 2*d floats
 * (FA_ESCRATCH when NULL). */
int fa_layer_params_fwd_f32(int32_t d, int32_t heads, int32_t dn, int32_t de, int32_t dt,
                            const float* wq, int64_t ldq, const float* bq, const float* wk,
                            int64_t ldk, const float* bk, const float* wv, int64_t ldv,
                            const float* bv, const float* bt, const float* wo, int64_t ldo,
                            float* wq_node, float* wk_aug, float* wv_aug, float* qbk, float* wo1,
                            float* wo2, float* scratch, hipStream_t stream);
int fa_layer_params_bwd_f32(int32_t d, int32_t heads, int32_t dn, int32_t de, int32_t dt,
                            const float* wq, int64_t ldq, const float* bq, const float* wk,
                            int64_t ldk, const float* bk, const float* bt,
                            const float* g_wq_node, const float* g_wk_aug, const float* g_wv_aug,
                            const float* g_qbk, const float* g_wo1, const float* g_wo2,
                            float* d_wq, float* d_bq, float* d_wk, float* d_bk, float* d_wv,
                            float* d_bv, float* d_bt, float* d_wo, float* scratch,
                            hipStream_t stream);

/* Row gather: out[i, :dim] = tab[idx[i], :dim] (idx NULL => i). */
int fa_gather_rows_f32(const float* tab, int64_t ld_tab, int64_t n_tab, const int64_t* idx,
                       int64_t n, int32_t dim, float* out, int64_t ld_out, hipStream_t stream);
/* The same from a bf16 table (raw 16-bit words), widened to float. */
int fa_gather_rows_bf16_f32(const uint16_t* tab, int64_t ld_tab, int64_t n_tab,
                            const int64_t* idx, int64_t n, int32_t dim, float* out,
                            int64_t ld_out, hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * TGN node memory (memorys.py:6-304). The state of a MailBox is node_memory
 * [num_nodes][m], node_memory_ts [num_nodes], mailbox [num_nodes][slots][2m + de] (rows of
 * ld_mailbox floats), mailbox_ts [num_nodes][slots] and next_pos [num_nodes] (int64).
 * Node ids are int32 (ids_are_int64 = 0) or int64; an id outside [0, num_nodes) gathers
 * zeros and writes nothing.
 * ------------------------------------------------------------------------------- */

/* Per source row i: mem_out[i] = node_memory[ids[i]], mem_ts_out[i] = node_memory_ts[ids[i]],
 * x_out[i, 0:mail_width] = mailbox[ids[i]] (the slots' mails, flattened), mail_ts_out[i] =
 * mailbox_ts[ids[i]]. Replaces MailBox.prep_input_mails (memorys.py:57-71), writing the mails
 * into the rows of the memory updater's input. */
int fa_mail_gather_f32(int64_t n, const void* ids, int32_t ids_are_int64, int64_t num_nodes,
                       const float* memory, int64_t ld_memory, int32_t dim_memory,
                       const float* memory_ts, const float* mailbox, int64_t ld_mailbox,
                       int64_t mail_width, const float* mailbox_ts, int32_t slots,
                       float* mem_out, int64_t ld_mem_out, float* mem_ts_out, float* x_out,
                       int64_t ld_x, float* mail_ts_out, hipStream_t stream);

/* out[i, j] = cos(w[j] * t_i + b[j]), t_i = ts[i] - mem_ts[i] (mem_ts NULL => ts[i]), j < dt,
 * the product and the sum rounded separately as in the reference's Linear(1, dt). The time
 * features of GRUMemeoryUpdater.forward (memorys.py:288-290, layers.py:17-29). */
int fa_time_rows_f32(int64_t n, const float* ts, const float* mem_ts, const float* w,
                     const float* b, int32_t dt, float* out, int64_t ld_out, hipStream_t stream);
/* Their gradient: dw[j] = sum_i -sin(w[j] t_i + b[j]) t_i g[i, j], db[j] the same without t_i.
 * Fixed-order sums (deterministic); scratch of fa_time_rows_grad_scratch_bytes(dt). */
size_t fa_time_rows_grad_scratch_bytes(int32_t dt);
int fa_time_rows_grad_f32(int64_t n, const float* ts, const float* mem_ts, const float* w,
                          const float* b, int32_t dt, const float* g, int64_t ld_g, float* dw,
                          float* db, void* scratch, size_t scratch_bytes, hipStream_t stream);

/* Elementwise part of torch.nn.GRUCell (memorys.py:291): gi = x W_ih^T + b_ih and
 * gh = h W_hh^T + b_hh with gate blocks [r | z | n], each m wide; hy = (1 - z) c + z h with
 * r = sigmoid(gi_r + gh_r), z = sigmoid(gi_z + gh_z), c = tanh(gi_n + r gh_n) (h NULL => 0).
 * b_ih / b_hh [3m] (each optional): gi / gh come without that bias, which is added here.
 * workspace [n][4m] keeps r, z, c, gh_n (with its bias) for fa_gru_bwd_f32. */
int fa_gru_fwd_f32(int64_t n, int32_t m, const float* gi, int64_t ld_gi, const float* gh,
                   int64_t ld_gh, const float* h, int64_t ld_h, const float* b_ih,
                   const float* b_hh, float* hy, int64_t ld_hy, float* workspace,
                   hipStream_t stream);
/* dgi, dgh [n][3m] (the gradients of gi and gh) from dhy; dh (optional) = dhy z, the direct
 * path only (the caller adds dgh W_hh). With db_ih and db_hh (both or neither) also the bias
 * gradients db_ih = sum over rows of dgi, db_hh = the same of dgh (fixed-order sums,
 * deterministic), through scratch of fa_gru_bwd_scratch_bytes(n, m). */
size_t fa_gru_bwd_scratch_bytes(int64_t n, int32_t m);
int fa_gru_bwd_f32(int64_t n, int32_t m, const float* dhy, int64_t ld_dhy, const float* workspace,
                   const float* h, int64_t ld_h, float* dgi, int64_t ld_dgi, float* dgh,
                   int64_t ld_dgh, float* dh, int64_t ld_dh, float* db_ih, float* db_hh,
                   void* scratch, size_t scratch_bytes, hipStream_t stream);
/* torch.nn.RNNCell with tanh (RNNMemeoryUpdater, memorys.py:332): hy = tanh(gi + gh), plus
 * b_ih / b_hh [m] (each optional) where gi / gh come without them; the backward gives
 * da = dhy (1 - hy^2), the gradient of both gi and gh. */
int fa_rnn_fwd_f32(int64_t n, int32_t m, const float* gi, int64_t ld_gi, const float* gh,
                   int64_t ld_gh, const float* b_ih, const float* b_hh, float* hy, int64_t ld_hy,
                   hipStream_t stream);
int fa_rnn_bwd_f32(int64_t n, int32_t m, const float* dhy, int64_t ld_dhy, const float* hy,
                   int64_t ld_hy, float* da, int64_t ld_da, hipStream_t stream);

/* node_memory[ids[r]] = mem[r], node_memory_ts[ids[r]] = ts[r] for r < rows, the last row of
 * each id winning (MailBox.update_memory, memorys.py:84-103, whose device index_put leaves the
 * winner among repeated ids unspecified). `last` [num_nodes] holds one tag per node, zero at
 * first use and kept by the caller between calls; `generation` must be non-zero and grow with
 * every call that shares `last` (rows < 2^32). */
int fa_memory_update_f32(int64_t rows, const void* ids, int32_t ids_are_int64, const float* mem,
                         int64_t ld_mem, int32_t dim_memory, const float* ts, float* node_memory,
                         int64_t ld_node_memory, float* node_memory_ts, int64_t num_nodes,
                         unsigned long long* last, uint32_t generation, hipStream_t stream);

/* MailBox.update_mailbox for deliver_to 'self', mail_combine 'last' (memorys.py:105-139):
 * n edges with sources src_ids and destinations dst_ids; write rows interleaved
 * (src_0, dst_0, src_1, ...). Row 2k writes [mem[k], mem[n+k], edge_feats[k]] for src_ids[k],
 * row 2k+1 writes [mem[n+k], mem[k], edge_feats[k]] for dst_ids[k]; row r's time is ts[r] (the
 * reference pairs the interleaved mails with ts[:2n] in its own order). The last row of each
 * node wins; it writes slot next_pos[node] and, with slots > 1, advances next_pos by one
 * modulo slots. `last` and `generation` as in fa_memory_update_f32 (2n < 2^32). */
int fa_mailbox_update_f32(int64_t n, const void* src_ids, const void* dst_ids,
                          int32_t ids_are_int64, const float* mem, int64_t ld_mem,
                          int32_t dim_memory, const float* edge_feats, int64_t ld_edge,
                          int32_t dim_edge, const float* ts, float* mailbox, int64_t ld_mailbox,
                          float* mailbox_ts, int64_t* next_pos, int32_t slots, int64_t num_nodes,
                          unsigned long long* last, uint32_t generation, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTAGG_H */
