// PyTorch-ROCm binding "fastAgg": the operator names, positional argument order, tensor
// layouts and return types of the FAST reference module
// (getFastAgg/cuda_operators/operators.cpp:606-625), implemented by the C ABI of
// libfastagg_hip.so (include/fastagg.h), plus the fused TGAT operators of this build.
//
// Every op validates its tensors (device, contiguity, dtype, shape) before any launch,
// allocates its outputs with torch on the inputs' device, enqueues on torch's current
// stream and never synchronises. Outputs that the reference returns as fresh zeros are
// allocated as zeros here too.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cstdlib>
#include <optional>
#include <vector>

#include "fastagg.h"

namespace {

// Same checks and messages as the reference (operators.cpp:4-6).
#define CHECK_CUDA(x) TORCH_CHECK((x).is_cuda(), #x " must be a CUDA tensor")
#define CHECK_CONTIGUOUS(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define CHECK_INPUT(x) \
  CHECK_CUDA(x);       \
  CHECK_CONTIGUOUS(x)
#define CHECK_DTYPE(x, t) \
  TORCH_CHECK((x).scalar_type() == (t), #x " must have dtype ", (t), ", got ", (x).scalar_type())
#define CHECK_DIM(x, d) TORCH_CHECK((x).dim() == (d), #x " must be ", (d), "-D, got ", (x).dim(), "-D")
#define CHECK_SAME_DEVICE(a, b) \
  TORCH_CHECK((a).device() == (b).device(), #a " and " #b " must be on the same device")

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_status(int st, const char* op) {
  TORCH_CHECK(st == FA_OK, "fastAgg.", op, ": ", fa_status_string(st), " (status ", st, ")");
}

// Optional NaN report on an output (FASTAGG_DEBUG_NAN=1), in place of the reference's
// unconditional device-to-host copies; it synchronises, so it is off by default.
void debug_nan(const at::Tensor& t, const char* op) {
  static const bool on = [] {
    const char* v = std::getenv("FASTAGG_DEBUG_NAN");
    return v && v[0] == '1';
  }();
  if (on && t.numel() > 0 && at::isnan(t).any().item<bool>())
    TORCH_WARN("fastAgg.", op, ": output contains NaN");
}

int64_t num_segments(const at::Tensor& indptr) { return indptr.numel() > 0 ? indptr.numel() - 1 : 0; }

// ----------------------------------------------------------------------------------
// Segmented softmax (edge_softmax.cu)
// ----------------------------------------------------------------------------------
at::Tensor softmax_fwd_impl(const at::Tensor& indptr, const at::Tensor& x, int64_t heads, int mode,
                            const char* op) {
  CHECK_DTYPE(indptr, at::kInt);
  CHECK_DIM(x, 2);
  CHECK_SAME_DEVICE(indptr, x);
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "input_feat must be float32 or float64");
  TORCH_CHECK(heads >= 0 && heads <= x.size(1), op, ": num_heads (", heads,
              ") must lie in [0, input_feat.size(1)=", x.size(1), "]");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  // every entry is written: softmax values in the segments, zeros outside them
  auto y = at::empty({x.size(0), heads}, x.options());
  const int64_t S = num_segments(indptr);
  int st;
  if (x.scalar_type() == at::kFloat)
    st = fa_edge_softmax_fwd_f32(indptr.data_ptr<int32_t>(), S, x.size(0), x.data_ptr<float>(),
                                 x.size(1), heads, y.data_ptr<float>(), heads, mode, stream_of(x));
  else
    st = fa_edge_softmax_fwd_f64(indptr.data_ptr<int32_t>(), S, x.size(0), x.data_ptr<double>(),
                                 x.size(1), heads, y.data_ptr<double>(), heads, mode, stream_of(x));
  check_status(st, op);
  debug_nan(y, op);
  return y;
}

at::Tensor softmax_bwd_impl(const at::Tensor& indptr, const at::Tensor& dy, const at::Tensor& y,
                            int64_t heads, const char* op) {
  CHECK_DTYPE(indptr, at::kInt);
  CHECK_DIM(dy, 2);
  CHECK_SAME_DEVICE(indptr, dy);
  CHECK_SAME_DEVICE(y, dy);
  TORCH_CHECK(dy.scalar_type() == at::kFloat || dy.scalar_type() == at::kDouble,
              "d_output must be float32 or float64");
  TORCH_CHECK(y.scalar_type() == dy.scalar_type(), "output and d_output must share a dtype");
  TORCH_CHECK(y.dim() == 2 && y.size(0) == dy.size(0) && y.size(1) >= heads,
              op, ": output must be [E, >=num_heads] with E = d_output.size(0)");
  TORCH_CHECK(heads >= 0 && heads <= dy.size(1), op, ": num_heads (", heads,
              ") must lie in [0, d_output.size(1)=", dy.size(1), "]");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(dy.device());
  // the kernels write the first num_heads columns of every row (zeros outside the
  // segments); wider outputs keep zeros in the other columns
  auto dx = heads == dy.size(1) ? at::empty({dy.size(0), dy.size(1)}, dy.options())
                                : at::zeros({dy.size(0), dy.size(1)}, dy.options());
  const int64_t S = num_segments(indptr);
  int st;
  if (dy.scalar_type() == at::kFloat)
    st = fa_edge_softmax_bwd_f32(indptr.data_ptr<int32_t>(), S, dy.size(0), dy.data_ptr<float>(),
                                 dy.size(1), y.data_ptr<float>(), y.size(1), heads,
                                 dx.data_ptr<float>(), dx.size(1), stream_of(dy));
  else
    st = fa_edge_softmax_bwd_f64(indptr.data_ptr<int32_t>(), S, dy.size(0), dy.data_ptr<double>(),
                                 dy.size(1), y.data_ptr<double>(), y.size(1), heads,
                                 dx.data_ptr<double>(), dx.size(1), stream_of(dy));
  check_status(st, op);
  debug_nan(dx, op);
  return dx;
}

// forward_edge_softmax (operators.cpp:167-205): output [E, num_heads].
std::vector<at::Tensor> forward_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                             at::Tensor input_feat, int64_t node_num_per_block,
                                             int64_t num_heads) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(input_feat);
  (void)node_num_per_block;  // launch tuning in the reference; no effect on the result
  return {softmax_fwd_impl(indptr, input_feat, num_heads, 0, "forward_edge_softmax")};
}

// backward_edge_softmax (operators.cpp:385-427): d_input [E, d_output.size(1)], heads < num_heads.
std::vector<at::Tensor> backward_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                              at::Tensor d_output, at::Tensor output,
                                              int64_t node_num_per_block, int64_t num_heads) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(d_output);
  CHECK_INPUT(output);
  (void)node_num_per_block;
  return {softmax_bwd_impl(indptr, d_output, output, num_heads, "backward_edge_softmax")};
}

// forward_csr_edge_softmax (operators.cpp:246-284): every head, any degree.
std::vector<at::Tensor> forward_csr_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                                 at::Tensor input_feat, int64_t node_num_per_block,
                                                 int64_t reduce_size) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(input_feat);
  (void)node_num_per_block;
  (void)reduce_size;
  CHECK_DIM(input_feat, 2);
  return {softmax_fwd_impl(indptr, input_feat, input_feat.size(1), 1, "forward_csr_edge_softmax")};
}

// backward_csr_edge_softmax (operators.cpp:470-512): every head of d_output.
std::vector<at::Tensor> backward_csr_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                                  at::Tensor d_output, at::Tensor output,
                                                  int64_t node_num_per_block, int64_t reduce_size) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(d_output);
  CHECK_INPUT(output);
  (void)node_num_per_block;
  (void)reduce_size;
  CHECK_DIM(d_output, 2);
  return {softmax_bwd_impl(indptr, d_output, output, d_output.size(1), "backward_csr_edge_softmax")};
}

// forward/backward_balanced_edge_softmax (operators.cpp:207-245, 428-469): batches of edges
// (int64 indptr [B+1]) with a 2-D int64 local-node-id table indices [B, maxN].
void check_balanced(const at::Tensor& indptr, const at::Tensor& indices, const at::Tensor& x) {
  CHECK_DTYPE(indptr, at::kLong);
  CHECK_DTYPE(indices, at::kLong);
  CHECK_DIM(indices, 2);
  CHECK_DIM(x, 2);
  CHECK_DTYPE(x, at::kFloat);
  CHECK_SAME_DEVICE(indptr, x);
  CHECK_SAME_DEVICE(indices, x);
  TORCH_CHECK(indptr.numel() >= indices.size(0) + 1,
              "indptr must hold indices.size(0)+1 batch offsets");
}

std::vector<at::Tensor> forward_balanced_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                                      at::Tensor input_feat,
                                                      int64_t edge_num_per_block,
                                                      int64_t reduce_size) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(input_feat);
  (void)edge_num_per_block;
  (void)reduce_size;
  check_balanced(indptr, indices, input_feat);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(input_feat.device());
  auto y = at::zeros_like(input_feat);
  const int st = fa_group_softmax_fwd_f32(
      indptr.data_ptr<int64_t>(), indices.size(0), indices.data_ptr<int64_t>(), indices.size(1),
      input_feat.size(0), input_feat.data_ptr<float>(), input_feat.size(1), input_feat.size(1),
      y.data_ptr<float>(), y.size(1), stream_of(input_feat));
  check_status(st, "forward_balanced_edge_softmax");
  debug_nan(y, "forward_balanced_edge_softmax");
  return {y};
}

std::vector<at::Tensor> backward_balanced_edge_softmax(at::Tensor indptr, at::Tensor indices,
                                                       at::Tensor d_output, at::Tensor output,
                                                       int64_t node_num_per_block,
                                                       int64_t reduce_size) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(d_output);
  CHECK_INPUT(output);
  (void)node_num_per_block;
  (void)reduce_size;
  check_balanced(indptr, indices, d_output);
  CHECK_DTYPE(output, at::kFloat);
  TORCH_CHECK(output.sizes() == d_output.sizes(), "output and d_output must have the same shape");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(d_output.device());
  auto dx = at::zeros_like(d_output);
  const int st = fa_group_softmax_bwd_f32(
      indptr.data_ptr<int64_t>(), indices.size(0), indices.data_ptr<int64_t>(), indices.size(1),
      d_output.size(0), d_output.data_ptr<float>(), d_output.size(1), output.data_ptr<float>(),
      output.size(1), d_output.size(1), dx.data_ptr<float>(), dx.size(1), stream_of(d_output));
  check_status(st, "backward_balanced_edge_softmax");
  debug_nan(dx, "backward_balanced_edge_softmax");
  return {dx};
}

// ----------------------------------------------------------------------------------
// Sum aggregation (aggregate_acc_kernel.cu, aggregate_shd_kernel.cu)
// ----------------------------------------------------------------------------------
void check_edge_pair(const at::Tensor& a, const at::Tensor& b, const at::Tensor& x) {
  CHECK_DTYPE(a, at::kLong);
  CHECK_DTYPE(b, at::kLong);
  CHECK_DIM(a, 1);
  CHECK_DIM(b, 1);
  TORCH_CHECK(a.numel() == b.numel(), "edge id arrays must have the same length");
  CHECK_DIM(x, 2);
  CHECK_DTYPE(x, at::kFloat);
  CHECK_SAME_DEVICE(a, x);
  CHECK_SAME_DEVICE(b, x);
}

// out [n_out, x.size(1)] = the scatter sum of x rows src[e] into rows dst[e] (every row written).
at::Tensor scatter_sum(const at::Tensor& dst, const at::Tensor& src, const int32_t* indptr,
                       int64_t n_seg, const at::Tensor& x, int64_t n_out, const char* op) {
  auto out = at::empty({n_out, x.size(1)}, x.options());
  auto scratch = at::empty({static_cast<int64_t>(fa_edge_scatter_sum_scratch_bytes())},
                           x.options().dtype(at::kByte));
  const int st = fa_edge_scatter_sum_f32(
      dst.data_ptr<int64_t>(), src.data_ptr<int64_t>(), dst.numel(), indptr, n_seg,
      x.data_ptr<float>(), x.size(1), x.size(0), static_cast<int32_t>(x.size(1)),
      out.data_ptr<float>(), out.size(1), n_out, scratch.data_ptr(), scratch.numel(), stream_of(x));
  check_status(st, op);
  return out;
}

// forward_tgat (operators.cpp:146-165): out[src_edges[e]] += input_feat[dst_edges[e]]
// for every edge (the reference argument names: src_edges holds destination ids).
std::vector<at::Tensor> forward_tgat(at::Tensor src_edges, at::Tensor dst_edges,
                                     at::Tensor input_feat, int64_t dst_num, int64_t aggNodePB,
                                     int64_t aggFeat) {
  CHECK_INPUT(src_edges);
  CHECK_INPUT(dst_edges);
  CHECK_INPUT(input_feat);
  (void)aggNodePB;
  (void)aggFeat;
  check_edge_pair(src_edges, dst_edges, input_feat);
  TORCH_CHECK(dst_num >= 0, "dst_num must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(input_feat.device());
  return {scatter_sum(src_edges, dst_edges, nullptr, 0, input_feat, dst_num, "forward_tgat")};
}

// backward_tgat (operators.cpp:364-384): d_out[dst_edges[e]] += d_input[src_edges[e]].
std::vector<at::Tensor> backward_tgat(at::Tensor src_edges, at::Tensor dst_edges, at::Tensor d_input,
                                      int64_t src_num, int64_t aggNodePB, int64_t aggFeat) {
  CHECK_INPUT(src_edges);
  CHECK_INPUT(dst_edges);
  CHECK_INPUT(d_input);
  (void)aggNodePB;
  (void)aggFeat;
  check_edge_pair(src_edges, dst_edges, d_input);
  TORCH_CHECK(src_num >= 0, "src_num must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(d_input.device());
  return {scatter_sum(dst_edges, src_edges, nullptr, 0, d_input, src_num, "backward_tgat")};
}

// forward_tgat_shd (operators.cpp:120-145): CSR segment sum written to the segment's dst.
std::vector<at::Tensor> forward_tgat_shd(at::Tensor indptr, at::Tensor indices, at::Tensor src_edges,
                                         at::Tensor dst_edges, at::Tensor input_feat,
                                         int64_t dst_nodes, int64_t aggNodePB, int64_t aggFeat) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(src_edges);
  CHECK_INPUT(dst_edges);
  CHECK_INPUT(input_feat);
  (void)aggNodePB;
  (void)aggFeat;
  CHECK_DTYPE(indptr, at::kInt);
  CHECK_SAME_DEVICE(indptr, input_feat);
  check_edge_pair(src_edges, dst_edges, input_feat);
  TORCH_CHECK(dst_nodes >= 0, "dst_nodes must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(input_feat.device());
  auto out = at::zeros({dst_nodes, input_feat.size(1)}, input_feat.options());
  const int st = fa_segment_sum_f32(
      indptr.data_ptr<int32_t>(), num_segments(indptr), src_edges.data_ptr<int64_t>(),
      dst_edges.data_ptr<int64_t>(), src_edges.numel(), input_feat.data_ptr<float>(),
      input_feat.size(1), input_feat.size(0), static_cast<int32_t>(input_feat.size(1)),
      out.data_ptr<float>(), out.size(1), dst_nodes, stream_of(input_feat));
  check_status(st, "forward_tgat_shd");
  return {out};
}

// backward_tgat_shd (operators.cpp:337-363): the transpose of forward_tgat_shd,
// d_out[src_edges[e]] += d_input[dst_edges[e]] over the edges of the segments (the
// reference argument names: dst_edges holds destination ids here).
std::vector<at::Tensor> backward_tgat_shd(at::Tensor indptr, at::Tensor indices,
                                          at::Tensor dst_edges, at::Tensor src_edges,
                                          at::Tensor d_input, int64_t src_nodes, int64_t aggNodePB,
                                          int64_t aggFeat) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(dst_edges);
  CHECK_INPUT(src_edges);
  CHECK_INPUT(d_input);
  (void)aggNodePB;
  (void)aggFeat;
  CHECK_DTYPE(indptr, at::kInt);
  CHECK_SAME_DEVICE(indptr, d_input);
  check_edge_pair(dst_edges, src_edges, d_input);
  TORCH_CHECK(src_nodes >= 0, "src_nodes must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(d_input.device());
  const int64_t S = num_segments(indptr);
  return {scatter_sum(src_edges, dst_edges, S > 0 ? indptr.data_ptr<int32_t>() : nullptr, S,
                      d_input, src_nodes, "backward_tgat_shd")};
}

// ----------------------------------------------------------------------------------
// Fused LeakyReLU + softmax + dropout + aggregation (fused_attention.cu)
// ----------------------------------------------------------------------------------
void check_fused(const at::Tensor& scores_like, const at::Tensor& V, const at::Tensor& indptr,
                 const at::Tensor& dst_eid, const at::Tensor& src_eid, int64_t num_heads) {
  CHECK_INPUT(V);
  CHECK_INPUT(dst_eid);
  CHECK_INPUT(src_eid);
  CHECK_DIM(scores_like, 2);
  CHECK_DTYPE(scores_like, at::kFloat);
  CHECK_DIM(V, 3);
  CHECK_DTYPE(V, at::kFloat);
  CHECK_DTYPE(indptr, at::kInt);
  CHECK_DTYPE(dst_eid, at::kLong);
  CHECK_DTYPE(src_eid, at::kLong);
  TORCH_CHECK(dst_eid.numel() == scores_like.size(0) && src_eid.numel() == scores_like.size(0),
              "dst_eid / src_eid must have one entry per edge");
  TORCH_CHECK(num_heads == scores_like.size(1), "num_heads must equal the score width");
  TORCH_CHECK(V.size(0) == scores_like.size(0) && V.size(1) == num_heads,
              "V_val must be [E, num_heads, dh]");
  TORCH_CHECK(num_heads <= 64, "at most 64 heads are supported");
  for (const at::Tensor* t : {&V, &indptr, &dst_eid, &src_eid}) CHECK_SAME_DEVICE((*t), scores_like);
}

// forward_fused_attn (operators.cpp:285-333) -> [out_agg, attn, edge_mask].
std::vector<at::Tensor> forward_fused_attn(at::Tensor input_feat, at::Tensor V_val, at::Tensor indptr,
                                           at::Tensor indices, at::Tensor dst_eid,
                                           at::Tensor src_eid, int64_t node_num, int64_t num_heads,
                                           double negative_slope, double attn_drop) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(input_feat);
  check_fused(input_feat, V_val, indptr, dst_eid, src_eid, num_heads);
  TORCH_CHECK(node_num >= 0, "node_num must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(input_feat.device());
  const int64_t E = input_feat.size(0), H = num_heads, dh = V_val.size(2);
  auto attn = at::zeros({E, H}, input_feat.options());
  auto out = at::zeros({node_num, H * dh}, input_feat.options());
  // Dropout mask U[0,1) from torch's generator (the reference draws it with cuRAND).
  auto edge_mask = at::rand({E, H}, input_feat.options());
  const int st = fa_fused_attn_fwd_f32(
      indptr.data_ptr<int32_t>(), num_segments(indptr), dst_eid.data_ptr<int64_t>(),
      src_eid.data_ptr<int64_t>(), E, node_num, input_feat.data_ptr<float>(),
      V_val.data_ptr<float>(), static_cast<int32_t>(H), static_cast<int32_t>(dh),
      static_cast<float>(negative_slope), static_cast<float>(attn_drop),
      edge_mask.data_ptr<float>(), attn.data_ptr<float>(), out.data_ptr<float>(),
      stream_of(input_feat));
  check_status(st, "forward_fused_attn");
  debug_nan(out, "forward_fused_attn");
  return {out, attn, edge_mask};
}

// backward_fused_attn (operators.cpp:513-565) -> [d_input, grad_V]; d_input is the
// gradient with respect to the LeakyReLU output.
std::vector<at::Tensor> backward_fused_attn(at::Tensor d_output, at::Tensor V_val, at::Tensor output,
                                            at::Tensor edge_mask, at::Tensor indptr,
                                            at::Tensor indices, at::Tensor dst_eid,
                                            at::Tensor src_eid, int64_t node_num, int64_t num_heads,
                                            double negative_slope, double attn_drop) {
  CHECK_INPUT(indptr);
  CHECK_INPUT(indices);
  CHECK_INPUT(d_output);
  CHECK_INPUT(output);
  CHECK_INPUT(edge_mask);
  (void)negative_slope;
  check_fused(output, V_val, indptr, dst_eid, src_eid, num_heads);
  CHECK_DTYPE(edge_mask, at::kFloat);
  TORCH_CHECK(edge_mask.sizes() == output.sizes(), "edge_mask must match output");
  CHECK_DIM(d_output, 2);
  CHECK_DTYPE(d_output, at::kFloat);
  TORCH_CHECK(d_output.size(1) == num_heads * V_val.size(2), "d_output must be [N, num_heads*dh]");
  CHECK_SAME_DEVICE(d_output, output);
  CHECK_SAME_DEVICE(edge_mask, output);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(output.device());
  const int64_t E = output.size(0), H = num_heads, dh = V_val.size(2);
  auto d_input = at::zeros({E, H}, output.options());
  auto grad_V = at::empty({E, H, dh}, output.options());   // every row is written by the call
  const size_t sb = fa_fused_attn_bwd_scratch_bytes();
  auto scratch = at::empty({static_cast<int64_t>(sb)}, output.options().dtype(at::kByte));
  const int st = fa_fused_attn_bwd_f32(
      indptr.data_ptr<int32_t>(), num_segments(indptr), dst_eid.data_ptr<int64_t>(),
      src_eid.data_ptr<int64_t>(), E, d_output.size(0), node_num, d_output.data_ptr<float>(),
      V_val.data_ptr<float>(), output.data_ptr<float>(), edge_mask.data_ptr<float>(),
      static_cast<int32_t>(H), static_cast<int32_t>(dh), static_cast<float>(attn_drop),
      d_input.data_ptr<float>(), grad_V.data_ptr<float>(), scratch.data_ptr(), sb,
      stream_of(output));
  check_status(st, "backward_fused_attn");
  debug_nan(d_input, "backward_fused_attn");
  return {d_input, grad_V};
}

// ----------------------------------------------------------------------------------
// Bookkeeping (utils.cu)
// ----------------------------------------------------------------------------------
// exclusive_sum (operators.cpp:580-586): int32 [n] -> int32 [n+1] = [0, cumsum].
at::Tensor exclusive_sum(at::Tensor in_degs) {
  CHECK_INPUT(in_degs);
  CHECK_DTYPE(in_degs, at::kInt);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(in_degs.device());
  const int64_t n = in_degs.numel();
  auto out = at::empty({n + 1}, in_degs.options());
  const size_t sb = fa_exclusive_sum_scratch_bytes(n);
  auto scratch = at::empty({static_cast<int64_t>(sb)}, in_degs.options().dtype(at::kByte));
  const int st = fa_exclusive_sum_i32(in_degs.data_ptr<int32_t>(), n, out.data_ptr<int32_t>(),
                                      scratch.data_ptr(), sb, stream_of(in_degs));
  check_status(st, "exclusive_sum");
  return out;
}

// cal_deg (operators.cpp:588-595): int32 histogram of edges over [0, nodes_num).
at::Tensor cal_deg(at::Tensor edges, int64_t nodes_num) {
  CHECK_INPUT(edges);
  CHECK_DTYPE(edges, at::kInt);
  TORCH_CHECK(nodes_num >= 0, "nodes_num must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(edges.device());
  auto deg = at::zeros({nodes_num}, edges.options());
  const int st = fa_degree_count_i32(edges.data_ptr<int32_t>(), edges.numel(),
                                     deg.data_ptr<int32_t>(), nodes_num, stream_of(edges));
  check_status(st, "cal_deg");
  return deg;
}

// getBalancedPtr (operators.cpp:597-604): int32 mask [n-1].
at::Tensor getBalancedPtr(at::Tensor densePtr, int64_t threshold) {
  CHECK_INPUT(densePtr);
  CHECK_DTYPE(densePtr, at::kInt);
  TORCH_CHECK(densePtr.numel() >= 1, "densePtr must hold at least one offset");
  TORCH_CHECK(threshold != 0, "threshold must be non-zero");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(densePtr.device());
  const int64_t n = densePtr.numel();
  auto mask = at::zeros({n - 1}, densePtr.options());
  const int st = fa_balance_mask_i32(densePtr.data_ptr<int32_t>(), n, static_cast<int32_t>(threshold),
                                     mask.data_ptr<int32_t>(), stream_of(densePtr));
  check_status(st, "getBalancedPtr");
  return mask;
}

// ----------------------------------------------------------------------------------
// Fused TGAT operators of this build (no reference counterpart)
// ----------------------------------------------------------------------------------
int64_t tgat_kspace(int64_t dn, int64_t de, int64_t dt_dim) {
  return fa_tgat_kspace(static_cast<int32_t>(dn), static_cast<int32_t>(de), static_cast<int32_t>(dt_dim));
}

// int32 [n_dst+1] full-CSR offsets from dst-sorted int64 destination ids.
at::Tensor rowptr_from_dst(at::Tensor dst, int64_t n_dst) {
  CHECK_INPUT(dst);
  CHECK_DTYPE(dst, at::kLong);
  CHECK_DIM(dst, 1);
  TORCH_CHECK(n_dst >= 0, "n_dst must be >= 0");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(dst.device());
  auto rowptr = at::empty({n_dst + 1}, dst.options().dtype(at::kInt));
  const int st = fa_rowptr_from_sorted_dst_i64(dst.data_ptr<int64_t>(), dst.numel(), n_dst,
                                               rowptr.data_ptr<int32_t>(), stream_of(dst));
  check_status(st, "rowptr_from_dst");
  return rowptr;
}

void check_table(const at::Tensor& t, const char* name) {
  CHECK_CUDA(t);
  TORCH_CHECK(t.dim() == 2, name, " must be 2-D");
  TORCH_CHECK(t.scalar_type() == at::kFloat || t.scalar_type() == at::kBFloat16, name,
              " must be float32 or bfloat16");
  TORCH_CHECK(t.size(1) == 0 || t.stride(1) == 1, name, " rows must be contiguous");
}

int32_t table_dtype(const at::Tensor& t) {
  return t.scalar_type() == at::kBFloat16 ? FA_BF16 : FA_F32;
}

// Rows with a leading dimension that is a multiple of 4 may be read up to the next multiple
// of 4 past their width (the padding values are ignored): the allocation must cover that.
void check_row_padding(const at::Tensor& t, const char* name) {
  const int64_t n = t.size(0), d = t.size(1), ld = d > 0 ? t.stride(0) : 0;
  if (n == 0 || d == 0 || (ld & 3) || !(d & 3)) return;
  const int64_t need = (t.storage_offset() + (n - 1) * ld + ((d + 3) / 4) * 4) * t.element_size();
  TORCH_CHECK(static_cast<int64_t>(t.storage().nbytes()) >= need, name,
              ": rows with a leading dimension divisible by 4 must be padded to a multiple of 4");
}

const int64_t* opt_index(const std::optional<at::Tensor>& idx, int64_t n, const at::Tensor& ref,
                         const char* name) {
  if (!idx.has_value()) return nullptr;
  const at::Tensor& t = *idx;
  CHECK_INPUT(t);
  CHECK_DTYPE(t, at::kLong);
  TORCH_CHECK(t.numel() == n, name, " must have one entry per edge");
  CHECK_SAME_DEVICE(t, ref);
  return t.data_ptr<int64_t>();
}

fa_tgat_graph make_graph(const at::Tensor& rowptr, const at::Tensor& node_tab,
                         const std::optional<at::Tensor>& node_idx, const at::Tensor& edge_tab,
                         const std::optional<at::Tensor>& edge_idx, const at::Tensor& dt,
                         const at::Tensor& time_w, const at::Tensor& time_b) {
  CHECK_INPUT(rowptr);
  CHECK_DTYPE(rowptr, at::kInt);
  CHECK_INPUT(dt);
  CHECK_DTYPE(dt, at::kFloat);
  CHECK_INPUT(time_w);
  CHECK_INPUT(time_b);
  CHECK_DTYPE(time_w, at::kFloat);
  CHECK_DTYPE(time_b, at::kFloat);
  check_table(node_tab, "node_tab");
  check_table(edge_tab, "edge_tab");
  check_row_padding(node_tab, "node_tab");
  check_row_padding(edge_tab, "edge_tab");
  TORCH_CHECK(time_w.numel() == time_b.numel(), "time_w and time_b must have the same length");
  const int64_t E = dt.numel();
  for (const at::Tensor* t : {&node_tab, &edge_tab, &dt, &time_w, &time_b})
    CHECK_SAME_DEVICE((*t), rowptr);
  fa_tgat_graph g{};
  g.n_dst = rowptr.numel() - 1;
  g.n_edges = E;
  g.rowptr = rowptr.data_ptr<int32_t>();
  g.node_tab = node_tab.data_ptr();
  g.node_dtype = table_dtype(node_tab);
  g.ld_node = node_tab.size(1) > 0 ? node_tab.stride(0) : 0;
  g.n_node = node_tab.size(0);
  g.dn = static_cast<int32_t>(node_tab.size(1));
  g.node_idx = opt_index(node_idx, E, rowptr, "node_idx");
  g.edge_tab = edge_tab.data_ptr();
  g.edge_dtype = table_dtype(edge_tab);
  g.ld_edge = edge_tab.size(1) > 0 ? edge_tab.stride(0) : 0;
  g.n_edge_rows = edge_tab.size(0);
  g.de = static_cast<int32_t>(edge_tab.size(1));
  g.edge_idx = opt_index(edge_idx, E, rowptr, "edge_idx");
  g.dt = dt.data_ptr<float>();
  g.time_w = time_w.data_ptr<float>();
  g.time_b = time_b.data_ptr<float>();
  g.dt_dim = static_cast<int32_t>(time_w.numel());
  TORCH_CHECK(g.n_dst >= 0, "rowptr must hold n_dst+1 offsets");
  return g;
}

// A [groups, n, c] block whose rows start on 128-byte boundaries (row stride rounded up to
// 32 floats): rows then never share a cache line, so rows written by different waves do
// not leave partly written lines behind. Returned as the [groups, n, c] view.
at::Tensor new_block(int64_t groups, int64_t n, int64_t c, const at::TensorOptions& opt) {
  const int64_t ld = (c + 31) / 32 * 32;
  return at::empty({groups, n, ld}, opt).narrow(2, 0, c);
}

// A per-destination block given as a [heads, n_dst, Kp] tensor of any strides with unit
// stride along Kp (head-major when contiguous; a permuted [n_dst, heads, Kp] works too).
void check_kspace(const at::Tensor& t, const fa_tgat_graph& g, int64_t heads, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  CHECK_DTYPE(t, at::kFloat);
  const int64_t kp = fa_tgat_kspace(g.dn, g.de, g.dt_dim);
  TORCH_CHECK(t.dim() == 3 && t.size(0) == heads && t.size(1) == g.n_dst && t.size(2) == kp, name,
              " must be [heads, n_dst, ", kp, "]");
  TORCH_CHECK(t.stride(2) == 1 || kp <= 1, name, " must have unit stride along Kp");
}

// qt [H, N, Kp] -> [xbar [H, N, Kp], scores [E, H], stats [N, H, 2]]
std::vector<at::Tensor> tgat_attn_fwd(at::Tensor rowptr, at::Tensor node_tab,
                                      std::optional<at::Tensor> node_idx, at::Tensor edge_tab,
                                      std::optional<at::Tensor> edge_idx, at::Tensor dt,
                                      at::Tensor time_w, at::Tensor time_b, at::Tensor qt,
                                      double slope, std::optional<at::Tensor> drop,
                                      uint64_t drop_seed, double drop_p) {
  fa_tgat_graph g = make_graph(rowptr, node_tab, node_idx, edge_tab, edge_idx, dt, time_w, time_b);
  TORCH_CHECK(qt.dim() == 3, "qt must be [heads, n_dst, Kp]");
  const int64_t H = qt.size(0);
  check_kspace(qt, g, H, "qt");
  const float* dptr = nullptr;
  if (drop.has_value()) {
    CHECK_INPUT((*drop));
    CHECK_DTYPE((*drop), at::kFloat);
    TORCH_CHECK(drop->dim() == 2 && drop->size(0) == g.n_edges && drop->size(1) == H,
                "drop must be [E, heads]");
    dptr = drop->data_ptr<float>();
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard(qt.device());
  auto xbar = new_block(H, g.n_dst, qt.size(2), qt.options());
  auto scores = at::empty({g.n_edges, H}, qt.options());
  auto stats = at::empty({g.n_dst, H, 2}, qt.options());
  const int st = fa_tgat_attn_fwd_f32(&g, static_cast<int32_t>(H), qt.data_ptr<float>(),
                                      qt.stride(1), qt.stride(0), static_cast<float>(slope), dptr,
                                      drop_seed, static_cast<float>(drop_p),
                                      xbar.data_ptr<float>(), xbar.stride(1), xbar.stride(0),
                                      scores.data_ptr<float>(), stats.data_ptr<float>(),
                                      stream_of(qt));
  check_status(st, "tgat_attn_fwd");
  return {xbar, scores, stats};
}

// -> [dqt, d_node (or empty), d_time_w, d_time_b]
std::vector<at::Tensor> tgat_attn_bwd(at::Tensor rowptr, at::Tensor node_tab,
                                      std::optional<at::Tensor> node_idx, at::Tensor edge_tab,
                                      std::optional<at::Tensor> edge_idx, at::Tensor dt,
                                      at::Tensor time_w, at::Tensor time_b, at::Tensor qt,
                                      double slope, std::optional<at::Tensor> drop,
                                      uint64_t drop_seed, double drop_p,
                                      std::optional<at::Tensor> xbar, at::Tensor scores,
                                      at::Tensor stats, at::Tensor dxbar, bool need_d_node,
                                      std::optional<at::Tensor> tdot, int64_t d_node_front) {
  fa_tgat_graph g = make_graph(rowptr, node_tab, node_idx, edge_tab, edge_idx, dt, time_w, time_b);
  TORCH_CHECK(qt.dim() == 3, "qt must be [heads, n_dst, Kp]");
  const int64_t H = qt.size(0);
  check_kspace(qt, g, H, "qt");
  TORCH_CHECK(xbar.has_value() || tdot.has_value(), "tgat_attn_bwd needs xbar or tdot");
  const float* xptr = nullptr;
  int64_t x_rs = 0, x_hs = 0;
  if (xbar.has_value()) {
    check_kspace(*xbar, g, H, "xbar");
    xptr = xbar->data_ptr<float>();
    x_rs = xbar->stride(1);
    x_hs = xbar->stride(0);
  }
  const float* tptr = nullptr;
  if (tdot.has_value()) {
    CHECK_INPUT((*tdot));
    CHECK_DTYPE((*tdot), at::kFloat);
    TORCH_CHECK(tdot->numel() == g.n_dst * H, "tdot must be [n_dst, heads]");
    tptr = tdot->data_ptr<float>();
  }
  check_kspace(dxbar, g, H, "dxbar");
  CHECK_INPUT(scores);
  CHECK_INPUT(stats);
  TORCH_CHECK(scores.numel() == g.n_edges * H && stats.numel() == g.n_dst * H * 2,
              "scores / stats do not match the graph");
  const float* dptr = nullptr;
  if (drop.has_value()) {
    CHECK_INPUT((*drop));
    CHECK_DTYPE((*drop), at::kFloat);
    TORCH_CHECK(drop->numel() == g.n_edges * H, "drop must be [E, heads]");
    dptr = drop->data_ptr<float>();
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard(qt.device());
  auto dqt = new_block(H, g.n_dst, qt.size(2), qt.options());
  // d_node: rows [d_node_front, d_node_front + E) of one allocation, the rows in front left
  // for the caller (the gradient of the destination rows of the same source tensor)
  TORCH_CHECK(d_node_front >= 0, "d_node_front must be >= 0");
  at::Tensor d_node;
  if (need_d_node)
    d_node = at::empty({d_node_front + g.n_edges, g.dn}, qt.options()).narrow(0, d_node_front, g.n_edges);
  auto d_tw = at::empty({g.dt_dim}, qt.options());
  auto d_tb = at::empty({g.dt_dim}, qt.options());
  const size_t sb = fa_tgat_attn_bwd_scratch_bytes(g.n_dst, g.dt_dim);
  auto scratch = at::empty({static_cast<int64_t>(sb)}, qt.options().dtype(at::kByte));
  const int st = fa_tgat_attn_bwd_f32(
      &g, static_cast<int32_t>(H), qt.data_ptr<float>(), qt.stride(1), qt.stride(0),
      static_cast<float>(slope), dptr, drop_seed, static_cast<float>(drop_p),
      xptr, x_rs, x_hs, tptr, scores.data_ptr<float>(),
      stats.data_ptr<float>(), dxbar.data_ptr<float>(), dxbar.stride(1), dxbar.stride(0),
      dqt.data_ptr<float>(), dqt.stride(1), dqt.stride(0),
      need_d_node && g.n_edges > 0 && g.dn > 0 ? d_node.data_ptr<float>() : nullptr,
      need_d_node ? g.dn : 0, d_tw.data_ptr<float>(), d_tb.data_ptr<float>(), scratch.data_ptr(),
      sb, stream_of(qt));
  check_status(st, "tgat_attn_bwd");
  return {dqt, need_d_node ? d_node : at::Tensor(), d_tw, d_tb};
}

// [n_edges, heads] multipliers of the hashed attention dropout (keep/(1-p) or 0).
at::Tensor dropout_mask(int64_t n_edges, int64_t heads, uint64_t seed, double p, at::Device device) {
  TORCH_CHECK(n_edges >= 0 && heads > 0, "n_edges must be >= 0 and heads > 0");
  TORCH_CHECK(p >= 0.0 && p < 1.0, "p must lie in [0, 1)");
  TORCH_CHECK(device.is_cuda(), "device must be a GPU");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  auto out = at::empty({n_edges, heads}, at::TensorOptions().dtype(at::kFloat).device(device));
  const int st = fa_dropout_mask_f32(seed, static_cast<float>(p), n_edges * heads,
                                     out.data_ptr<float>(), stream_of(out));
  check_status(st, "dropout_mask");
  return out;
}

at::Tensor tgat_attn_weights(at::Tensor dst, at::Tensor scores, at::Tensor stats) {
  CHECK_INPUT(dst);
  CHECK_INPUT(scores);
  CHECK_INPUT(stats);
  CHECK_DTYPE(dst, at::kLong);
  CHECK_DTYPE(scores, at::kFloat);
  CHECK_DTYPE(stats, at::kFloat);
  CHECK_DIM(scores, 2);
  TORCH_CHECK(dst.numel() == scores.size(0), "dst must have one entry per edge");
  TORCH_CHECK(stats.dim() == 3 && stats.size(1) == scores.size(1) && stats.size(2) == 2,
              "stats must be [n_dst, heads, 2]");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
  auto att = at::empty_like(scores);
  const int st = fa_tgat_attn_weights_f32(dst.data_ptr<int64_t>(), scores.size(0), stats.size(0),
                                          static_cast<int32_t>(scores.size(1)),
                                          scores.data_ptr<float>(), stats.data_ptr<float>(),
                                          att.data_ptr<float>(), stream_of(scores));
  check_status(st, "tgat_attn_weights");
  return att;
}

// -> [n, max(dim, width)] float32; columns past dim (when width > dim) are zero
at::Tensor gather_rows(at::Tensor tab, std::optional<at::Tensor> idx, int64_t n, int64_t width) {
  check_table(tab, "tab");
  const int64_t* ip = nullptr;
  if (idx.has_value()) {
    CHECK_INPUT((*idx));
    CHECK_DTYPE((*idx), at::kLong);
    n = idx->numel();
    ip = idx->data_ptr<int64_t>();
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard(tab.device());
  const int64_t ow = width > tab.size(1) ? width : tab.size(1);
  auto out = at::empty({n, ow}, tab.options().dtype(at::kFloat));
  if (ow > tab.size(1) && n > 0) out.narrow(1, tab.size(1), ow - tab.size(1)).zero_();
  const int64_t ld = tab.size(1) > 0 ? tab.stride(0) : 0;
  const int32_t dim = static_cast<int32_t>(tab.size(1));
  const int st = tab.scalar_type() == at::kBFloat16
                     ? fa_gather_rows_bf16_f32(reinterpret_cast<const uint16_t*>(tab.data_ptr()), ld,
                                               tab.size(0), ip, n, dim, out.data_ptr<float>(), ow,
                                               stream_of(tab))
                     : fa_gather_rows_f32(tab.data_ptr<float>(), ld, tab.size(0), ip, n, dim,
                                          out.data_ptr<float>(), ow, stream_of(tab));
  check_status(st, "gather_rows");
  return out;
}

static const float* opt_ptr(const std::optional<at::Tensor>& t, int64_t numel, const char* name) {
  if (!t.has_value() || !t->defined()) return nullptr;
  CHECK_INPUT((*t));
  CHECK_DTYPE((*t), at::kFloat);
  TORCH_CHECK(t->numel() == numel, name, ": wrong size");
  return t->data_ptr<float>();
}

static void check_param(const at::Tensor& t, int64_t rows, int64_t cols, const char* name) {
  CHECK_INPUT(t);
  CHECK_DTYPE(t, at::kFloat);
  TORCH_CHECK(t.numel() == rows * cols, name, ": wrong size");
}

// -> [wq_node, wk_aug, wv_aug, qbk, wo1, wo2]
std::vector<at::Tensor> layer_params_fwd(at::Tensor wq, at::Tensor bq, at::Tensor wk,
                                         at::Tensor bk, at::Tensor wv, at::Tensor bv,
                                         std::optional<at::Tensor> bt, at::Tensor wo,
                                         int64_t heads, int64_t dn, int64_t de, int64_t dt) {
  const int64_t d = bq.numel();
  const int64_t kp = fa_tgat_kspace(static_cast<int32_t>(dn), static_cast<int32_t>(de),
                                    static_cast<int32_t>(dt));
  check_param(wq, d, dn + dt, "wq");
  check_param(bq, d, 1, "bq");
  check_param(wk, d, dn + de + dt, "wk");
  check_param(bk, d, 1, "bk");
  check_param(wv, d, dn + de + dt, "wv");
  check_param(bv, d, 1, "bv");
  check_param(wo, d, d + dn, "wo");
  const float* btp = opt_ptr(bt, dt, "bt");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(wq.device());
  auto o = wq.options();
  auto wq_node = at::empty({d, dn}, o), wk_aug = at::empty({d, kp}, o), wv_aug = at::empty({d, kp}, o);
  auto qbk = at::empty({heads, kp}, o), wo1 = at::empty({d, d}, o), wo2 = at::empty({d, dn}, o);
  const int st = fa_layer_params_fwd_f32(
      static_cast<int32_t>(d), static_cast<int32_t>(heads), static_cast<int32_t>(dn),
      static_cast<int32_t>(de), static_cast<int32_t>(dt), wq.data_ptr<float>(), dn + dt,
      bq.data_ptr<float>(), wk.data_ptr<float>(), dn + de + dt, bk.data_ptr<float>(),
      wv.data_ptr<float>(), dn + de + dt, bv.data_ptr<float>(), btp, wo.data_ptr<float>(), d + dn,
      wq_node.data_ptr<float>(), wk_aug.data_ptr<float>(), wv_aug.data_ptr<float>(),
      qbk.data_ptr<float>(), wo1.data_ptr<float>(), wo2.data_ptr<float>(),
      at::empty({2 * d}, o).data_ptr<float>(), stream_of(wq));
  check_status(st, "layer_params_fwd");
  return {wq_node, wk_aug, wv_aug, qbk, wo1, wo2};
}

// -> [d_wq, d_bq, d_wk, d_bk, d_wv, d_bv, d_bt, d_wo]
std::vector<at::Tensor> layer_params_bwd(at::Tensor wq, at::Tensor bq, at::Tensor wk,
                                         at::Tensor bk, std::optional<at::Tensor> bt,
                                         std::optional<at::Tensor> g_wq_node,
                                         std::optional<at::Tensor> g_wk_aug,
                                         std::optional<at::Tensor> g_wv_aug,
                                         std::optional<at::Tensor> g_qbk,
                                         std::optional<at::Tensor> g_wo1,
                                         std::optional<at::Tensor> g_wo2, int64_t heads,
                                         int64_t dn, int64_t de, int64_t dt) {
  const int64_t d = bq.numel();
  const int64_t kp = fa_tgat_kspace(static_cast<int32_t>(dn), static_cast<int32_t>(de),
                                    static_cast<int32_t>(dt));
  check_param(wq, d, dn + dt, "wq");
  check_param(bq, d, 1, "bq");
  check_param(wk, d, dn + de + dt, "wk");
  check_param(bk, d, 1, "bk");
  const float* btp = opt_ptr(bt, dt, "bt");
  const float* p_wq = opt_ptr(g_wq_node, d * dn, "g_wq_node");
  const float* p_wk = opt_ptr(g_wk_aug, d * kp, "g_wk_aug");
  const float* p_wv = opt_ptr(g_wv_aug, d * kp, "g_wv_aug");
  const float* p_qb = opt_ptr(g_qbk, heads * kp, "g_qbk");
  const float* p_o1 = opt_ptr(g_wo1, d * d, "g_wo1");
  const float* p_o2 = opt_ptr(g_wo2, d * dn, "g_wo2");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(wq.device());
  auto o = wq.options();
  auto d_wq = at::empty({d, dn + dt}, o), d_bq = at::empty({d}, o);
  auto d_wk = at::empty({d, dn + de + dt}, o), d_bk = at::empty({d}, o);
  auto d_wv = at::empty({d, dn + de + dt}, o), d_bv = at::empty({d}, o);
  auto d_bt = at::empty({dt}, o), d_wo = at::empty({d, d + dn}, o);
  const int st = fa_layer_params_bwd_f32(
      static_cast<int32_t>(d), static_cast<int32_t>(heads), static_cast<int32_t>(dn),
      static_cast<int32_t>(de), static_cast<int32_t>(dt), wq.data_ptr<float>(), dn + dt,
      bq.data_ptr<float>(), wk.data_ptr<float>(), dn + de + dt, bk.data_ptr<float>(), btp, p_wq,
      p_wk, p_wv, p_qb, p_o1, p_o2, d_wq.data_ptr<float>(), d_bq.data_ptr<float>(),
      d_wk.data_ptr<float>(), d_bk.data_ptr<float>(), d_wv.data_ptr<float>(),
      d_bv.data_ptr<float>(), dt > 0 ? d_bt.data_ptr<float>() : nullptr, d_wo.data_ptr<float>(),
      at::empty({2 * d}, o).data_ptr<float>(), stream_of(wq));
  check_status(st, "layer_params_bwd");
  return {d_wq, d_bq, d_wk, d_bk, d_wv, d_bv, d_bt, d_wo};
}

// [n, groups]: dot products of a's and b's column groups of `width` per row.
at::Tensor row_group_dots(at::Tensor a, at::Tensor b, int64_t groups) {
  CHECK_INPUT(a);
  CHECK_INPUT(b);
  CHECK_DTYPE(a, at::kFloat);
  CHECK_DTYPE(b, at::kFloat);
  TORCH_CHECK(a.dim() == 2 && a.sizes() == b.sizes(), "a and b must be the same [n, cols]");
  TORCH_CHECK(groups > 0 && a.size(1) % groups == 0, "cols must split into groups");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  auto out = at::empty({a.size(0), groups}, a.options());
  const int st = fa_row_group_dots_f32(a.size(0), static_cast<int32_t>(groups),
                                       static_cast<int32_t>(a.size(1) / groups), a.data_ptr<float>(),
                                       a.size(1), b.data_ptr<float>(), b.size(1),
                                       out.data_ptr<float>(), stream_of(a));
  check_status(st, "row_group_dots");
  return out;
}

// -> [out [n, d], y [n, d], stats [n, 2]]
std::vector<at::Tensor> tgat_epilogue_fwd(at::Tensor r1, std::optional<at::Tensor> r2,
                                          std::optional<at::Tensor> bias, at::Tensor gamma,
                                          at::Tensor beta, double eps, uint64_t drop_seed,
                                          double drop_p) {
  CHECK_CUDA(r1);
  CHECK_DTYPE(r1, at::kFloat);
  TORCH_CHECK(r1.dim() == 2 && r1.stride(1) == 1, "r1 must be a row-major [n, d] matrix");
  const int64_t n = r1.size(0), d = r1.size(1);
  const float* r2p = nullptr;
  int64_t ld2 = d;
  if (r2.has_value()) {
    CHECK_CUDA((*r2));
    CHECK_DTYPE((*r2), at::kFloat);
    TORCH_CHECK(r2->dim() == 2 && r2->size(0) == n && r2->size(1) == d && r2->stride(1) == 1,
                "r2 must match r1");
    r2p = r2->data_ptr<float>();
    ld2 = r2->stride(0);
  }
  CHECK_INPUT(gamma);
  CHECK_INPUT(beta);
  TORCH_CHECK(gamma.numel() == d && beta.numel() == d, "gamma / beta must have d entries");
  const float* bp = nullptr;
  if (bias.has_value()) {
    CHECK_INPUT((*bias));
    CHECK_DTYPE((*bias), at::kFloat);
    TORCH_CHECK(bias->numel() == d, "bias must have d entries");
    bp = bias->data_ptr<float>();
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard(r1.device());
  auto out = at::empty({n, d}, r1.options());
  auto y = at::empty({n, d}, r1.options());
  auto stats = at::empty({n, 2}, r1.options());
  const int st = fa_tgat_epilogue_fwd_f32(n, static_cast<int32_t>(d), r1.data_ptr<float>(),
                                          r1.stride(0), r2p, ld2, bp, gamma.data_ptr<float>(),
                                          beta.data_ptr<float>(), static_cast<float>(eps),
                                          drop_seed, static_cast<float>(drop_p),
                                          out.data_ptr<float>(), y.data_ptr<float>(),
                                          stats.data_ptr<float>(), stream_of(r1));
  check_status(st, "tgat_epilogue_fwd");
  return {out, y, stats};
}

// -> [du [n, d], dgamma [d], dbeta [d], dbias [d] (empty unless need_dbias)]
std::vector<at::Tensor> tgat_epilogue_bwd(at::Tensor dout, at::Tensor y, at::Tensor stats,
                                          at::Tensor gamma, double drop_p, bool need_dbias) {
  CHECK_INPUT(dout);
  CHECK_INPUT(y);
  CHECK_INPUT(stats);
  CHECK_INPUT(gamma);
  TORCH_CHECK(dout.sizes() == y.sizes() && dout.dim() == 2, "dout must match y [n, d]");
  const int64_t n = y.size(0), d = y.size(1);
  TORCH_CHECK(stats.numel() == 2 * n && gamma.numel() == d, "stats / gamma do not match y");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(y.device());
  auto du = at::empty({n, d}, y.options());
  auto dgamma = at::empty({d}, y.options());
  auto dbeta = at::empty({d}, y.options());
  at::Tensor dbias;
  if (need_dbias) dbias = at::empty({d}, y.options());
  const size_t sb = fa_tgat_epilogue_bwd_scratch_bytes(n, static_cast<int32_t>(d));
  auto scratch = at::empty({static_cast<int64_t>(sb > 0 ? sb : 1)}, y.options().dtype(at::kByte));
  const int st = fa_tgat_epilogue_bwd_f32(n, static_cast<int32_t>(d), dout.data_ptr<float>(),
                                          y.data_ptr<float>(), stats.data_ptr<float>(),
                                          gamma.data_ptr<float>(), static_cast<float>(drop_p),
                                          du.data_ptr<float>(), dgamma.data_ptr<float>(),
                                          dbeta.data_ptr<float>(),
                                          need_dbias ? dbias.data_ptr<float>() : nullptr,
                                          scratch.data_ptr(), sb, stream_of(y));
  check_status(st, "tgat_epilogue_bwd");
  return {du, dgamma, dbeta, dbias};
}

// ----- per-head projections --------------------------------------------------------

// x: [n, groups*j] with unit column stride; w: [groups, j, c] contiguous; y: [groups, n, c]
// with unit stride along c.
void check_rowmat(const at::Tensor& t, const char* name) {
  CHECK_CUDA(t);
  CHECK_DTYPE(t, at::kFloat);
  TORCH_CHECK(t.dim() == 2 && (t.stride(1) == 1 || t.size(1) <= 1), name,
              " must be a [n, d] matrix with unit column stride");
}

void check_block(const at::Tensor& t, const char* name) {
  CHECK_CUDA(t);
  CHECK_DTYPE(t, at::kFloat);
  TORCH_CHECK(t.dim() == 3 && (t.stride(2) == 1 || t.size(2) <= 1), name,
              " must be a [groups, n, c] block with unit stride along c");
}

// y[g] = x[:, g*J:(g+1)*J] @ w[g] (+ bias[g])  -> [groups, n, c]
at::Tensor head_proj(at::Tensor x, at::Tensor w, std::optional<at::Tensor> bias) {
  check_rowmat(x, "x");
  CHECK_INPUT(w);
  CHECK_DTYPE(w, at::kFloat);
  TORCH_CHECK(w.dim() == 3, "w must be [groups, j, c]");
  const int64_t G = w.size(0), J = w.size(1), C = w.size(2), n = x.size(0);
  TORCH_CHECK(x.size(1) == G * J, "x must have groups*j columns");
  const float* bp = nullptr;
  if (bias.has_value()) {
    CHECK_INPUT((*bias));
    CHECK_DTYPE((*bias), at::kFloat);
    TORCH_CHECK(bias->numel() == G * C, "bias must be [groups, c]");
    bp = bias->data_ptr<float>();
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  auto y = new_block(G, n, C, x.options());
  if (n == 0 || G == 0 || C == 0) return y;
  TORCH_CHECK(J > 0, "head_proj: j must be positive");
  const int st = fa_head_proj_f32(n, static_cast<int32_t>(J), static_cast<int32_t>(C),
                                  static_cast<int32_t>(G), x.data_ptr<float>(), x.stride(0), J,
                                  w.data_ptr<float>(), J * C, C, bp, C, y.data_ptr<float>(),
                                  y.stride(0), y.stride(1), stream_of(x));
  check_status(st, "head_proj");
  return y;
}

// z[:, g*J:(g+1)*J] = y[g] @ w[g]^T  -> [n, groups*j]
at::Tensor head_reduce(at::Tensor y, at::Tensor w) {
  check_block(y, "y");
  CHECK_INPUT(w);
  CHECK_DTYPE(w, at::kFloat);
  TORCH_CHECK(w.dim() == 3 && w.size(0) == y.size(0) && w.size(2) == y.size(2),
              "w must be [groups, j, c] matching y");
  const int64_t G = w.size(0), J = w.size(1), C = w.size(2), n = y.size(1);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(y.device());
  auto z = at::empty({n, G * J}, y.options());
  if (n == 0 || G == 0 || J == 0) return z;
  if (C == 0) return z.zero_();
  const int st = fa_head_reduce_f32(n, static_cast<int32_t>(J), static_cast<int32_t>(C),
                                    static_cast<int32_t>(G), y.data_ptr<float>(), y.stride(0),
                                    y.stride(1), w.data_ptr<float>(), J * C, C,
                                    z.data_ptr<float>(), G * J, J, stream_of(y));
  check_status(st, "head_reduce");
  return z;
}

// dw[g] = x[:, g*J:(g+1)*J]^T @ y[g] (row J: column sums of y[g] when ones) -> [groups, j+ones, c]
at::Tensor head_wgrad(at::Tensor x, at::Tensor y, int64_t groups, bool ones) {
  check_rowmat(x, "x");
  check_block(y, "y");
  const int64_t G = groups, n = x.size(0), C = y.size(2);
  TORCH_CHECK(G > 0 && y.size(0) == G && y.size(1) == n && x.size(1) % G == 0,
              "head_wgrad: x [n, groups*j] and y [groups, n, c] do not match");
  const int64_t J = x.size(1) / G;
  TORCH_CHECK(J > 0 && C > 0, "head_wgrad: empty j or c");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(y.device());
  auto dw = at::empty({G, J + (ones ? 1 : 0), C}, y.options());
  const size_t sb = fa_head_wgrad_scratch_bytes(n, static_cast<int32_t>(J),
                                                static_cast<int32_t>(C),
                                                static_cast<int32_t>(G), ones ? 1 : 0);
  auto scratch = at::empty({static_cast<int64_t>(sb > 0 ? sb : 1)}, y.options().dtype(at::kByte));
  const int st = fa_head_wgrad_f32(n, static_cast<int32_t>(J), static_cast<int32_t>(C),
                                   static_cast<int32_t>(G), n > 0 ? x.data_ptr<float>() : nullptr,
                                   x.stride(0), J, n > 0 ? y.data_ptr<float>() : nullptr,
                                   y.stride(0), y.stride(1), ones ? 1 : 0, dw.data_ptr<float>(),
                                   scratch.data_ptr(), sb, stream_of(y));
  check_status(st, "head_wgrad");
  return dw;
}


// ----------------------------------------------------------------------------------
// TGN node memory (memorys.py): mail gather, time rows, recurrent cell gates, write-back
// ----------------------------------------------------------------------------------
void check_ids(const at::Tensor& ids, const char* name) {
  CHECK_INPUT(ids);
  TORCH_CHECK(ids.scalar_type() == at::kInt || ids.scalar_type() == at::kLong, name,
              " must be int32 or int64, got ", ids.scalar_type());
  CHECK_DIM(ids, 1);
}

void check_f32(const at::Tensor& t, int64_t dims, const char* name) {
  CHECK_INPUT(t);
  CHECK_DTYPE(t, at::kFloat);
  TORCH_CHECK(t.dim() == dims, name, " must be ", dims, "-D, got ", t.dim(), "-D");
}

// -> [mem [n, m], mem_ts [n], x [n, x_width] (mails in columns [0, slots*mail)), mail_ts [n, slots]]
std::vector<at::Tensor> mail_gather(at::Tensor ids, at::Tensor node_memory, at::Tensor node_memory_ts,
                                    at::Tensor mailbox, at::Tensor mailbox_ts, int64_t x_width) {
  check_ids(ids, "ids");
  check_f32(node_memory, 2, "node_memory");
  check_f32(node_memory_ts, 1, "node_memory_ts");
  check_f32(mailbox, 3, "mailbox");
  check_f32(mailbox_ts, 2, "mailbox_ts");
  const int64_t nodes = node_memory.size(0), m = node_memory.size(1);
  const int64_t slots = mailbox.size(1), mail_w = slots * mailbox.size(2);
  TORCH_CHECK(node_memory_ts.numel() == nodes && mailbox.size(0) == nodes &&
                  mailbox_ts.size(0) == nodes && mailbox_ts.size(1) == slots,
              "mail_gather: the memory and mailbox tensors must have one row per node");
  TORCH_CHECK(x_width >= mail_w, "mail_gather: x_width must hold the mails (", mail_w, ")");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(ids.device());
  const int64_t n = ids.numel();
  auto opt = node_memory.options();
  auto mem = at::empty({n, m}, opt);
  auto mem_ts = at::empty({n}, opt);
  auto x = at::empty({n, x_width}, opt);
  auto mail_ts = at::empty({n, slots}, opt);
  const int st = fa_mail_gather_f32(
      n, ids.data_ptr(), ids.scalar_type() == at::kLong ? 1 : 0, nodes, node_memory.data_ptr<float>(),
      m, static_cast<int32_t>(m), node_memory_ts.data_ptr<float>(), mailbox.data_ptr<float>(), mail_w,
      mail_w, mailbox_ts.data_ptr<float>(), static_cast<int32_t>(slots), mem.data_ptr<float>(), m,
      mem_ts.data_ptr<float>(), x.data_ptr<float>(), x_width, mail_ts.data_ptr<float>(),
      stream_of(ids));
  check_status(st, "mail_gather");
  return {mem, mem_ts, x, mail_ts};
}

// out[:, col:col+dt] = cos(w (ts - mem_ts) + b), in place.
void time_rows_(at::Tensor out, int64_t col, at::Tensor ts, std::optional<at::Tensor> mem_ts,
                at::Tensor w, at::Tensor b) {
  check_f32(out, 2, "out");
  check_f32(ts, 1, "ts");
  CHECK_INPUT(w);
  CHECK_INPUT(b);
  CHECK_DTYPE(w, at::kFloat);
  CHECK_DTYPE(b, at::kFloat);
  const int64_t n = out.size(0), dt = w.numel();
  TORCH_CHECK(b.numel() == dt && ts.numel() == n, "time_rows_: w, b of dt and ts of n rows");
  TORCH_CHECK(col >= 0 && col + dt <= out.size(1), "time_rows_: columns out of range");
  const float* mt = opt_ptr(mem_ts, n, "mem_ts");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
  const int st = fa_time_rows_f32(n, ts.data_ptr<float>(), mt, w.data_ptr<float>(), b.data_ptr<float>(),
                                  static_cast<int32_t>(dt), out.data_ptr<float>() + col, out.size(1),
                                  stream_of(out));
  check_status(st, "time_rows_");
}

// -> [dw [dt], db [dt]] for g [n, dt] (rows of any stride, unit column stride)
std::vector<at::Tensor> time_rows_grad(at::Tensor g, at::Tensor ts, std::optional<at::Tensor> mem_ts,
                                       at::Tensor w, at::Tensor b) {
  CHECK_CUDA(g);
  CHECK_DTYPE(g, at::kFloat);
  CHECK_DIM(g, 2);
  TORCH_CHECK(g.stride(1) == 1 || g.size(1) <= 1, "time_rows_grad: g must have unit column stride");
  check_f32(ts, 1, "ts");
  CHECK_INPUT(w);
  CHECK_INPUT(b);
  CHECK_DTYPE(w, at::kFloat);
  CHECK_DTYPE(b, at::kFloat);
  const int64_t n = g.size(0), dt = w.numel();
  TORCH_CHECK(g.size(1) == dt && b.numel() == dt && ts.numel() == n, "time_rows_grad: shapes");
  const float* mt = opt_ptr(mem_ts, n, "mem_ts");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(g.device());
  auto dw = at::empty({dt}, w.options());
  auto db = at::empty({dt}, w.options());
  const size_t sb = fa_time_rows_grad_scratch_bytes(static_cast<int32_t>(dt));
  auto scratch = at::empty({static_cast<int64_t>(sb / 4 + 1)}, w.options());
  const int64_t ld = n > 0 ? g.stride(0) : dt;
  const int st = fa_time_rows_grad_f32(n, ts.data_ptr<float>(), mt, w.data_ptr<float>(),
                                       b.data_ptr<float>(), static_cast<int32_t>(dt),
                                       g.data_ptr<float>(), ld < dt ? dt : ld, dw.data_ptr<float>(),
                                       db.data_ptr<float>(), scratch.data_ptr<float>(), sb,
                                       stream_of(g));
  check_status(st, "time_rows_grad");
  return {dw, db};
}

// -> [hy [n, m], workspace [n, 4m]]
std::vector<at::Tensor> gru_fwd(at::Tensor gi, at::Tensor gh, std::optional<at::Tensor> h,
                                std::optional<at::Tensor> b_ih, std::optional<at::Tensor> b_hh) {
  check_f32(gi, 2, "gi");
  check_f32(gh, 2, "gh");
  const int64_t n = gi.size(0), m = gi.size(1) / 3;
  TORCH_CHECK(gi.size(1) == 3 * m && gh.sizes() == gi.sizes(), "gru_fwd: gi, gh must be [n, 3m]");
  const float* hp = opt_ptr(h, n * m, "h");
  const float* bi = opt_ptr(b_ih, 3 * m, "b_ih");
  const float* bh = opt_ptr(b_hh, 3 * m, "b_hh");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(gi.device());
  auto hy = at::empty({n, m}, gi.options());
  auto ws = at::empty({n, 4 * m}, gi.options());
  const int st = fa_gru_fwd_f32(n, static_cast<int32_t>(m), gi.data_ptr<float>(), 3 * m,
                                gh.data_ptr<float>(), 3 * m, hp, m, bi, bh, hy.data_ptr<float>(),
                                m, ws.data_ptr<float>(), stream_of(gi));
  check_status(st, "gru_fwd");
  return {hy, ws};
}

// -> [dgi [n, 3m], dgh [n, 3m], dh [n, m] (dhy z; empty unless need_dh), db_ih [3m], db_hh [3m]]
std::vector<at::Tensor> gru_bwd(at::Tensor dhy, at::Tensor ws, std::optional<at::Tensor> h,
                                bool need_dh) {
  check_f32(dhy, 2, "dhy");
  check_f32(ws, 2, "workspace");
  const int64_t n = dhy.size(0), m = dhy.size(1);
  TORCH_CHECK(ws.size(0) == n && ws.size(1) == 4 * m, "gru_bwd: workspace must be [n, 4m]");
  const float* hp = opt_ptr(h, n * m, "h");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(dhy.device());
  auto dgi = at::empty({n, 3 * m}, dhy.options());
  auto dgh = at::empty({n, 3 * m}, dhy.options());
  auto dh = need_dh ? at::empty({n, m}, dhy.options()) : at::empty({0}, dhy.options());
  auto db_ih = at::empty({3 * m}, dhy.options());
  auto db_hh = at::empty({3 * m}, dhy.options());
  const size_t sb = fa_gru_bwd_scratch_bytes(n, static_cast<int32_t>(m));
  auto scratch = at::empty({static_cast<int64_t>(sb / 4 + 1)}, dhy.options());
  const int st = fa_gru_bwd_f32(n, static_cast<int32_t>(m), dhy.data_ptr<float>(), m,
                                ws.data_ptr<float>(), hp, m, dgi.data_ptr<float>(), 3 * m,
                                dgh.data_ptr<float>(), 3 * m, need_dh ? dh.data_ptr<float>() : nullptr,
                                m, db_ih.data_ptr<float>(), db_hh.data_ptr<float>(),
                                scratch.data_ptr<float>(), sb, stream_of(dhy));
  check_status(st, "gru_bwd");
  return {dgi, dgh, dh, db_ih, db_hh};
}

at::Tensor rnn_fwd(at::Tensor gi, at::Tensor gh, std::optional<at::Tensor> b_ih,
                   std::optional<at::Tensor> b_hh) {
  check_f32(gi, 2, "gi");
  check_f32(gh, 2, "gh");
  TORCH_CHECK(gh.sizes() == gi.sizes(), "rnn_fwd: gi, gh must have one shape");
  const int64_t n = gi.size(0), m = gi.size(1);
  const float* bi = opt_ptr(b_ih, m, "b_ih");
  const float* bh = opt_ptr(b_hh, m, "b_hh");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(gi.device());
  auto hy = at::empty({n, m}, gi.options());
  const int st = fa_rnn_fwd_f32(n, static_cast<int32_t>(m), gi.data_ptr<float>(), m,
                                gh.data_ptr<float>(), m, bi, bh, hy.data_ptr<float>(), m,
                                stream_of(gi));
  check_status(st, "rnn_fwd");
  return hy;
}

at::Tensor rnn_bwd(at::Tensor dhy, at::Tensor hy) {
  check_f32(dhy, 2, "dhy");
  check_f32(hy, 2, "hy");
  TORCH_CHECK(dhy.sizes() == hy.sizes(), "rnn_bwd: dhy, hy must have one shape");
  const int64_t n = hy.size(0), m = hy.size(1);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(hy.device());
  auto da = at::empty({n, m}, hy.options());
  const int st = fa_rnn_bwd_f32(n, static_cast<int32_t>(m), dhy.data_ptr<float>(), m,
                                hy.data_ptr<float>(), m, da.data_ptr<float>(), m, stream_of(hy));
  check_status(st, "rnn_bwd");
  return da;
}

void check_last(const at::Tensor& last, int64_t nodes, int64_t generation) {
  CHECK_INPUT(last);
  CHECK_DTYPE(last, at::kLong);
  TORCH_CHECK(last.numel() == nodes, "last must hold one tag per node");
  TORCH_CHECK(generation > 0 && generation <= 0xffffffffLL, "generation must be in [1, 2^32)");
}

// node_memory[ids[r]] = mem[r], node_memory_ts[ids[r]] = ts[r], the last row of an id winning.
void memory_update_(at::Tensor ids, at::Tensor mem, at::Tensor ts, at::Tensor node_memory,
                    at::Tensor node_memory_ts, at::Tensor last, int64_t generation) {
  check_ids(ids, "ids");
  check_f32(mem, 2, "mem");
  check_f32(ts, 1, "ts");
  check_f32(node_memory, 2, "node_memory");
  check_f32(node_memory_ts, 1, "node_memory_ts");
  const int64_t rows = ids.numel(), nodes = node_memory.size(0), m = node_memory.size(1);
  TORCH_CHECK(mem.size(0) == rows && mem.size(1) == m && ts.numel() == rows,
              "memory_update_: mem [rows, m] and ts [rows] for the ids");
  TORCH_CHECK(node_memory_ts.numel() == nodes, "memory_update_: node_memory_ts [num_nodes]");
  check_last(last, nodes, generation);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(ids.device());
  const int st = fa_memory_update_f32(
      rows, ids.data_ptr(), ids.scalar_type() == at::kLong ? 1 : 0, mem.data_ptr<float>(), m,
      static_cast<int32_t>(m), ts.data_ptr<float>(), node_memory.data_ptr<float>(), m,
      node_memory_ts.data_ptr<float>(), nodes,
      reinterpret_cast<unsigned long long*>(last.data_ptr<int64_t>()),
      static_cast<uint32_t>(generation), stream_of(ids));
  check_status(st, "memory_update_");
}

// The mails of n edges (mem rows 0..n-1 sources, n..2n-1 destinations) into the mailbox.
void mailbox_update_(at::Tensor src_ids, at::Tensor dst_ids, at::Tensor mem,
                     std::optional<at::Tensor> edge_feats, at::Tensor ts, at::Tensor mailbox,
                     at::Tensor mailbox_ts, at::Tensor next_pos, at::Tensor last, int64_t generation) {
  check_ids(src_ids, "src_ids");
  check_ids(dst_ids, "dst_ids");
  TORCH_CHECK(src_ids.scalar_type() == dst_ids.scalar_type() && src_ids.numel() == dst_ids.numel(),
              "mailbox_update_: src_ids and dst_ids must match in dtype and length");
  check_f32(mem, 2, "mem");
  check_f32(ts, 1, "ts");
  check_f32(mailbox, 3, "mailbox");
  check_f32(mailbox_ts, 2, "mailbox_ts");
  CHECK_INPUT(next_pos);
  CHECK_DTYPE(next_pos, at::kLong);
  const int64_t n = src_ids.numel(), nodes = mailbox.size(0), slots = mailbox.size(1);
  const int64_t m = mem.size(1);
  int64_t de = 0;
  const float* ef = nullptr;
  if (edge_feats.has_value() && edge_feats->defined()) {
    check_f32(*edge_feats, 2, "edge_feats");
    TORCH_CHECK(edge_feats->size(0) == n, "mailbox_update_: edge_feats [n, de]");
    de = edge_feats->size(1);
    ef = edge_feats->data_ptr<float>();
  }
  TORCH_CHECK(mem.size(0) >= 2 * n, "mailbox_update_: mem needs 2n rows");
  TORCH_CHECK(ts.numel() >= 2 * n, "mailbox_update_: ts needs 2n entries");
  TORCH_CHECK(mailbox.size(2) == 2 * m + de, "mailbox_update_: mailbox rows of 2m + de, got ",
              mailbox.size(2), " for m = ", m, ", de = ", de);
  TORCH_CHECK(mailbox_ts.size(0) == nodes && mailbox_ts.size(1) == slots && next_pos.numel() == nodes,
              "mailbox_update_: mailbox_ts [num_nodes, slots] and next_pos [num_nodes]");
  check_last(last, nodes, generation);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(mem.device());
  const int st = fa_mailbox_update_f32(
      n, src_ids.data_ptr(), dst_ids.data_ptr(), src_ids.scalar_type() == at::kLong ? 1 : 0,
      mem.data_ptr<float>(), m, static_cast<int32_t>(m), ef, de, static_cast<int32_t>(de),
      ts.data_ptr<float>(), mailbox.data_ptr<float>(), slots * mailbox.size(2),
      mailbox_ts.data_ptr<float>(), next_pos.data_ptr<int64_t>(), static_cast<int32_t>(slots), nodes,
      reinterpret_cast<unsigned long long*>(last.data_ptr<int64_t>()),
      static_cast<uint32_t>(generation), stream_of(mem));
  check_status(st, "mailbox_update_");
}

}  // namespace

PYBIND11_MODULE(fastAgg, m) {
  namespace py = pybind11;
  m.doc() = "MI355X-native FAST temporal-attention aggregation operators (gfx950 HIP kernels)";
  // utilities
  m.def("cal_deg", &cal_deg, "cal_deg (HIP)", py::arg("edges"), py::arg("nodes_num"));
  m.def("exclusive_sum", &exclusive_sum, "exclusive_sum (HIP)", py::arg("in_degs"));
  m.def("getBalancedPtr", &getBalancedPtr, "balanced_ptr (HIP)", py::arg("densePtr"),
        py::arg("threshold"));
  // global-based
  m.def("forward_tgat", &forward_tgat, "forward_tgat (HIP)", py::arg("src_edges"),
        py::arg("dst_edges"), py::arg("input_feat"), py::arg("dst_num"), py::arg("aggNodePB"),
        py::arg("aggFeat"));
  m.def("backward_tgat", &backward_tgat, "backward_tgat (HIP)", py::arg("src_edges"),
        py::arg("dst_edges"), py::arg("d_input"), py::arg("src_num"), py::arg("aggNodePB"),
        py::arg("aggFeat"));
  m.def("forward_edge_softmax", &forward_edge_softmax, "esm (HIP)", py::arg("indptr"),
        py::arg("indices"), py::arg("input_feat"), py::arg("node_num_per_block"),
        py::arg("num_heads"));
  m.def("backward_edge_softmax", &backward_edge_softmax, "esm (HIP)", py::arg("indptr"),
        py::arg("indices"), py::arg("d_output"), py::arg("output"), py::arg("node_num_per_block"),
        py::arg("num_heads"));
  // csr-based
  m.def("forward_tgat_shd", &forward_tgat_shd, "forward_tgat_shd (HIP)", py::arg("indptr"),
        py::arg("indices"), py::arg("src_edges"), py::arg("dst_edges"), py::arg("input_feat"),
        py::arg("dst_nodes"), py::arg("aggNodePB"), py::arg("aggFeat"));
  m.def("backward_tgat_shd", &backward_tgat_shd, "backward_tgat_shd (HIP)", py::arg("indptr"),
        py::arg("indices"), py::arg("dst_edges"), py::arg("src_edges"), py::arg("d_input"),
        py::arg("src_nodes"), py::arg("aggNodePB"), py::arg("aggFeat"));
  m.def("forward_balanced_edge_softmax", &forward_balanced_edge_softmax, "esm_csr (HIP)",
        py::arg("indptr"), py::arg("indices"), py::arg("input_feat"),
        py::arg("edge_num_per_block"), py::arg("reduce_size"));
  m.def("backward_balanced_edge_softmax", &backward_balanced_edge_softmax, "esm_csr (HIP)",
        py::arg("indptr"), py::arg("indices"), py::arg("d_output"), py::arg("output"),
        py::arg("node_num_per_block"), py::arg("reduce_size"));
  m.def("forward_csr_edge_softmax", &forward_csr_edge_softmax, "esm_online (HIP)",
        py::arg("indptr"), py::arg("indices"), py::arg("input_feat"),
        py::arg("node_num_per_block"), py::arg("reduce_size"));
  m.def("backward_csr_edge_softmax", &backward_csr_edge_softmax, "esm_online (HIP)",
        py::arg("indptr"), py::arg("indices"), py::arg("d_output"), py::arg("output"),
        py::arg("node_num_per_block"), py::arg("reduce_size"));
  // fused
  m.def("forward_fused_attn", &forward_fused_attn, "fused attn (HIP)", py::arg("input_feat"),
        py::arg("V_val"), py::arg("indptr"), py::arg("indices"), py::arg("dst_eid"),
        py::arg("src_eid"), py::arg("node_num"), py::arg("num_heads"), py::arg("negative_slope"),
        py::arg("attn_drop"));
  m.def("backward_fused_attn", &backward_fused_attn, "fused attn (HIP)", py::arg("d_output"),
        py::arg("V_val"), py::arg("output"), py::arg("edge_mask"), py::arg("indptr"),
        py::arg("indices"), py::arg("dst_eid"), py::arg("src_eid"), py::arg("node_num"),
        py::arg("num_heads"), py::arg("negative_slope"), py::arg("attn_drop"));
  // fused TGAT operators of this build
  m.def("tgat_kspace", &tgat_kspace, "padded K-space width of one key/value input row",
        py::arg("dn"), py::arg("de"), py::arg("dt_dim"));
  m.def("rowptr_from_dst", &rowptr_from_dst, "full-CSR offsets from dst-sorted edge ids",
        py::arg("dst"), py::arg("n_dst"));
  m.def("tgat_attn_fwd", &tgat_attn_fwd,
        "fused gather + time encoding + score + segment softmax + aggregation (forward)",
        py::arg("rowptr"), py::arg("node_tab"), py::arg("node_idx"), py::arg("edge_tab"),
        py::arg("edge_idx"), py::arg("dt"), py::arg("time_w"), py::arg("time_b"), py::arg("qt"),
        py::arg("slope"), py::arg("drop"), py::arg("drop_seed") = 0, py::arg("drop_p") = 0.0);
  m.def("tgat_attn_bwd", &tgat_attn_bwd, "backward of tgat_attn_fwd", py::arg("rowptr"),
        py::arg("node_tab"), py::arg("node_idx"), py::arg("edge_tab"), py::arg("edge_idx"),
        py::arg("dt"), py::arg("time_w"), py::arg("time_b"), py::arg("qt"), py::arg("slope"),
        py::arg("drop"), py::arg("drop_seed"), py::arg("drop_p"), py::arg("xbar"),
        py::arg("scores"), py::arg("stats"), py::arg("dxbar"), py::arg("need_d_node"),
        py::arg("tdot") = py::none(), py::arg("d_node_front") = 0);
  m.def("dropout_mask", &dropout_mask, "multipliers of the hashed attention dropout",
        py::arg("n_edges"), py::arg("heads"), py::arg("seed"), py::arg("p"), py::arg("device"));
  m.def("tgat_attn_weights", &tgat_attn_weights, "normalised attention from scores and stats",
        py::arg("dst"), py::arg("scores"), py::arg("stats"));
  m.def("gather_rows", &gather_rows, "row gather tab[idx] (float32 or bf16 table, float32 rows)", py::arg("tab"), py::arg("idx"),
        py::arg("n"), py::arg("width") = 0);
  m.def("head_proj", &head_proj, "per-head projection y[g] = x[:, g-block] @ w[g] (+ bias[g])",
        py::arg("x"), py::arg("w"), py::arg("bias") = py::none());
  m.def("head_reduce", &head_reduce, "per-head transpose product z[:, g-block] = y[g] @ w[g]^T",
        py::arg("y"), py::arg("w"));
  m.def("head_reduce_supported",
        [](int64_t j, int64_t c, int64_t ldy, bool rows16) {
          return fa_head_reduce_supported(static_cast<int32_t>(j), static_cast<int32_t>(c), ldy,
                                          rows16 ? 1 : 0);
        },
        "path head_reduce takes for (j, c, ldy): 2 split-bf16, 1 float32, 0 unsupported",
        py::arg("j"), py::arg("c"), py::arg("ldy"), py::arg("rows16"));
  m.def("head_wgrad", &head_wgrad, "per-head weight gradient x[:, g-block]^T @ y[g]",
        py::arg("x"), py::arg("y"), py::arg("groups"), py::arg("ones") = false);
  m.def("tgat_epilogue_fwd", &tgat_epilogue_fwd, "LayerNorm(ReLU(dropout(r1 + r2 + bias)))",
        py::arg("r1"), py::arg("r2"), py::arg("bias"), py::arg("gamma"), py::arg("beta"),
        py::arg("eps"), py::arg("drop_seed"), py::arg("drop_p"));
  m.def("layer_params_fwd", &layer_params_fwd, "per-step weight layouts of one layer",
        py::arg("wq"), py::arg("bq"), py::arg("wk"), py::arg("bk"), py::arg("wv"), py::arg("bv"),
        py::arg("bt"), py::arg("wo"), py::arg("heads"), py::arg("dn"), py::arg("de"), py::arg("dt"));
  m.def("layer_params_bwd", &layer_params_bwd, "backward of layer_params_fwd", py::arg("wq"),
        py::arg("bq"), py::arg("wk"), py::arg("bk"), py::arg("bt"), py::arg("g_wq_node"),
        py::arg("g_wk_aug"), py::arg("g_wv_aug"), py::arg("g_qbk"), py::arg("g_wo1"),
        py::arg("g_wo2"), py::arg("heads"), py::arg("dn"), py::arg("de"), py::arg("dt"));
  m.def("row_group_dots", &row_group_dots, "per-row dot products of column groups",
        py::arg("a"), py::arg("b"), py::arg("groups"));
  m.def("tgat_epilogue_bwd", &tgat_epilogue_bwd, "backward of tgat_epilogue_fwd", py::arg("dout"),
        py::arg("y"), py::arg("stats"), py::arg("gamma"), py::arg("drop_p"),
        py::arg("need_dbias") = false);
  // TGN node memory
  m.def("mail_gather", &mail_gather, "per-row memory, mails and times gathered by node id",
        py::arg("ids"), py::arg("node_memory"), py::arg("node_memory_ts"), py::arg("mailbox"),
        py::arg("mailbox_ts"), py::arg("x_width"));
  m.def("time_rows_", &time_rows_, "out[:, col:col+dt] = cos(w (ts - mem_ts) + b)", py::arg("out"),
        py::arg("col"), py::arg("ts"), py::arg("mem_ts"), py::arg("w"), py::arg("b"));
  m.def("time_rows_grad", &time_rows_grad, "dw, db of time_rows_ for the column gradient g",
        py::arg("g"), py::arg("ts"), py::arg("mem_ts"), py::arg("w"), py::arg("b"));
  m.def("gru_fwd", &gru_fwd, "GRUCell gates from gi, gh (and h; the biases when gi, gh lack them)",
        py::arg("gi"), py::arg("gh"), py::arg("h") = py::none(), py::arg("b_ih") = py::none(),
        py::arg("b_hh") = py::none());
  m.def("gru_bwd", &gru_bwd, "GRUCell gate and bias gradients", py::arg("dhy"), py::arg("workspace"),
        py::arg("h") = py::none(), py::arg("need_dh") = false);
  m.def("rnn_fwd", &rnn_fwd, "RNNCell (tanh) from gi, gh (the biases when gi, gh lack them)",
        py::arg("gi"), py::arg("gh"), py::arg("b_ih") = py::none(), py::arg("b_hh") = py::none());
  m.def("rnn_bwd", &rnn_bwd, "RNNCell (tanh) gradient of gi and gh", py::arg("dhy"), py::arg("hy"));
  m.def("memory_update_", &memory_update_, "node memory write-back, last row of an id wins",
        py::arg("ids"), py::arg("mem"), py::arg("ts"), py::arg("node_memory"),
        py::arg("node_memory_ts"), py::arg("last"), py::arg("generation"));
  m.def("mailbox_update_", &mailbox_update_, "mailbox write-back ('self', 'last')",
        py::arg("src_ids"), py::arg("dst_ids"), py::arg("mem"), py::arg("edge_feats"), py::arg("ts"),
        py::arg("mailbox"), py::arg("mailbox_ts"), py::arg("next_pos"), py::arg("last"),
        py::arg("generation"));
  m.attr("abi_version") = fa_abi_version();
}
