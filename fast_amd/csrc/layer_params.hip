// Per-step parameter preparation of the temporal attention layer (layers.py:105-169 weights
// in the layouts the fused kernels use), one kernel each way instead of a chain of small
// torch ops:
//   forward : wq_node = W_q[:, :Dn]; wo1 = W_o[:, :D]; wo2 = W_o[:, D:];
//             wk_aug, wv_aug = [W | b] in the K-space column layout (node, edge and time
//             parts each padded to a multiple of 4 columns, the bias at column kb, zeros
//             after it);
//             qb = b_q + W_q[:, Dn:] cos(b_t) (the query bias with the time encoding of
//             dt = 0 folded in, layers.py:109-110) and qbk[h] = qb[h-block] wk_aug[h-block].
//   backward: the gradients of W_q, b_q, W_k, b_k, W_v, b_v, b_t and W_o from those of the
//             six outputs, each written once (no zero-filled partial gradients to add).
// qb (and, backward, dqb = the gradient of qb) are D dot products of at most max(Dt, Kp)
// terms, formed first by a wave per output into 2*D floats of caller scratch. All sums run
// in a fixed order.
#include "fa_common.hpp"

namespace fa {
namespace {

constexpr int kLpMaxD = 512;       // largest dim_out
constexpr int kLpBlocks = 256;     // workgroups of the elementwise launch

struct LpParams {
  int D, H, dh, Dn, De, Dt, kp, kb;
  int cn4, ce4;                     // first K-space column of the edge / time parts
  const float* wq; int64_t ldq;     // [D, Dn + Dt]
  const float* bq;                  // [D]
  const float* wk; int64_t ldk;     // [D, Dn + De + Dt]
  const float* bk;
  const float* wv; int64_t ldv;
  const float* bv;
  const float* bt;                  // [Dt]
  const float* wo; int64_t ldo;     // [D, D + Dn]
  // forward outputs
  float* wq_node; float* wk_aug; float* wv_aug; float* qbk; float* wo1; float* wo2;
  // backward inputs (any may be null: zero gradient)
  const float* g_wq_node; const float* g_wk_aug; const float* g_wv_aug; const float* g_qbk;
  const float* g_wo1; const float* g_wo2;
  // backward outputs
  float* d_wq; float* d_bq; float* d_wk; float* d_bk; float* d_wv; float* d_bv; float* d_bt;
  float* d_wo;
};

// Input column of K-space column c (node, edge, time parts), or -1 for padding and the
// bias / zero columns.
__device__ __forceinline__ int kspace_input(const LpParams& P, int c) {
  if (c < P.cn4) return c < P.Dn ? c : -1;
  if (c < P.ce4) return c - P.cn4 < P.De ? P.Dn + (c - P.cn4) : -1;
  if (c < P.kb) return c - P.ce4 < P.Dt ? P.Dn + P.De + (c - P.ce4) : -1;
  return -1;
}

__device__ __forceinline__ float aug_value(const float* w, int64_t ld, const float* b,
                                          const LpParams& P, int i, int c) {
  if (c == P.kb) return b[i];
  const int col = kspace_input(P, c);
  return col >= 0 ? w[i * ld + col] : 0.f;
}

// vec[i] = qb[i] = b_q[i] + sum_t W_q[i, Dn + t] cos(b_t[t]) and, with DQB, vec[D + i] =
// dqb[i] = sum_c g_qbk[h(i), c] wk_aug[i, c]: a wave per output i, lanes over the sum,
// fixed-order wave sums.
template <bool DQB>
__global__ __launch_bounds__(kBlock) void lp_vectors(LpParams P, float* vec) {
  const int lane = lane_id();
  const int i = blockIdx.x * kWavesPerBlock + uniform(threadIdx.x / kWave);
  if (i >= P.D) return;
  float s = 0.f;
  for (int t = lane; t < P.Dt; t += kWave) s = fmaf(P.wq[i * P.ldq + P.Dn + t], cosf(P.bt[t]), s);
  s = wave_sum(s);
  if (lane == 0) vec[i] = P.bq[i] + s;
  if (DQB) {
    float d = 0.f;
    if (P.g_qbk) {
      const int h = i / P.dh;
      for (int c = lane; c < P.kp; c += kWave)
        d = fmaf(P.g_qbk[h * P.kp + c], aug_value(P.wk, P.ldk, P.bk, P, i, c), d);
    }
    d = wave_sum(d);
    if (lane == 0) vec[P.D + i] = d;
  }
}

__global__ __launch_bounds__(kBlock) void layer_params_fwd(LpParams P, const float* qb) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n_aug = static_cast<int64_t>(P.D) * P.kp;
  for (int64_t e = tid; e < n_aug; e += stride) {
    const int i = static_cast<int>(e / P.kp), c = static_cast<int>(e - static_cast<int64_t>(i) * P.kp);
    P.wk_aug[e] = aug_value(P.wk, P.ldk, P.bk, P, i, c);
    P.wv_aug[e] = aug_value(P.wv, P.ldv, P.bv, P, i, c);
  }
  // qbk[h, c] = sum_j qb[h*dh + j] wk_aug[h*dh + j, c]: a wave per output, lanes over j,
  // fixed-order wave sums (a thread per output would wait on dh loads in a row)
  const int64_t wave = tid / kWave, waves = stride / kWave;
  const int lane = lane_id();
  for (int64_t e = wave; e < static_cast<int64_t>(P.H) * P.kp; e += waves) {
    const int h = static_cast<int>(e / P.kp), c = static_cast<int>(e - static_cast<int64_t>(h) * P.kp);
    float s = 0.f;
    for (int j = lane; j < P.dh; j += kWave) {
      const int i = h * P.dh + j;
      s = fmaf(qb[i], aug_value(P.wk, P.ldk, P.bk, P, i, c), s);
    }
    s = wave_sum(s);
    if (lane == 0) P.qbk[e] = s;
  }
  for (int64_t e = tid; e < static_cast<int64_t>(P.D) * P.Dn; e += stride) {
    const int i = static_cast<int>(e / P.Dn), n = static_cast<int>(e - static_cast<int64_t>(i) * P.Dn);
    P.wq_node[e] = P.wq[i * P.ldq + n];
    P.wo2[e] = P.wo[i * P.ldo + P.D + n];
  }
  for (int64_t e = tid; e < static_cast<int64_t>(P.D) * P.D; e += stride) {
    const int i = static_cast<int>(e / P.D), j = static_cast<int>(e - static_cast<int64_t>(i) * P.D);
    P.wo1[e] = P.wo[i * P.ldo + j];
  }
}

__device__ __forceinline__ float at_or_zero(const float* p, int64_t i) { return p ? p[i] : 0.f; }

__global__ __launch_bounds__(kBlock) void layer_params_bwd(LpParams P, const float* vec) {
  const float* qb = vec;
  const float* dqb = vec + P.D;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int din = P.Dn + P.De + P.Dt;
  // K-space column of input column `col`
  auto kcol = [&](int col) {
    if (col < P.Dn) return col;
    if (col < P.Dn + P.De) return P.cn4 + (col - P.Dn);
    return P.ce4 + (col - P.Dn - P.De);
  };
  // d wk_aug[i, c] in total = g_wk_aug[i, c] + qb[i] g_qbk[h(i), c]
  for (int64_t e = tid; e < static_cast<int64_t>(P.D) * (din + 1); e += stride) {
    const int i = static_cast<int>(e / (din + 1)), col = static_cast<int>(e - static_cast<int64_t>(i) * (din + 1));
    const int c = col < din ? kcol(col) : P.kb;
    const int64_t a = static_cast<int64_t>(i) * P.kp + c;
    const float gk = at_or_zero(P.g_wk_aug, a) + qb[i] * at_or_zero(P.g_qbk, (i / P.dh) * P.kp + c);
    const float gv = at_or_zero(P.g_wv_aug, a);
    if (col < din) {
      P.d_wk[static_cast<int64_t>(i) * din + col] = gk;
      P.d_wv[static_cast<int64_t>(i) * din + col] = gv;
    } else {
      P.d_bk[i] = gk;
      P.d_bv[i] = gv;
    }
  }
  // W_q: node columns from wq_node's gradient, time columns dqb[i] cos(b_t); b_q = dqb
  const int dq_in = P.Dn + P.Dt;
  for (int64_t e = tid; e < static_cast<int64_t>(P.D) * dq_in; e += stride) {
    const int i = static_cast<int>(e / dq_in), col = static_cast<int>(e - static_cast<int64_t>(i) * dq_in);
    P.d_wq[e] = col < P.Dn ? at_or_zero(P.g_wq_node, static_cast<int64_t>(i) * P.Dn + col)
                           : dqb[i] * cosf(P.bt[col - P.Dn]);
  }
  for (int64_t e = tid; e < P.D; e += stride) P.d_bq[e] = dqb[e];
  // b_t: -sin(b_t[t]) sum_i dqb[i] W_q[i, Dn + t]
  // (a wave per t, lanes over i, fixed-order wave sums)
  const int64_t wave = tid / kWave, waves = stride / kWave;
  const int lane = lane_id();
  for (int64_t t = wave; t < P.Dt; t += waves) {
    float s = 0.f;
    for (int i = lane; i < P.D; i += kWave) s = fmaf(dqb[i], P.wq[i * P.ldq + P.Dn + t], s);
    s = wave_sum(s);
    if (lane == 0) P.d_bt[t] = -sinf(P.bt[t]) * s;
  }
  // W_o = [wo1 | wo2]
  const int do_in = P.D + P.Dn;
  for (int64_t e = tid; e < static_cast<int64_t>(P.D) * do_in; e += stride) {
    const int i = static_cast<int>(e / do_in), col = static_cast<int>(e - static_cast<int64_t>(i) * do_in);
    P.d_wo[e] = col < P.D ? at_or_zero(P.g_wo1, static_cast<int64_t>(i) * P.D + col)
                          : at_or_zero(P.g_wo2, static_cast<int64_t>(i) * P.Dn + (col - P.D));
  }
}

// The shape and the inputs both directions read (W_q, b_q, W_k, b_k, b_t).
int fill_lp(int32_t d, int32_t heads, int32_t dn, int32_t de, int32_t dt, const float* wq,
            int64_t ldq, const float* bq, const float* wk, int64_t ldk, const float* bk,
            const float* bt, LpParams& P) {
  if (d <= 0 || d > kLpMaxD || heads <= 0 || d % heads || dn <= 0 || de < 0 || dt < 0)
    return FA_EINVAL;
  if (!wq || !bq || !wk || !bk || (dt > 0 && !bt)) return FA_EINVAL;
  if (ldq < dn + dt || ldk < dn + de + dt) return FA_EINVAL;
  P = LpParams{};
  P.D = d; P.H = heads; P.dh = d / heads; P.Dn = dn; P.De = de; P.Dt = dt;
  P.cn4 = 4 * static_cast<int>(ceil_div(dn, 4));
  P.ce4 = P.cn4 + 4 * static_cast<int>(ceil_div(de, 4));
  P.kb = P.ce4 + 4 * static_cast<int>(ceil_div(dt, 4));
  P.kp = P.kb + 4;
  P.wq = wq; P.ldq = ldq; P.bq = bq; P.wk = wk; P.ldk = ldk; P.bk = bk; P.bt = bt;
  return FA_OK;
}

int lp_grid(const LpParams& P) {
  const int64_t work = static_cast<int64_t>(P.D) * P.kp;
  const int64_t want = ceil_div(work, kBlock);
  return static_cast<int>(want < kLpBlocks ? (want < 1 ? 1 : want) : kLpBlocks);
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_layer_params_fwd_f32(int32_t d, int32_t heads, int32_t dn, int32_t de,
                                       int32_t dt, const float* wq, int64_t ldq, const float* bq,
                                       const float* wk, int64_t ldk, const float* bk,
                                       const float* wv, int64_t ldv, const float* bv,
                                       const float* bt, const float* wo, int64_t ldo,
                                       float* wq_node, float* wk_aug, float* wv_aug, float* qbk,
                                       float* wo1, float* wo2, float* scratch,
                                       hipStream_t stream) {
  LpParams P;
  const int st = fill_lp(d, heads, dn, de, dt, wq, ldq, bq, wk, ldk, bk, bt, P);
  if (st != FA_OK) return st;
  if (!wv || !bv || !wo || ldv < dn + de + dt || ldo < d + dn) return FA_EINVAL;
  if (!wq_node || !wk_aug || !wv_aug || !qbk || !wo1 || !wo2) return FA_EINVAL;
  P.wv = wv; P.ldv = ldv; P.bv = bv; P.wo = wo; P.ldo = ldo;
  if (!scratch) return FA_ESCRATCH;
  P.wq_node = wq_node; P.wk_aug = wk_aug; P.wv_aug = wv_aug; P.qbk = qbk; P.wo1 = wo1; P.wo2 = wo2;
  hipLaunchKernelGGL(lp_vectors<false>, dim3(static_cast<unsigned>(ceil_div(d, kWavesPerBlock))),
                     dim3(kBlock), 0, stream, P, scratch);
  hipLaunchKernelGGL(layer_params_fwd, dim3(static_cast<unsigned>(lp_grid(P))), dim3(kBlock), 0,
                     stream, P, static_cast<const float*>(scratch));
  return launch_status();
}

extern "C" int fa_layer_params_bwd_f32(int32_t d, int32_t heads, int32_t dn, int32_t de,
                                       int32_t dt, const float* wq, int64_t ldq, const float* bq,
                                       const float* wk, int64_t ldk, const float* bk,
                                       const float* bt, const float* g_wq_node,
                                       const float* g_wk_aug, const float* g_wv_aug,
                                       const float* g_qbk, const float* g_wo1,
                                       const float* g_wo2, float* d_wq, float* d_bq, float* d_wk,
                                       float* d_bk, float* d_wv, float* d_bv, float* d_bt,
                                       float* d_wo, float* scratch, hipStream_t stream) {
  LpParams P;
  const int st = fill_lp(d, heads, dn, de, dt, wq, ldq, bq, wk, ldk, bk, bt, P);
  if (st != FA_OK) return st;
  if (!d_wq || !d_bq || !d_wk || !d_bk || !d_wv || !d_bv || !d_wo || (dt > 0 && !d_bt))
    return FA_EINVAL;
  P.g_wq_node = g_wq_node; P.g_wk_aug = g_wk_aug; P.g_wv_aug = g_wv_aug; P.g_qbk = g_qbk;
  P.g_wo1 = g_wo1; P.g_wo2 = g_wo2;
  P.d_wq = d_wq; P.d_bq = d_bq; P.d_wk = d_wk; P.d_bk = d_bk; P.d_wv = d_wv; P.d_bv = d_bv;
  P.d_bt = d_bt; P.d_wo = d_wo;
  if (!scratch) return FA_ESCRATCH;
  hipLaunchKernelGGL(lp_vectors<true>, dim3(static_cast<unsigned>(ceil_div(d, kWavesPerBlock))),
                     dim3(kBlock), 0, stream, P, scratch);
  hipLaunchKernelGGL(layer_params_bwd, dim3(static_cast<unsigned>(lp_grid(P))), dim3(kBlock), 0,
                     stream, P, static_cast<const float*>(scratch));
  return launch_status();
}
