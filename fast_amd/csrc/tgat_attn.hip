// Fused TGAT temporal attention over sampled temporal neighbours.
//
// For destination v with edges e in rowptr[v]..rowptr[v+1] and heads h:
//   x_e        = [node_tab[node_row(e)] | edge_tab[edge_row(e)] | cos(w*dt_e + b) | 1]
//   z[e,h]     = qt[v,h,:] . x_e                     (qt = Q_h W_k,aug[h], bias in col Kb)
//   s[e,h]     = leaky_relu(z, slope)
//   a[e,h]     = exp(s - max_v,h) / sum_v,h          (softmax over the destination's edges)
//   xbar[v,h]  = sum_e a[e,h] * drop[e,h] * x_e      (column Kb = sum_e a*drop)
//
// x_e is gathered and time-encoded on the fly and never stored. Layout of one row in
// "K-space" (float4 chunks): node chunks [0,cn), edge chunks [cn,cn+ce), time chunks
// [cn+ce, cn+ce+ct), then one bias chunk (1,0,0,0). One wavefront per destination
// (grid-stride); lane l owns chunks l, l+64, ... (NS slots). Per-destination rows (qt,
// xbar, dxbar, dqt) are [heads][Kp] blocks at a row stride per destination.
//
// Gathers are buffer loads through a per-row descriptor sized to the row (reads past the
// row end or of a row id out of range return 0), issued only by the lanes whose chunk lies
// in that table; the other lanes take their chunk (time, bias or zero) from a per-wave LDS
// tile row. Wave-level control flow depends only on wave-uniform values, except for those
// exec-masked loads and LDS reads.
//
// Latency structure: the per-edge ids, dt, dropout multipliers (and scores in backward) of
// up to 64 edges are loaded with one coalesced vector load per array and broadcast with
// readlane; row gathers run two batches deep (the next batch's loads are in flight while
// the current one is scored); time encodings are evaluated by all 64 lanes (dims lane,
// lane+64, ...) into the LDS tile.
//
// Backward, per destination, in one pass over the edges:
//   T_h     = dxbar[h] . xbar[h]                      (= sum_e a*drop*(dxbar[h] . x_e))
//   da'     = dxbar[h] . x_e
//   dz      = a * (drop*da' - T_h) * leaky'(s)
//   dqt[h] += dz * x_e
//   (bias column of dqt, x_e = 1: with sum_e a = 1 and T_h = sum_e a*drop*da', the sum of dz
//    over the destination's edges is -(1 - slope) * sum over the edges with s <= 0 of
//    a * (drop*da' - T_h); that form is accumulated instead, since the plain sum of dz
//    cancels to a small number and would keep only the rounding of its terms. The bias chunk
//    (1, 0, 0, 0) is the last chunk, so it lies in the last register slot of one lane, which
//    multiplies that slot by dz * (s > 0 ? 0 : (slope - 1) / slope) = the term above in place
//    of dz: see bias_dz. A slope of 0 leaves the plain sum of dz)
//   dx_e    = sum_h a*drop*dxbar[h] + dz*qt[h]        -> node-row gradient, time-encoding grads
#include <float.h>

#include "fa_common.hpp"
#include <type_traits>

namespace fa {
namespace {


// Tunables (build-time): edges per batch (two batches are in flight), and the minimum
// waves per SIMD the compiler must allow for the forward / backward kernels.
#ifndef FA_TGAT_BATCH
#define FA_TGAT_BATCH 2
#endif
// Minimum waves per SIMD the fused kernels are compiled for (a register budget). For the
// common shapes (up to 2 heads, Kp <= 512) the forward runs at 4 waves and the backward at 3,
// which measured faster than the register-unconstrained builds despite a few spilled
// values; other shapes leave the choice to the compiler.
constexpr int fwd_min_waves(int H, int NS) { return (H <= 2 && NS <= 2) ? 4 : 1; }
constexpr int bwd_min_waves(int H, int NS) { return (H <= 2 && NS <= 2) ? 3 : 1; }
constexpr int kBatch = FA_TGAT_BATCH;
constexpr int kMaxBlocks = 2048;      // grid cap of the grid-stride kernels (time-grad partial rows)
constexpr uint32_t kOob = 0x7ffffff0u;  // buffer offset past every descriptor's range

struct TgatParams {
  int64_t n_dst, n_edges;
  const int32_t* rowptr;
  const char* node_tab; int64_t ld_node; int64_t n_node; int dn; const int64_t* node_idx;
  const char* edge_tab; int64_t ld_edge; int64_t n_erow; int de; const int64_t* edge_idx;
  int node_bf16, edge_bf16;           // table element type: bf16 (else float32)
  // Row access mode: 0 = chunk loads (aligned rows, width a multiple of 4); 1 = chunk loads
  // over the padded row (aligned rows, ld a multiple of 4, width not), the components past
  // the width zeroed; 2 = element loads (unaligned rows).
  int node_tail, edge_tail;
  uint32_t node_row_bytes, edge_row_bytes;  // descriptor range of a valid row
  uint64_t node_stride, edge_stride;        // bytes between rows
  int dnode_dwords;                   // node-gradient rows stored dword by dword
  const float* dt; const float* time_w; const float* time_b; int dt_dim;
  int cn, ce, ct, cp;                 // chunk counts; cp = cn+ce+ct+1
  int tvs;                            // LDS row stride of the tiles: 4*ct + bias chunk + zero chunk
  int64_t kp;                         // row stride of qt / xbar = 4*cp
  const float* qt; int64_t qt_rs, qt_hs;    // row (destination) and head strides
  float slope;
  const float* drop;                  // explicit [E][H] multipliers, or
  uint64_t drop_seed; float drop_p, drop_scale; int drop_hash;  // hashed dropout
  // forward outputs / backward input
  float* xbar; int64_t xbar_rs, xbar_hs;
  float* scores; float* stats;
  // backward
  const float* dxbar; int64_t dxbar_rs, dxbar_hs;
  const float* tdot;                  // [n_dst][H] dxbar . xbar when given (xbar then unread)
  float* dqt; int64_t dqt_rs, dqt_hs;
  float* d_node; int64_t ld_dnode;
  float* partial;                     // [gridDim.x][2][dt_dim]
};

// ----- buffer access -------------------------------------------------------------------
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // raw (unformatted) 32-bit buffer

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kRsrcWord3);
}

// AUX: the cache-policy bits of the access; kStream (non-temporal) marks the per-destination
// K-space rows, read or written once per launch, so that they leave the caches first and
// the gathered table rows, which repeat, stay.
constexpr int kStream = 2;
template <int AUX = 0>
__device__ __forceinline__ float4 bload4(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, AUX);
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                     __uint_as_float(v[3]));
}

// Four dword loads: each dword is range-checked on its own, so a chunk that crosses the end
// of the row keeps its in-range part and reads 0 past it.
__device__ __forceinline__ float4 bload4_dwords(rsrc_t r, uint32_t off) {
  const int o = static_cast<int>(off);
  return make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4, 0, 0)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 8, 0, 0)),
                     __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 12, 0, 0)));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Four bf16 values widened to float: one 8-byte load (chunk-aligned rows) ...
__device__ __forceinline__ float4 bload4_bf16(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
  return make_float4(bf16_lo(v[0]), bf16_hi(v[0]), bf16_lo(v[1]), bf16_hi(v[1]));
}

// ... or four 2-byte loads, each range-checked (row ends, unaligned rows).
__device__ __forceinline__ float4 bload4_bf16_elems(rsrc_t r, uint32_t off) {
  const int o = static_cast<int>(off);
  return make_float4(bf16_lo(__builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0)),
                     bf16_lo(__builtin_amdgcn_raw_buffer_load_b16(r, o + 2, 0, 0)),
                     bf16_lo(__builtin_amdgcn_raw_buffer_load_b16(r, o + 4, 0, 0)),
                     bf16_lo(__builtin_amdgcn_raw_buffer_load_b16(r, o + 6, 0, 0)));
}

// One row chunk of 4 values as float (the branches are wave-uniform).
__device__ __forceinline__ float4 load_chunk(rsrc_t r, uint32_t off, int bf16, int mode) {
  if (bf16) return mode == 2 ? bload4_bf16_elems(r, off) : bload4_bf16(r, off);
  return mode == 2 ? bload4_dwords(r, off) : bload4(r, off);
}

// Keeps the first `valid` components (a chunk that crosses the end of a feature row).
__device__ __forceinline__ float4 keep_first(const float4& v, int valid) {
  return make_float4(v.x, valid > 1 ? v.y : 0.f, valid > 2 ? v.z : 0.f, valid > 3 ? v.w : 0.f);
}

// Four dword stores: each dword is range-checked on its own, so a chunk that crosses the end
// of the row writes only its in-range part.
__device__ __forceinline__ void bstore4_dwords(rsrc_t r, uint32_t off, const float4& x) {
  const int o = static_cast<int>(off);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.x), r, o, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.y), r, o + 4, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.z), r, o + 8, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x.w), r, o + 12, 0, 0);
}

// The same non-temporal policy for plain float4 pointers.
typedef float nt4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float4* p) {
  const nt4 v = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store_nt(float4* p, const float4& x) {
  const nt4 v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<nt4*>(p));
}

template <int AUX = 0>
__device__ __forceinline__ void bstore4(rsrc_t r, uint32_t off, const float4& x) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  u4 v;
  v[0] = __float_as_uint(x.x);
  v[1] = __float_as_uint(x.y);
  v[2] = __float_as_uint(x.z);
  v[3] = __float_as_uint(x.w);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(off), 0, AUX);
}

__device__ __forceinline__ int64_t clamp_edge(int64_t e, int64_t n_edges) {
  return e < 0 ? 0 : (e > n_edges ? n_edges : e);
}

__device__ __forceinline__ int lane_int(int v, int j) { return __builtin_amdgcn_readlane(v, j); }
__device__ __forceinline__ float lane_flt(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// ----- per-lane chunk bookkeeping ------------------------------------------------------
// Each lane owns the K-space chunks lane + 64k (slot k). Row chunks (node / edge feature
// rows) come from global memory; every other chunk is read from the wave's LDS tile row of
// the edge, laid out as [time chunks (ct) | bias chunk (1,0,0,0) | zero chunk], so a lane
// picks between two values with one select and no branch.
// The multiplier of the last register slot: dz, except in the lane holding the bias chunk,
// where it is the bias column's non-cancelling term dz * (s > 0 ? 0 : (slope - 1) / slope).
__device__ __forceinline__ float bias_dz(const TgatParams& P, bool bias_lane, float s, float dz) {
  const float kq = P.slope != 0.f ? (P.slope - 1.f) / P.slope : 1.f;
  return bias_lane ? dz * (s > 0.f && P.slope != 0.f ? 0.f : kq) : dz;
}

template <int NS>
struct LaneCtx {
  uint32_t noff[NS];      // byte offset of a node chunk in the node row (kOob elsewhere)
  uint32_t eoff[NS];      // byte offset of an edge chunk in the edge row (kOob elsewhere)
  uint32_t toff[NS];      // element offset of the chunk in the LDS tile row (zero chunk for rows)
  bool is_node[NS], is_edge[NS];
  bool slot_node[NS], slot_time[NS];  // wave-uniform: slot k holds some node / time chunk
  uint32_t time_off;      // LDS tile offset of this lane's time chunk (zero chunk if none)
  float w0, b0, w1, b1;   // time dims j = lane and lane + 64
  bool bias_lane;         // slot NS-1 holds the bias chunk (chunk cp-1)
};

template <int NS>
__device__ __forceinline__ void setup_lane(const TgatParams& P, LaneCtx<NS>& L) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int c = lane + k * kWave;
    if (k == 0) L.time_off = 4u * static_cast<uint32_t>(P.ct + 1);
    L.slot_node[k] = k * kWave < P.cn;
    L.slot_time[k] = P.ct > 0 && k * kWave < P.cn + P.ce + P.ct && (k + 1) * kWave > P.cn + P.ce;
    L.noff[k] = kOob;
    L.eoff[k] = kOob;
    L.toff[k] = 4u * static_cast<uint32_t>(P.ct + 1);
    L.is_node[k] = false;
    L.is_edge[k] = false;
    if (c < P.cn) {
      L.noff[k] = (P.node_bf16 ? 8u : 16u) * static_cast<uint32_t>(c);
      L.is_node[k] = true;
    } else if (c < P.cn + P.ce) {
      L.eoff[k] = (P.edge_bf16 ? 8u : 16u) * static_cast<uint32_t>(c - P.cn);
      L.is_edge[k] = true;
    } else if (c < P.cn + P.ce + P.ct) {
      L.toff[k] = 4u * static_cast<uint32_t>(c - P.cn - P.ce);
      L.time_off = L.toff[k];
    } else if (c == P.cn + P.ce + P.ct) {
      L.toff[k] = 4u * static_cast<uint32_t>(P.ct);
    }
  }
  L.bias_lane = lane + (NS - 1) * kWave == P.cp - 1;
  L.w0 = lane < P.dt_dim ? P.time_w[lane] : 0.f;
  L.b0 = lane < P.dt_dim ? P.time_b[lane] : 0.f;
  L.w1 = lane + kWave < P.dt_dim ? P.time_w[lane + kWave] : 0.f;
  L.b1 = lane + kWave < P.dt_dim ? P.time_b[lane + kWave] : 0.f;
}

// Writes the constant part [dt_dim, tvs) of `rows` rows of this wave's tiles: time padding
// and the zero chunk get 0; the bias chunk gets (1,0,0,0) in the first `cos_rows` rows
// (cosine tiles) and zeros in the others (-sin tiles, whose non-time chunks must be 0).
__device__ __forceinline__ void init_tiles(const TgatParams& P, float* tile, int rows,
                                           int cos_rows) {
  const int lane = lane_id();
  const int pad = P.tvs - P.dt_dim;
  for (int i = lane; i < rows * pad; i += kWave) {
    const int r = i / pad;
    const int j = P.dt_dim + (i - r * pad);
    tile[r * P.tvs + j] = (j == 4 * P.ct && r < cos_rows) ? 1.f : 0.f;
  }
  lds_sync();
}

// ----- per-edge metadata ---------------------------------------------------------------
// Per-lane metadata of up to 64 consecutive edges c0 + lane: row ids (split in 32-bit
// halves for readlane), dt, dropout multipliers and (backward) scores.
constexpr uint32_t kNoRow = 0xffffffffu;  // staged row id of a missing / out-of-range row

template <int H, bool SCORES>
struct EdgeMeta {
  uint32_t nid, eid;                        // row ids, kNoRow when outside the table
  float t;
  float dr[H];
  float sc[H];
};

template <int H, bool SCORES>
__device__ __forceinline__ void stage_meta(const TgatParams& P, int64_t c0, int cnt,
                                           EdgeMeta<H, SCORES>& M) {
  const int lane = lane_id();
  const int64_t e = c0 + (lane < cnt ? lane : 0);
  const int64_t nr = P.node_idx ? P.node_idx[e] : e;
  const int64_t er = P.edge_idx ? P.edge_idx[e] : e;
  // range-checked here, once per edge, so that one 32-bit value per row reaches the loads
  M.nid = (nr >= 0 && nr < P.n_node) ? static_cast<uint32_t>(nr) : kNoRow;
  M.eid = (er >= 0 && er < P.n_erow) ? static_cast<uint32_t>(er) : kNoRow;
  M.t = P.dt_dim > 0 ? P.dt[e] : 0.f;
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float dr = 1.f;
    if (P.drop) dr = P.drop[e * H + h];
    else if (P.drop_hash) dr = drop_mult(P.drop_seed, static_cast<uint64_t>(e * H + h), P.drop_p, P.drop_scale);
    M.dr[h] = dr;
    M.sc[h] = SCORES ? P.scores[e * H + h] : 0.f;
  }
}

template <int H, bool SCORES>
__device__ __forceinline__ uint32_t meta_node(const EdgeMeta<H, SCORES>& M, int j) {
  return static_cast<uint32_t>(lane_int(static_cast<int>(M.nid), j));
}

template <int H, bool SCORES>
__device__ __forceinline__ uint32_t meta_edge(const EdgeMeta<H, SCORES>& M, int j) {
  return static_cast<uint32_t>(lane_int(static_cast<int>(M.eid), j));
}

// Issues the row-chunk loads of batch entries [jb, jb+nb): the lanes of node chunks load
// from the node row, the lanes of edge chunks from the edge row, through buffer
// descriptors whose range is the row itself (zero for a row id out of range), so the
// hardware returns 0 past the row end and for missing rows; the other lanes load nothing.
template <int NS, int H, bool SCORES>
__device__ __forceinline__ void issue_rows(const TgatParams& P, const LaneCtx<NS>& L,
                                           const EdgeMeta<H, SCORES>& M, int jb, int nb,
                                           float4 (&x)[kBatch][NS]) {
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    if (b < nb) {
      const uint32_t nrow = meta_node(M, jb + b);
      const uint32_t erow = meta_edge(M, jb + b);
      const bool nok = nrow != kNoRow, eok = erow != kNoRow;
      const rsrc_t nr = make_rsrc(P.node_tab + static_cast<uint64_t>(nok ? nrow : 0u) * P.node_stride,
                                  nok ? P.node_row_bytes : 0u);
      const rsrc_t er = make_rsrc(P.edge_tab + static_cast<uint64_t>(eok ? erow : 0u) * P.edge_stride,
                                  eok ? P.edge_row_bytes : 0u);
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        if (L.is_node[k]) {
          float4 v = load_chunk(nr, L.noff[k], P.node_bf16, P.node_tail);
          if (P.node_tail == 1) v = keep_first(v, P.dn - static_cast<int>(L.noff[k] >> (P.node_bf16 ? 1 : 2)));
          x[b][k] = v;
        } else if (L.is_edge[k]) {
          float4 v = load_chunk(er, L.eoff[k], P.edge_bf16, P.edge_tail);
          if (P.edge_tail == 1) v = keep_first(v, P.de - static_cast<int>(L.eoff[k] >> (P.edge_bf16 ? 1 : 2)));
          x[b][k] = v;
        }
      }
    }
  }
}

template <bool SIN>
__device__ __forceinline__ void encode_one(float a, float* rc, float* rs, int j, bool ok) {
  float sv, cv;
  sincos_hw(a, sv, cv);
  if (fabsf(a) > trig::kMaxArg) {  // outside the reduction's range (not expected for times)
    if (SIN) sincosf(a, &sv, &cv);
    else cv = cosf(a);
  }
  if (ok) {
    rc[j] = cv;
    if (SIN) rs[j] = -sv;
  }
}

// cos (and, with SIN, -sin) of the time arguments of batch entries [jb, jb+nb) into the
// LDS tiles tc[b][j] / ts[b][j]; every lane evaluates dims lane, lane+64, ...
template <int NS, int H, bool SCORES, bool SIN>
__device__ __forceinline__ void encode_times(const TgatParams& P, const LaneCtx<NS>& L,
                                             const EdgeMeta<H, SCORES>& M, int jb, int nb,
                                             float* tc, float* ts) {
  const int lane = lane_id();
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    if (b >= nb) break;
    const float t = lane_flt(M.t, jb + b);
    float* rc = tc + b * P.tvs;
    float* rs = SIN ? ts + b * P.tvs : nullptr;
    encode_one<SIN>(time_arg(t, L.w0, L.b0), rc, rs, lane, lane < P.dt_dim);
    if (P.dt_dim > kWave)
      encode_one<SIN>(time_arg(t, L.w1, L.b1), rc, rs, lane + kWave, lane + kWave < P.dt_dim);
    for (int j0 = 2 * kWave; j0 < P.dt_dim; j0 += kWave) {
      const int j = j0 + lane;
      const int jc = j < P.dt_dim ? j : P.dt_dim - 1;
      encode_one<SIN>(time_arg(t, P.time_w[jc], P.time_b[jc]), rc, rs, j, j < P.dt_dim);
    }
  }
}

// Completes the batch's chunks: lanes of row chunks keep what they loaded, every other lane
// reads its chunk (time, bias or zero) from the LDS tile row of the entry.
template <int NS>
__device__ __forceinline__ void assemble_x(const TgatParams& P, const LaneCtx<NS>& L, int nb,
                                           const float* tc, float4 (&x)[kBatch][NS]) {
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    if (b >= nb) break;
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if (!(L.is_node[k] || L.is_edge[k]))
        x[b][k] = *reinterpret_cast<const float4*>(tc + b * P.tvs + L.toff[k]);
  }
}

// Rows of a per-destination [heads][Kp] block: destination v, head h starts at
// base + v*rs + h*hs.
template <int H, int NS>
__device__ __forceinline__ void load_rows(const float* base, int64_t rs, int64_t hs, int64_t v,
                                          int64_t kp, float4 (&r)[H][NS]) {
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const rsrc_t rr = make_rsrc(base + v * rs + h * hs, 4u * static_cast<uint32_t>(kp));
#pragma unroll
    for (int k = 0; k < NS; ++k) r[h][k] = bload4<kStream>(rr, 16u * static_cast<uint32_t>(lane + k * kWave));
  }
}

// q~ chunks the backward reads: the node chunks (with a node-row gradient) and the time
// chunks (the time gradient); the edge chunks and the bias chunk enter no gradient through q~.
__device__ __forceinline__ bool q_chunk_used(const TgatParams& P, int c) {
  const int t0 = P.cn + P.ce;
  return (c >= t0 && c < t0 + P.ct) || (P.d_node && c < P.cn);
}

// load_rows of q~ for the backward: the chunks it does not read come back as zeros, unread.
template <int H, int NS>
__device__ __forceinline__ void load_q_rows(const TgatParams& P, int64_t v, float4 (&r)[H][NS]) {
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const rsrc_t rr = make_rsrc(P.qt + v * P.qt_rs + h * P.qt_hs, 4u * static_cast<uint32_t>(P.kp));
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int c = lane + k * kWave;
      r[h][k] = bload4<kStream>(rr, q_chunk_used(P, c) ? 16u * static_cast<uint32_t>(c) : 0x7ffffff0u);
    }
  }
}

template <int H, int NS>
__device__ __forceinline__ void store_rows(float* base, int64_t rs, int64_t hs, int64_t v,
                                           int64_t kp, const float4 (&r)[H][NS]) {
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const rsrc_t rr = make_rsrc(base + v * rs + h * hs, 4u * static_cast<uint32_t>(kp));
#pragma unroll
    for (int k = 0; k < NS; ++k) bstore4<kStream>(rr, 16u * static_cast<uint32_t>(lane + k * kWave), r[h][k]);
  }
}

template <int NS>
__device__ __forceinline__ float row_dot(const float4 (&a)[NS], const float4 (&b)[NS]) {
  float p = 0.f;
#pragma unroll
  for (int k = 0; k < NS; ++k) p += dot4(a[k], b[k]);
  return p;
}

// ---------------------------------------------------------------------------------
// Forward: one wave per destination (grid-stride over destinations), online softmax over
// batches of kBatch edges.
// Dynamic LDS: per wave one [kBatch][tvs] cosine tile.
// ---------------------------------------------------------------------------------
template <int H, int NS>
struct FwdState {
  float4 q[H][NS];
  float4 acc[H][NS];
  float m[H], l[H];
};

template <int H, int NS>
__device__ __forceinline__ void fwd_batch(const TgatParams& P, const LaneCtx<NS>& L,
                                          const EdgeMeta<H, false>& M, int64_t c0, int jb, int nb,
                                          float* tc, float4 (&x)[kBatch][NS],
                                          FwdState<H, NS>& S) {
  const int lane = lane_id();
  if (P.dt_dim > 0) {
    lds_sync();
    encode_times<NS, H, false, false>(P, L, M, jb, nb, tc, nullptr);
    lds_sync();
  }
  assemble_x<NS>(P, L, nb, tc, x);
  float sc[kBatch][H];
#pragma unroll
  for (int b = 0; b < kBatch; ++b)
#pragma unroll
    for (int h = 0; h < H; ++h) sc[b][h] = leaky(wave_sum(row_dot<NS>(S.q[h], x[b])), P.slope);
  {
    // scores of the batch: lane b*H+h stores s[c0+jb+b, h] (contiguous)
    float mine = 0.f;
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int h = 0; h < H; ++h) mine = (lane == b * H + h) ? sc[b][h] : mine;
    if (lane < nb * H) P.scores[(c0 + jb) * H + lane] = mine;
  }
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    if (b >= nb) break;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float s = sc[b][h];
      const float dr = lane_flt(M.dr[h], jb + b);
      // online softmax; s and m are wave-uniform, so this branch does not diverge. The
      // first edge has m = -inf and r = 0.
      if (s > S.m[h]) {
        const float r = exp_fast(S.m[h] - s);
        S.l[h] *= r;
#pragma unroll
        for (int k = 0; k < NS; ++k) scale4(S.acc[h][k], r);
        S.m[h] = s;
      }
      const float pe = exp_fast(s - S.m[h]);
      S.l[h] += pe;
      const float w = pe * dr;
#pragma unroll
      for (int k = 0; k < NS; ++k) fma4(S.acc[h][k], w, x[b][k]);
    }
  }
}

template <int H, int NS>
__global__ __launch_bounds__(kBlock, fwd_min_waves(H, NS)) void tgat_fwd(TgatParams P) {
  extern __shared__ float lds[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = lane_id();
  float* tc = lds + wave * (kBatch * P.tvs);
  LaneCtx<NS> L;
  setup_lane<NS>(P, L);
  init_tiles(P, tc, kBatch, kBatch);

  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave; v < P.n_dst;
       v += total_waves) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
    FwdState<H, NS> S;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      S.m[h] = -INFINITY;
      S.l[h] = 0.f;
#pragma unroll
      for (int k = 0; k < NS; ++k) S.acc[h][k] = f4_zero();
    }
    if (e1 <= e0) {  // zero-degree destination: xbar = 0
      store_rows<H, NS>(P.xbar, P.xbar_rs, P.xbar_hs, v, P.kp, S.acc);
      if (lane < H) {
        P.stats[(v * H + lane) * 2 + 0] = -INFINITY;
        P.stats[(v * H + lane) * 2 + 1] = 0.f;
      }
      continue;
    }
    // Prologue: the first chunk's metadata and the q~ rows are fetched together, and the
    // first batch's gathers are in flight before anything waits on q~.
    int64_t c0 = e0;
    int cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
    EdgeMeta<H, false> M;
    stage_meta<H, false>(P, c0, cnt, M);
    load_rows<H, NS>(P.qt, P.qt_rs, P.qt_hs, v, P.kp, S.q);
    float4 xa[kBatch][NS], xb[kBatch][NS];
    issue_rows<NS, H, false>(P, L, M, 0, cnt < kBatch ? cnt : kBatch, xa);
    for (;;) {
      for (int jb = 0; jb < cnt; jb += 2 * kBatch) {
        const int na = cnt - jb < kBatch ? cnt - jb : kBatch;
        const int nb2 = cnt - jb - kBatch;
        const int nb = nb2 < 0 ? 0 : (nb2 < kBatch ? nb2 : kBatch);
        if (nb > 0) issue_rows<NS, H, false>(P, L, M, jb + kBatch, nb, xb);
        fwd_batch<H, NS>(P, L, M, c0, jb, na, tc, xa, S);
        if (nb > 0) {
          const int nn2 = cnt - jb - 2 * kBatch;
          const int nn = nn2 < 0 ? 0 : (nn2 < kBatch ? nn2 : kBatch);
          if (nn > 0) issue_rows<NS, H, false>(P, L, M, jb + 2 * kBatch, nn, xa);
          fwd_batch<H, NS>(P, L, M, c0, jb + kBatch, nb, tc, xb, S);
        }
      }
      c0 += kWave;
      if (c0 >= e1) break;
      cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
      stage_meta<H, false>(P, c0, cnt, M);
      issue_rows<NS, H, false>(P, L, M, 0, cnt < kBatch ? cnt : kBatch, xa);
    }

#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float inv = 1.f / S.l[h];
#pragma unroll
      for (int k = 0; k < NS; ++k) scale4(S.acc[h][k], inv);
    }
    store_rows<H, NS>(P.xbar, P.xbar_rs, P.xbar_hs, v, P.kp, S.acc);
    if (lane < H) {
      float mm = 0.f, ll = 0.f;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        mm = lane == h ? S.m[h] : mm;
        ll = lane == h ? S.l[h] : ll;
      }
      P.stats[(v * H + lane) * 2 + 0] = mm;
      P.stats[(v * H + lane) * 2 + 1] = ll;
    }
  }
}

// ---------------------------------------------------------------------------------
// Forward, two edges at a time: the halves of the wave (lanes 0-31 and 32-63) take the
// alternate edges c0 + 2p + half of the wave's destination. Each half holds a whole
// K-space row in its 32 lanes (lane hl owns chunks hl + 32k, k < NS), so the dot products
// reduce over 32 lanes, the softmax update runs for two edges per instruction and the
// slots are fuller (94 chunks in 96 slots at C3, against 128). The halves keep separate
// online-softmax states, merged once per destination. Rows are read with per-lane 64-bit
// addresses (the two halves read different rows), so rows must be whole chunks (row mode
// 0). Dynamic LDS: the time weights [dt_dim] (w, b), then per wave two time-tile rows
// [2][tvs].
// ---------------------------------------------------------------------------------

// Pairs whose row loads are in flight in the pair forward, and the waves per SIMD its
// register budget is sized for.
#ifndef FA_PAIR_DEPTH
#define FA_PAIR_DEPTH 2
#endif
#ifndef FA_PAIR_FWD_WAVES
#define FA_PAIR_FWD_WAVES 4
#endif
constexpr int kPairDepth = FA_PAIR_DEPTH;

template <int NS>
struct PairCtx {
  // byte offset of the lane's chunk in its node / edge row (0 for the other chunks, which
  // read the row's first chunk and discard it)
  uint32_t off[NS];
  // float offset in the time-tile row of the lane's chunk: the chunk itself for time, bias
  // and padding chunks, the tile's zero chunk for row chunks (every lane reads one)
  uint32_t toff[NS];
  bool is_node[NS], is_edge[NS], live[NS];   // live: chunk < cp (stored)
  // The lane's time chunk (at most one per lane while ct <= 32): its K-space chunk index,
  // else `zero_chunk`, and its offset in a tile row, else the tile's zero chunk.
  int tci;
  uint32_t ttoff;
  bool bias_lane;   // slot NS-1 holds the bias chunk (chunk cp-1)
};

template <int NS>
__device__ __forceinline__ void setup_pair(const TgatParams& P, PairCtx<NS>& L, int zero_chunk = 0) {
  const int hl = lane_id() & (kHalf - 1);
  L.tci = zero_chunk;
  L.ttoff = 4u * static_cast<uint32_t>(P.ct + 1);
  L.bias_lane = hl + (NS - 1) * kHalf == P.cp - 1;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int c = hl + k * kHalf;
    L.is_node[k] = c < P.cn;
    L.is_edge[k] = c >= P.cn && c < P.cn + P.ce;
    L.live[k] = c < P.cp;
    uint32_t off = 4u * static_cast<uint32_t>(P.ct + 1);
    if (L.is_node[k]) off = (P.node_bf16 ? 8u : 16u) * static_cast<uint32_t>(c);
    else if (L.is_edge[k]) off = (P.edge_bf16 ? 8u : 16u) * static_cast<uint32_t>(c - P.cn);
    else if (c < P.cn + P.ce + P.ct) {
      off = 4u * static_cast<uint32_t>(c - P.cn - P.ce);
      L.tci = c;
      L.ttoff = off;
    } else if (c == P.cn + P.ce + P.ct) {
      off = 4u * static_cast<uint32_t>(P.ct);
    }
    L.toff[k] = (L.is_node[k] || L.is_edge[k]) ? 4u * static_cast<uint32_t>(P.ct + 1) : off;
    L.off[k] = (L.is_node[k] || L.is_edge[k]) ? off : 0u;
  }
}

// Floats before the tiles in LDS: the time weights, rounded up to a whole chunk.
__host__ __device__ __forceinline__ int pair_tile_base(int dt_dim) { return (2 * dt_dim + 3) & ~3; }

// Floats of LDS per wave: two time-tile rows and the q~ rows.
__host__ __device__ __forceinline__ int pair_wave_floats(int tvs, int heads, int ns) {
  return 2 * tvs + 4 * heads * ns * kHalf;
}

// The time weights and phases, interleaved (w, b) per dimension, into `twb` (all waves of the
// workgroup).
__device__ __forceinline__ void stage_time_weights(const TgatParams& P, float2* twb) {
  for (int d = threadIdx.x; d < P.dt_dim; d += blockDim.x) twb[d] = make_float2(P.time_w[d], P.time_b[d]);
  __syncthreads();
}

__device__ __forceinline__ void pair_time(float t, float2 wb, float* row, int d, bool ok) {
  float sv, cv;
  const float a = time_arg(t, wb.x, wb.y);
  sincos_hw(a, sv, cv);
  if (fabsf(a) > trig::kMaxArg) cv = cosf(a);  // outside the reduction's range
  if (ok) row[d] = cv;
}

// The value lane j holds, for every lane (j may differ per lane).
__device__ __forceinline__ int pick_int(int v, int j) { return __builtin_amdgcn_ds_bpermute(j << 2, v); }
__device__ __forceinline__ float pick_flt(float v, int j) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(j << 2, __float_as_int(v)));
}

// A zero chunk in global memory: the load of every lane without a row chunk to read. It is a
// plain (non-const) global so that selecting between it and a table row keeps a global
// pointer: a generic pointer would make the loads flat loads, which also count against the
// LDS wait counter. Nothing writes it.
// A zero row as long as the longest row the pair kernels take (32 lanes x 4 slots of
// 16-byte chunks), read in place of a missing row.
constexpr int kPairZeroRowFloats = 4 * kHalf * 4;
__device__ __align__(16) float g_zero_row[kPairZeroRowFloats];

// Row chunks of one edge per half-wave, loaded as they are stored: float4 (BF = false) or
// four bf16 words in x.x, x.y (BF = true, widened by pair_widen where the chunk is used).
// Every lane issues its load with the whole wave active, from its node row or its edge row;
// a missing row (or no edge table, or an edge past the staged ones) is the zero row, and a
// lane whose chunk is no row chunk reads the first chunk of the edge row, which pair_widen
// discards. No branch and no conversion sits between a load and the code that consumes it a
// step later, so the compiler can wait for exactly that load (a conditional write into a
// register that still has a load in flight, or a branch around the load, makes it wait for
// every load the wave has in flight). Row strides are below 2^32 bytes, so each row address
// is one 32 x 32 -> 64-bit multiply-add.
template <int NS, bool BF>
__device__ __forceinline__ void pair_load(const TgatParams& P, const PairCtx<NS>& L, uint32_t nid,
                                          uint32_t eid, bool ok, float4 (&x)[NS]) {
  const bool nok = ok && nid != kNoRow && P.dn > 0, eok = ok && eid != kNoRow && P.de > 0;
  const char* zero = reinterpret_cast<const char*>(g_zero_row);
  const char* nrow = nok ? P.node_tab + static_cast<uint64_t>(nid) * static_cast<uint32_t>(P.node_stride) : zero;
  const char* erow = eok ? P.edge_tab + static_cast<uint64_t>(eid) * static_cast<uint32_t>(P.edge_stride) : zero;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const char* a = (L.is_node[k] ? nrow : erow) + L.off[k];
    if constexpr (BF) {
      const uint2 w = *reinterpret_cast<const uint2*>(a);
      x[k] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), 0.f, 0.f);
    } else {
      x[k] = load_nt(reinterpret_cast<const float4*>(a));
    }
  }
}

// The K-space chunks of the lane's edge: row chunks from the loads (bf16 words widened),
// every other chunk (time, bias, padding) from the time-tile row, by selects.
template <int NS, bool BF>
__device__ __forceinline__ void pair_widen(const PairCtx<NS>& L, const float* row,
                                           const float4 (&x)[NS], float4 (&xs)[NS]) {
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(row + L.toff[k]);
    float4 v = x[k];
    if constexpr (BF) {
      const uint32_t w0 = __float_as_uint(v.x), w1 = __float_as_uint(v.y);
      v = make_float4(bf16_lo(w0), bf16_hi(w0), bf16_lo(w1), bf16_hi(w1));
    }
    const bool r = L.is_node[k] || L.is_edge[k];
    xs[k] = make_float4(r ? v.x : t.x, r ? v.y : t.y, r ? v.z : t.z, r ? v.w : t.w);
  }
}

// Row chunks of this lane's edge of pair p (edge index 2p + half among the staged ones);
// lanes whose edge is past cnt, or whose row is missing, get zeros.
template <int NS, int H, bool SC, bool BF>
__device__ __forceinline__ void pair_rows(const TgatParams& P, const PairCtx<NS>& L,
                                          const EdgeMeta<H, SC>& M, int p, int cnt,
                                          float4 (&x)[NS]) {
  const int j = 2 * p + (lane_id() >= kHalf ? 1 : 0);
  const int jj = j < cnt ? j : 0;
  const uint32_t nid = static_cast<uint32_t>(pick_int(static_cast<int>(M.nid), jj));
  const uint32_t eid = static_cast<uint32_t>(pick_int(static_cast<int>(M.eid), jj));
  pair_load<NS, BF>(P, L, nid, eid, j < cnt, x);
}

template <int H, int NS>
struct PairState {
  const float4* q;    // the destination's q~ rows in LDS: [H][32 * NS] chunks
  float4 acc[H][NS];
  float m[H], l[H];
};

// Pair p: time encoding of both edges into the halves' tile rows, the other chunks from
// the tiles, scores, and the two online-softmax updates.
template <int H, int NS, bool BF>
__device__ __forceinline__ void pair_step(const TgatParams& P, const PairCtx<NS>& L,
                                          const EdgeMeta<H, false>& M, int64_t c0, int p,
                                          int cnt, const float2* twb, float* tile,
                                          const float4 (&xr)[NS], PairState<H, NS>& S) {
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int j = 2 * p + half;
  const bool valid = j < cnt;
  const int jj = valid ? j : 0;
  float* row = tile + half * P.tvs;
  if (P.dt_dim > 0) {
    lds_sync();
    const float t = pick_flt(M.t, jj);
    for (int d = hl; d < P.dt_dim; d += kHalf) pair_time(t, twb[d], row, d, true);
    lds_sync();
  }
  float4 x[NS];
  pair_widen<NS, BF>(L, row, xr, x);
  float sc[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float d = 0.f;
#pragma unroll
    for (int k = 0; k < NS; ++k) d += dot4(S.q[h * NS * kHalf + hl + k * kHalf], x[k]);
    sc[h] = leaky(half_sum(d), P.slope);
  }
  // scores: lane hl == h of each valid half writes s[c0 + j, h]
  {
    float mine = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) mine = hl == h ? sc[h] : mine;
    if (valid && hl < H) P.scores[(c0 + j) * H + hl] = mine;
  }
  float dr[H];  // picked with every lane active (bpermute reads nothing from idle lanes)
#pragma unroll
  for (int h = 0; h < H; ++h) dr[h] = pick_flt(M.dr[h], jj);
  if (valid) {
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float s = sc[h];
      if (s > S.m[h]) {  // uniform within a half
        const float r = exp_fast(S.m[h] - s);
        S.l[h] *= r;
#pragma unroll
        for (int k = 0; k < NS; ++k) scale4(S.acc[h][k], r);
        S.m[h] = s;
      }
      const float pe = exp_fast(s - S.m[h]);
      S.l[h] += pe;
      const float w = pe * dr[h];
#pragma unroll
      for (int k = 0; k < NS; ++k) fma4(S.acc[h][k], w, x[k]);
    }
  }
}

template <int H, int NS, bool BF>
__global__ __launch_bounds__(kBlock, FA_PAIR_FWD_WAVES) void tgat_fwd_pair(TgatParams P) {
  extern __shared__ float lds[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  float2* twb = reinterpret_cast<float2*>(lds);
  float* tile = lds + pair_tile_base(P.dt_dim) + wave * pair_wave_floats(P.tvs, H, NS);
  float4* qs = reinterpret_cast<float4*>(tile + 2 * P.tvs);
  PairCtx<NS> L;
  setup_pair<NS>(P, L);
  stage_time_weights(P, twb);
  init_tiles(P, tile, 2, 2);
  // chunks past cp stay zero (their x chunks are zero too)
  for (int i = lane; i < H * NS * kHalf; i += kWave) qs[i] = f4_zero();

  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave; v < P.n_dst;
       v += total_waves) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
    PairState<H, NS> S;
    S.q = qs;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      S.m[h] = -INFINITY;
      S.l[h] = 0.f;
#pragma unroll
      for (int k = 0; k < NS; ++k) S.acc[h][k] = f4_zero();
    }
    if (e1 <= e0) {  // zero-degree destination: xbar = 0
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float* dst = P.xbar + v * P.xbar_rs + h * P.xbar_hs;
#pragma unroll
        for (int k = 0; k < NS; ++k)
          if (half == 0 && L.live[k]) *reinterpret_cast<float4*>(dst + 4 * (hl + k * kHalf)) = f4_zero();
      }
      if (lane < H) {
        P.stats[(v * H + lane) * 2 + 0] = -INFINITY;
        P.stats[(v * H + lane) * 2 + 1] = 0.f;
      }
      continue;
    }
    int64_t c0 = e0;
    int cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
    EdgeMeta<H, false> M;
    stage_meta<H, false>(P, c0, cnt, M);
    // the q~ rows' loads, then the first pair's row loads (which wait for the staged ids),
    // are all in flight before the q~ rows go to LDS
    constexpr int QR = (NS * kHalf + kWave - 1) / kWave;  // q~ chunks per lane and head
    float4 qv[H][QR];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float4* src = reinterpret_cast<const float4*>(P.qt + v * P.qt_rs + h * P.qt_hs);
#pragma unroll
      for (int r = 0; r < QR; ++r) {
        const int c = lane + r * kWave;
        qv[h][r] = c < P.cp ? load_nt(src + c) : f4_zero();
      }
    }
    float4 xr[kPairDepth][NS];
#pragma unroll
    for (int r = 0; r < kPairDepth; ++r) pair_rows<NS, H, false, BF>(P, L, M, r, cnt, xr[r]);
    lds_sync();  // the previous destination's reads of qs are done
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int r = 0; r < QR; ++r) {
        const int c = lane + r * kWave;
        if (c < P.cp) qs[h * NS * kHalf + c] = qv[h][r];
      }
    lds_sync();
    for (;;) {
      const int np = (cnt + 1) >> 1;
      // A ring of kPairDepth pairs in flight: each slot is refilled right after its pair is
      // processed, with the loads of the pair kPairDepth ahead, issued whether or not that
      // pair exists (past the last pair they read the zero chunk), so every path leaves the
      // same loads in flight and the compiler waits for exactly the pair it processes.
      for (int p = 0; p < np; p += kPairDepth) {
#pragma unroll
        for (int r = 0; r < kPairDepth; ++r) {
          if (p + r < np) pair_step<H, NS, BF>(P, L, M, c0, p + r, cnt, twb, tile, xr[r], S);
          pair_rows<NS, H, false, BF>(P, L, M, p + r + kPairDepth, cnt, xr[r]);
        }
      }
      c0 += kWave;
      if (c0 >= e1) break;
      cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
      stage_meta<H, false>(P, c0, cnt, M);
#pragma unroll
      for (int r = 0; r < kPairDepth; ++r) pair_rows<NS, H, false, BF>(P, L, M, r, cnt, xr[r]);
    }
    // merge the halves: M = max(m0, m1), weights exp(m - M) (0 for a half without edges)
    const int other = lane ^ kHalf;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float mo = pick_flt(S.m[h], other), lo = pick_flt(S.l[h], other);
      const float mx = S.m[h] > mo ? S.m[h] : mo;
      const float r = S.m[h] == -INFINITY ? 0.f : exp_fast(S.m[h] - mx);
      const float ro = mo == -INFINITY ? 0.f : exp_fast(mo - mx);
      const float lt = S.l[h] * r + lo * ro;
      const float inv = 1.f / lt;
      float* dst = P.xbar + v * P.xbar_rs + h * P.xbar_hs;
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        float4 a = S.acc[h][k], b;
        b.x = pick_flt(a.x, other);
        b.y = pick_flt(a.y, other);
        b.z = pick_flt(a.z, other);
        b.w = pick_flt(a.w, other);
        a.x = (a.x * r + b.x * ro) * inv;
        a.y = (a.y * r + b.y * ro) * inv;
        a.z = (a.z * r + b.z * ro) * inv;
        a.w = (a.w * r + b.w * ro) * inv;
        if (half == 0 && L.live[k]) store_nt(reinterpret_cast<float4*>(dst + 4 * (hl + k * kHalf)), a);
      }
      if (lane == h) {
        P.stats[(v * H + h) * 2 + 0] = mx;
        P.stats[(v * H + h) * 2 + 1] = lt;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Backward: one wave per destination (grid-stride), one pass over the edges.
// Dynamic LDS: per wave [kBatch][tvs] cos and -sin tiles, then the workgroup's time-grad
// reduction buffer [kWavesPerBlock][2][tvs].
// ---------------------------------------------------------------------------------
template <int H, int NS>
struct BwdState {
  float4 q[H][NS], g[H][NS], dq[H][NS];
  float4 gw, gb;  // time-grad accumulators of this lane's time chunk (at most one: ct <= 64)
  float mh[H], il[H], T[H];  // row max, 1 / softmax denominator, dxbar . xbar
  float cb;       // lane h < H: the bias column of head h's dq~ (the non-cancelling form)
};

template <int H, int NS>
__device__ __forceinline__ void bwd_batch(const TgatParams& P, const LaneCtx<NS>& L,
                                          const EdgeMeta<H, true>& M, int64_t c0, int jb, int nb,
                                          float* tc, float* ts, float4 (&x)[kBatch][NS],
                                          BwdState<H, NS>& S) {
  if (P.dt_dim > 0) {
    lds_sync();
    encode_times<NS, H, true, true>(P, L, M, jb, nb, tc, ts);
    lds_sync();
  }
  assemble_x<NS>(P, L, nb, tc, x);
  const int lane = lane_id();
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
    if (b >= nb) break;
    const int j = jb + b;
    const int64_t e = c0 + j;
    float dap[H], ad[H], dz[H];
#pragma unroll
    for (int h = 0; h < H; ++h) dap[h] = wave_sum(row_dot<NS>(S.g[h], x[b]));
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float s = lane_flt(M.sc[h], j);
      const float dr = lane_flt(M.dr[h], j);
      const float a = exp_fast(s - S.mh[h]) * S.il[h];
      ad[h] = a * dr;
      const float gz = a * (dr * dap[h] - S.T[h]);
      dz[h] = gz * (s > 0.f ? 1.f : P.slope);
      const float cz = s > 0.f ? 0.f : (P.slope - 1.f) * gz;
      S.cb = lane == h ? S.cb + cz : S.cb;
#pragma unroll
      for (int k = 0; k < NS; ++k) fma4(S.dq[h][k], dz[h], x[b][k]);
    }
    const float t = lane_flt(M.t, j);
    const rsrc_t rd = make_rsrc(P.d_node ? P.d_node + e * P.ld_dnode : P.dxbar,
                                P.d_node ? 4u * static_cast<uint32_t>(P.dn) : 0u);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      // the input gradient dx_e is used for node chunks (when d_node is wanted) and time
      // chunks only; slots holding neither are skipped (a wave-uniform test)
      const bool want_node = P.d_node && L.slot_node[k];
      if (!(want_node || L.slot_time[k])) continue;
      float4 dx = f4_zero();
#pragma unroll
      for (int h = 0; h < H; ++h) {
        fma4(dx, ad[h], S.g[h][k]);
        fma4(dx, dz[h], S.q[h][k]);
      }
      // node-row gradient (the descriptor drops the lanes outside the node part)
      if (want_node) {
        if (P.dnode_dwords) bstore4_dwords(rd, L.noff[k], dx);
        else bstore4(rd, L.noff[k], dx);
      }
      // d cos(w t + b) = -sin(w t + b) * (t dw + db); the pad dims carry dx = 0
      if (L.slot_time[k]) {
        // the -sin tile is zero outside the time dims, so only time chunks contribute
        const float4 sn = *reinterpret_cast<const float4*>(ts + b * P.tvs + L.toff[k]);
        const float4 pr = make_float4(sn.x * dx.x, sn.y * dx.y, sn.z * dx.z, sn.w * dx.w);
        S.gb.x += pr.x;
        S.gb.y += pr.y;
        S.gb.z += pr.z;
        S.gb.w += pr.w;
        fma4(S.gw, t, pr);
      }
    }
  }
}

template <int H, int NS>
__global__ __launch_bounds__(kBlock, bwd_min_waves(H, NS)) void tgat_bwd(TgatParams P) {
  extern __shared__ float lds[];
  const int wave = uniform(threadIdx.x / kWave);
  float* tc = lds + wave * (2 * kBatch * P.tvs);
  float* ts = tc + kBatch * P.tvs;
  float* red = lds + kWavesPerBlock * 2 * kBatch * P.tvs;

  LaneCtx<NS> L;
  setup_lane<NS>(P, L);
  init_tiles(P, tc, 2 * kBatch, kBatch);
  BwdState<H, NS> S;
  S.gw = f4_zero();
  S.gb = f4_zero();

  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave; v < P.n_dst;
       v += total_waves) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int k = 0; k < NS; ++k) S.dq[h][k] = f4_zero();
    S.cb = 0.f;
    if (e1 <= e0) {
      store_rows<H, NS>(P.dqt, P.dqt_rs, P.dqt_hs, v, P.kp, S.dq);
      continue;
    }
    // Prologue: the first chunk's metadata and the per-destination rows (q~, dxbar, xbar)
    // are fetched together; the first batch's gathers are issued before T waits on them.
    int64_t c0 = e0;
    int cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
    EdgeMeta<H, true> M;
    stage_meta<H, true>(P, c0, cnt, M);
    load_q_rows<H, NS>(P, v, S.q);
    load_rows<H, NS>(P.dxbar, P.dxbar_rs, P.dxbar_hs, v, P.kp, S.g);
#pragma unroll
    for (int h = 0; h < H; ++h) {
      S.mh[h] = P.stats[(v * H + h) * 2 + 0];
      S.il[h] = 1.f / P.stats[(v * H + h) * 2 + 1];
    }
    float4 xa[kBatch][NS], xb[kBatch][NS];
    issue_rows<NS, H, true>(P, L, M, 0, cnt < kBatch ? cnt : kBatch, xa);
    if (P.tdot) {
#pragma unroll
      for (int h = 0; h < H; ++h) S.T[h] = P.tdot[v * H + h];
    } else {  // head by head: one x-bar row in registers at a time
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const rsrc_t rr = make_rsrc(P.xbar + v * P.xbar_rs + h * P.xbar_hs, 4u * static_cast<uint32_t>(P.kp));
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < NS; ++k) d += dot4(S.g[h][k], bload4(rr, 16u * static_cast<uint32_t>(lane_id() + k * kWave)));
        S.T[h] = wave_sum(d);
      }
    }
    for (;;) {
      for (int jb = 0; jb < cnt; jb += 2 * kBatch) {
        const int na = cnt - jb < kBatch ? cnt - jb : kBatch;
        const int nb2 = cnt - jb - kBatch;
        const int nb = nb2 < 0 ? 0 : (nb2 < kBatch ? nb2 : kBatch);
        if (nb > 0) issue_rows<NS, H, true>(P, L, M, jb + kBatch, nb, xb);
        bwd_batch<H, NS>(P, L, M, c0, jb, na, tc, ts, xa, S);
        if (nb > 0) {
          const int nn2 = cnt - jb - 2 * kBatch;
          const int nn = nn2 < 0 ? 0 : (nn2 < kBatch ? nn2 : kBatch);
          if (nn > 0) issue_rows<NS, H, true>(P, L, M, jb + 2 * kBatch, nn, xa);
          bwd_batch<H, NS>(P, L, M, c0, jb + kBatch, nb, tc, ts, xb, S);
        }
      }
      c0 += kWave;
      if (c0 >= e1) break;
      cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
      stage_meta<H, true>(P, c0, cnt, M);
      issue_rows<NS, H, true>(P, L, M, 0, cnt < kBatch ? cnt : kBatch, xa);
    }
    // the bias column (chunk cp-1, component x) from the lanes of cb
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float cb = lane_read(S.cb, h);
      if (L.bias_lane) S.dq[h][NS - 1].x = cb;
    }
    store_rows<H, NS>(P.dqt, P.dqt_rs, P.dqt_hs, v, P.kp, S.dq);
  }

  // Time-grad partials of this workgroup: waves combined in a fixed order. Every time dim
  // is owned by exactly one lane (time chunks span at most 64 chunks); the other lanes hold
  // zeros and write them to the zero chunk, which the sum below does not read.
  if (P.dt_dim <= 0) return;
  {
    float* rw = red + (wave * 2 + 0) * P.tvs + L.time_off;
    float* rb = red + (wave * 2 + 1) * P.tvs + L.time_off;
    rw[0] = S.gw.x; rw[1] = S.gw.y; rw[2] = S.gw.z; rw[3] = S.gw.w;
    rb[0] = S.gb.x; rb[1] = S.gb.y; rb[2] = S.gb.z; rb[3] = S.gb.w;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 2 * P.dt_dim; idx += kBlock) {
    const int which = idx / P.dt_dim;
    const int j = idx - which * P.dt_dim;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) sum += red[(w * 2 + which) * P.tvs + j];
    P.partial[(static_cast<int64_t>(blockIdx.x) * 2 + which) * P.dt_dim + j] = sum;
  }
}

// ---------------------------------------------------------------------------------
// Backward, two edges at a time, in the layout of the two-edge forward: the halves take
// alternate edges, each holds a whole K-space row in its 32 lanes. The destination's q~ and
// dxbar rows sit in LDS ([H][32 * NS + 1] chunks each, the last chunk zero), read per pair;
// dq~ accumulates per half in registers and the halves are added once per destination.
// Each lane owns at most one time chunk (ct <= 32) and accumulates its time gradients.
// Dynamic LDS: the time weights, then per wave the cos rows [2][tvs], the -sin rows
// [2][tvs], q~ and dxbar; then the workgroup's time-grad buffer [kWavesPerBlock][2][tvs].
// ---------------------------------------------------------------------------------
__host__ __device__ __forceinline__ int pair_row_chunks(int ns) { return ns * kHalf + 1; }

__host__ __device__ __forceinline__ int pair_bwd_wave_floats(int tvs, int heads, int ns) {
  return 4 * tvs + 2 * 4 * heads * pair_row_chunks(ns);
}

template <int H, int NS>
struct PairBwd {
  float4 dq[H][NS];
  float4 gw, gb;              // time-grad accumulators of this lane's time chunk
  float mh[H], il[H], T[H];   // row max, 1 / softmax denominator, dxbar . xbar
};

template <int H, int NS, bool BF, bool DN>
__device__ __forceinline__ void pair_bwd_step(const TgatParams& P, const PairCtx<NS>& L,
                                              const EdgeMeta<H, true>& M, int64_t c0, int p,
                                              int cnt, const float2* twb, float* tc, float* ts,
                                              const float4* qs, const float4* gs,
                                              const float4 (&xr)[NS], PairBwd<H, NS>& S) {
  constexpr int QS = NS * kHalf + 1;
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int j = 2 * p + half;
  const bool valid = j < cnt;
  const int jj = valid ? j : 0;
  float* rc = tc + half * P.tvs;
  float* rs = ts + half * P.tvs;
  const float t = pick_flt(M.t, jj);
  if (P.dt_dim > 0) {
    lds_sync();
    for (int d = hl; d < P.dt_dim; d += kHalf) {
      const float2 wb = twb[d];
      const float a = time_arg(t, wb.x, wb.y);
      float sv, cv;
      sincos_hw(a, sv, cv);
      if (fabsf(a) > trig::kMaxArg) sincosf(a, &sv, &cv);  // outside the reduction's range
      rc[d] = cv;
      rs[d] = -sv;
    }
    lds_sync();
  }
  float4 x[NS];
  pair_widen<NS, BF>(L, rc, xr, x);
  float dap[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float d = 0.f;
#pragma unroll
    for (int k = 0; k < NS; ++k) d += dot4(gs[h * QS + hl + k * kHalf], x[k]);
    dap[h] = half_sum(d);
  }
  // per-edge factors; an idle half (odd edge count) gets zeros and contributes nothing
  float ad[H], dz[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const float sc = pick_flt(M.sc[h], jj);
    const float dr = pick_flt(M.dr[h], jj);
    const float a = valid ? exp_fast(sc - S.mh[h]) * S.il[h] : 0.f;
    ad[h] = a * dr;
    const float gz = a * (dr * dap[h] - S.T[h]);
    dz[h] = gz * (sc > 0.f ? 1.f : P.slope);
#pragma unroll
    for (int k = 0; k < NS - 1; ++k) fma4(S.dq[h][k], dz[h], x[k]);
    fma4(S.dq[h][NS - 1], bias_dz(P, L.bias_lane, sc, dz[h]), x[NS - 1]);
  }
  // node-row gradient of this half's edge: dx = sum_h ad_h dxbar_h + dz_h q~_h
  if (DN && P.d_node) {
    float* drow = P.d_node + (c0 + jj) * P.ld_dnode;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      if (k * kHalf >= P.cn) continue;  // no node chunk in this slot (wave-uniform)
      float4 dx = f4_zero();
#pragma unroll
      for (int h = 0; h < H; ++h) {
        fma4(dx, ad[h], gs[h * QS + hl + k * kHalf]);
        fma4(dx, dz[h], qs[h * QS + hl + k * kHalf]);
      }
      if (valid && L.is_node[k]) *reinterpret_cast<float4*>(drow + 4 * (hl + k * kHalf)) = dx;
    }
  }
  // d cos(w t + b) = -sin(w t + b) * (t dw + db), on this lane's time chunk
  if (P.dt_dim > 0) {
    float4 dx = f4_zero();
#pragma unroll
    for (int h = 0; h < H; ++h) {
      fma4(dx, ad[h], gs[h * QS + L.tci]);
      fma4(dx, dz[h], qs[h * QS + L.tci]);
    }
    const float4 sn = *reinterpret_cast<const float4*>(rs + L.ttoff);
    const float4 pr = make_float4(sn.x * dx.x, sn.y * dx.y, sn.z * dx.z, sn.w * dx.w);
    S.gb.x += pr.x;
    S.gb.y += pr.y;
    S.gb.z += pr.z;
    S.gb.w += pr.w;
    fma4(S.gw, t, pr);
  }
}

__device__ __forceinline__ float4 pick_f4(const float4& v, int j) {
  return make_float4(pick_flt(v.x, j), pick_flt(v.y, j), pick_flt(v.z, j), pick_flt(v.w, j));
}

// Waves per SIMD the register budget is sized for (three leave 168 registers for the widest).
#ifndef FA_PAIR_BWD_WAVES
#define FA_PAIR_BWD_WAVES 3
#endif
#ifndef FA_PAIR_BWD_WAVES_NODN
#define FA_PAIR_BWD_WAVES_NODN 4
#endif
constexpr int pair_bwd_min_waves(int H, int NS, bool DN) {
  return H * NS >= 6 ? (DN ? FA_PAIR_BWD_WAVES : FA_PAIR_BWD_WAVES_NODN) : 4;
}

// DN: the node-row gradient is written (else P.d_node is null and its code is left out).
template <int H, int NS, bool BF, bool DN>
__global__ __launch_bounds__(kBlock, pair_bwd_min_waves(H, NS, DN)) void tgat_bwd_pair(TgatParams P) {
  constexpr int QS = NS * kHalf + 1;
  extern __shared__ float lds[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = lane_id();
  const int half = lane >= kHalf ? 1 : 0, hl = lane & (kHalf - 1);
  const int other = lane ^ kHalf;
  float2* twb = reinterpret_cast<float2*>(lds);
  float* tc = lds + pair_tile_base(P.dt_dim) + wave * pair_bwd_wave_floats(P.tvs, H, NS);
  float* ts = tc + 2 * P.tvs;
  float4* qs = reinterpret_cast<float4*>(ts + 2 * P.tvs);
  float4* gs = qs + H * QS;
  float* red = lds + pair_tile_base(P.dt_dim) + kWavesPerBlock * pair_bwd_wave_floats(P.tvs, H, NS);

  PairCtx<NS> L;
  setup_pair<NS>(P, L, NS * kHalf);
  stage_time_weights(P, twb);
  init_tiles(P, tc, 4, 2);
  // chunks past cp (and the extra zero chunk) stay zero
  for (int i = lane; i < 2 * H * QS; i += kWave) qs[i] = f4_zero();
  PairBwd<H, NS> S;
  S.gw = f4_zero();
  S.gb = f4_zero();

  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave; v < P.n_dst;
       v += total_waves) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int k = 0; k < NS; ++k) S.dq[h][k] = f4_zero();
    if (e1 <= e0) {
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float* dst = P.dqt + v * P.dqt_rs + h * P.dqt_hs;
#pragma unroll
        for (int k = 0; k < NS; ++k)
          if (half == 0 && L.live[k]) *reinterpret_cast<float4*>(dst + 4 * (hl + k * kHalf)) = f4_zero();
      }
      continue;
    }
    int64_t c0 = e0;
    int cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
    EdgeMeta<H, true> M;
    stage_meta<H, true>(P, c0, cnt, M);
    float4 xa[NS], xb[NS];
    pair_rows<NS, H, true, BF>(P, L, M, 0, cnt, xa);
    // the destination's rows: q~ (the chunks the backward reads, q_chunk_used) and dxbar
    // into LDS, T = dxbar . xbar per head
    lds_sync();  // the previous destination's reads of qs / gs are done
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const float4* qr = reinterpret_cast<const float4*>(P.qt + v * P.qt_rs + h * P.qt_hs);
      const float4* gr = reinterpret_cast<const float4*>(P.dxbar + v * P.dxbar_rs + h * P.dxbar_hs);
      float d = 0.f;
      if (P.tdot) {
        // every load of the two rows first, then the LDS writes
        constexpr int QR = (NS * kHalf + kWave - 1) / kWave;
        float4 qv[QR], gv[QR];
#pragma unroll
        for (int r = 0; r < QR; ++r) {
          const int c = lane + r * kWave;
          qv[r] = c < P.cp && q_chunk_used(P, c) ? load_nt(qr + c) : f4_zero();
          gv[r] = c < P.cp ? load_nt(gr + c) : f4_zero();
        }
#pragma unroll
        for (int r = 0; r < QR; ++r) {
          const int c = lane + r * kWave;
          if (c < P.cp) {
            qs[h * QS + c] = qv[r];
            gs[h * QS + c] = gv[r];
          }
        }
        S.T[h] = P.tdot[v * H + h];
      } else {
        const float4* xr = reinterpret_cast<const float4*>(P.xbar + v * P.xbar_rs + h * P.xbar_hs);
        for (int c = lane; c < P.cp; c += kWave) {
          const float4 g = gr[c];
          qs[h * QS + c] = q_chunk_used(P, c) ? qr[c] : f4_zero();
          gs[h * QS + c] = g;
          d += dot4(g, xr[c]);
        }
        S.T[h] = wave_sum(d);
      }
      S.mh[h] = P.stats[(v * H + h) * 2 + 0];
      S.il[h] = 1.f / P.stats[(v * H + h) * 2 + 1];
    }
    lds_sync();
    for (;;) {
      const int np = (cnt + 1) >> 1;
      // next pair's loads issued unconditionally (see the forward)
      for (int p = 0; p < np; p += 2) {
        pair_rows<NS, H, true, BF>(P, L, M, p + 1, cnt, xb);
        pair_bwd_step<H, NS, BF, DN>(P, L, M, c0, p, cnt, twb, tc, ts, qs, gs, xa, S);
        pair_rows<NS, H, true, BF>(P, L, M, p + 2, cnt, xa);
        if (p + 1 < np) pair_bwd_step<H, NS, BF, DN>(P, L, M, c0, p + 1, cnt, twb, tc, ts, qs, gs, xb, S);
      }
      c0 += kWave;
      if (c0 >= e1) break;
      cnt = static_cast<int>(e1 - c0 < kWave ? e1 - c0 : kWave);
      stage_meta<H, true>(P, c0, cnt, M);
      pair_rows<NS, H, true, BF>(P, L, M, 0, cnt, xa);
    }
    // dq~ = the two halves' sums
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float* dst = P.dqt + v * P.dqt_rs + h * P.dqt_hs;
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const float4 o = pick_f4(S.dq[h][k], other);
        const float4 a = S.dq[h][k];
        const float4 sum = make_float4(a.x + o.x, a.y + o.y, a.z + o.z, a.w + o.w);
        if (half == 0 && L.live[k]) store_nt(reinterpret_cast<float4*>(dst + 4 * (hl + k * kHalf)), sum);
      }
    }
  }

  // Time-grad partials of this workgroup: the halves added, then the waves in a fixed order.
  // Each time dim is owned by one lane of each half; lanes without a time chunk write zeros
  // to the zero chunk, which the sum below does not read.
  if (P.dt_dim <= 0) return;
  {
    const float4 ow = pick_f4(S.gw, other), ob = pick_f4(S.gb, other);
    if (half == 0) {
      float* rw = red + (wave * 2 + 0) * P.tvs + L.ttoff;
      float* rb = red + (wave * 2 + 1) * P.tvs + L.ttoff;
      rw[0] = S.gw.x + ow.x; rw[1] = S.gw.y + ow.y; rw[2] = S.gw.z + ow.z; rw[3] = S.gw.w + ow.w;
      rb[0] = S.gb.x + ob.x; rb[1] = S.gb.y + ob.y; rb[2] = S.gb.z + ob.z; rb[3] = S.gb.w + ob.w;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 2 * P.dt_dim; idx += kBlock) {
    const int which = idx / P.dt_dim;
    const int jd = idx - which * P.dt_dim;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) sum += red[(w * 2 + which) * P.tvs + jd];
    P.partial[(static_cast<int64_t>(blockIdx.x) * 2 + which) * P.dt_dim + jd] = sum;
  }
}

// ---------------------------------------------------------------------------------
// Head-split forward (4 or 8 heads): a workgroup takes one destination at a time; its four
// waves gather each batch of kHsBatch edges' K-space rows once, together, into LDS (row
// chunks by per-lane global loads, the time chunks evaluated in place, the bias chunk), and
// wave w scores and accumulates heads [w*HG, (w+1)*HG) from LDS with its q~ rows in
// registers. A lane owns chunks lane + 64k of a row (NS slots). Rows must be chunk loads
// (modes 0 and 1). Dynamic LDS: the time table [ct + 1][2] float4, then the batch rows
// [kHsBatch][64 NS] float4.
// ---------------------------------------------------------------------------------
constexpr int kHsBatch = 8;

// Read (never written) by gather tasks of non-row chunks and for missing rows; no table row
// chunk lies past 4 * 192 floats from its row start.
__device__ __align__(16) float kZeroRow[4 * 3 * kWave];

// Library cosine for arguments outside the fast reduction's range, kept out of line so
// that its registers do not count against the callers' main path.
__device__ __attribute__((noinline)) float cos_far(float a) { return cosf(a); }

// The time weights and phases by chunk into LDS, `twt` [ct + 1][2] (w chunk, b chunk; the
// last entry and the dims past dt_dim zero), for all waves of the workgroup.
__device__ __forceinline__ void stage_time_table(const TgatParams& P, float* twt) {
  const int n = 4 * (P.ct + 1);
  for (int d = threadIdx.x; d < n; d += blockDim.x) {
    const bool ok = d < P.dt_dim;
    twt[8 * (d >> 2) + (d & 3)] = ok ? P.time_w[d] : 0.f;
    twt[8 * (d >> 2) + 4 + (d & 3)] = ok ? P.time_b[d] : 0.f;
  }
  __syncthreads();
}

// Per-edge data of a batch, staged in LDS by one thread per edge: row ids (kNoRow when
// missing or out of range) and dt.
struct HsEdge {
  uint32_t nid, eid;
  float t;
};

__device__ __forceinline__ void hs_stage_edges(const TgatParams& P, int64_t c0, int nb, HsEdge* ed) {
  const int b = threadIdx.x;
  if (b < nb) {
    const int64_t e = c0 + b;
    const int64_t nr = P.node_idx ? P.node_idx[e] : e;
    const int64_t er = P.edge_idx ? P.edge_idx[e] : e;
    ed[b].nid = (nr >= 0 && nr < P.n_node) ? static_cast<uint32_t>(nr) : kNoRow;
    ed[b].eid = (er >= 0 && er < P.n_erow) ? static_cast<uint32_t>(er) : kNoRow;
    ed[b].t = P.dt_dim > 0 ? P.dt[e] : 0.f;
  }
}

// The batch's K-space rows into LDS: every thread first issues the row-chunk loads of all
// its tasks (chunk c of edge b; non-row chunks and missing rows read the static zero row),
// then completes them (bf16 widening, the row end of padded rows, the time cosines, the
// bias chunk) and stores them.
template <int RS>
__device__ __forceinline__ void hs_gather(const TgatParams& P, const float4* twt, const HsEdge* ed,
                                          int nb, float4* xs) {
  constexpr int G = (kHsBatch * RS + kBlock - 1) / kBlock;  // tasks per thread
  const char* zero = reinterpret_cast<const char*>(kZeroRow);
  const int tasks = nb * P.cp;
  float4 val[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i = threadIdx.x + g * kBlock;
    const int b = i < tasks ? i / P.cp : 0, c = i < tasks ? i - b * P.cp : P.cp;
    const char* ptr = zero;
    if (c < P.cn) {
      const uint32_t r = ed[b].nid;
      if (r != kNoRow) ptr = P.node_tab + static_cast<uint64_t>(r) * P.node_stride + (P.node_bf16 ? 8 : 16) * c;
    } else if (c < P.cn + P.ce) {
      const uint32_t r = ed[b].eid;
      if (r != kNoRow) ptr = P.edge_tab + static_cast<uint64_t>(r) * P.edge_stride + (P.edge_bf16 ? 8 : 16) * (c - P.cn);
    }
    const bool bf = c < P.cn ? P.node_bf16 : P.edge_bf16;
    if (bf) {
      const uint2 w = *reinterpret_cast<const uint2*>(ptr);
      val[g] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
    } else {
      val[g] = *reinterpret_cast<const float4*>(ptr);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i = threadIdx.x + g * kBlock;
    if (i >= tasks) continue;
    const int b = i / P.cp, c = i - b * P.cp;
    float4 v = val[g];
    if (c < P.cn) {
      if (P.node_tail == 1) v = keep_first(v, P.dn - 4 * c);
    } else if (c < P.cn + P.ce) {
      if (P.edge_tail == 1) v = keep_first(v, P.de - 4 * (c - P.cn));
    } else if (c < P.cn + P.ce + P.ct) {
      const int tj = c - P.cn - P.ce;
      const float t = ed[b].t;
      const float4 w = twt[2 * tj], bb = twt[2 * tj + 1];
      const float a[4] = {time_arg(t, w.x, bb.x), time_arg(t, w.y, bb.y), time_arg(t, w.z, bb.z),
                          time_arg(t, w.w, bb.w)};
      float cv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float sv;
        sincos_hw(a[q], sv, cv[q]);
        if (fabsf(a[q]) > trig::kMaxArg) cv[q] = cos_far(a[q]);  // outside the reduction's range
        if (4 * tj + q >= P.dt_dim) cv[q] = 0.f;
      }
      v = make_float4(cv[0], cv[1], cv[2], cv[3]);
    } else {
      v = c == P.cn + P.ce + P.ct ? make_float4(1.f, 0.f, 0.f, 0.f) : f4_zero();
    }
    xs[b * RS + c] = v;
  }
}

template <int H, int NS>
__global__ __launch_bounds__(kBlock) void tgat_fwd_hs(TgatParams P) {
  constexpr int HG = H / kWavesPerBlock;   // heads per wave
  constexpr int RS = NS * kWave;           // chunks per LDS row
  extern __shared__ float lds[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = lane_id();
  float4* twt = reinterpret_cast<float4*>(lds);
  float4* xs = twt + 2 * (P.ct + 1);
  HsEdge* ed = reinterpret_cast<HsEdge*>(xs + kHsBatch * RS);
  stage_time_table(P, lds);
  for (int i = threadIdx.x; i < kHsBatch * RS; i += kBlock) xs[i] = f4_zero();
  __syncthreads();

  for (int64_t v = blockIdx.x; v < P.n_dst; v += gridDim.x) {
    const int64_t e0 = clamp_edge(P.rowptr[v], P.n_edges);
    const int64_t e1 = clamp_edge(P.rowptr[v + 1], P.n_edges);
    float4 q[HG][NS], acc[HG][NS];
    float m[HG], l[HG];
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const int h = wave * HG + g;
      const rsrc_t rr = make_rsrc(P.qt + v * P.qt_rs + h * P.qt_hs, 4u * static_cast<uint32_t>(P.kp));
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        q[g][k] = bload4<kStream>(rr, 16u * static_cast<uint32_t>(lane + k * kWave));
        acc[g][k] = f4_zero();
      }
      m[g] = -INFINITY;
      l[g] = 0.f;
    }
    for (int64_t c0 = e0; c0 < e1; c0 += kHsBatch) {
      const int nb = static_cast<int>(e1 - c0 < kHsBatch ? e1 - c0 : kHsBatch);
      __syncthreads();  // the previous batch's reads are done
      hs_stage_edges(P, c0, nb, ed);
      __syncthreads();
      hs_gather<RS>(P, twt, ed, nb, xs);
      __syncthreads();
      for (int b = 0; b < nb; ++b) {
        const int64_t e = c0 + b;
        float4 x[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) x[k] = xs[b * RS + lane + k * kWave];
#pragma unroll
        for (int g = 0; g < HG; ++g) {
          const int h = wave * HG + g;
          const float s = leaky(wave_sum(row_dot<NS>(q[g], x)), P.slope);
          if (lane == 0) P.scores[e * H + h] = s;
          float dr = 1.f;
          if (P.drop) dr = P.drop[e * H + h];
          else if (P.drop_hash) dr = drop_mult(P.drop_seed, static_cast<uint64_t>(e * H + h), P.drop_p, P.drop_scale);
          if (s > m[g]) {  // wave-uniform
            const float r = exp_fast(m[g] - s);
            l[g] *= r;
#pragma unroll
            for (int k = 0; k < NS; ++k) scale4(acc[g][k], r);
            m[g] = s;
          }
          const float pe = exp_fast(s - m[g]);
          l[g] += pe;
#pragma unroll
          for (int k = 0; k < NS; ++k) fma4(acc[g][k], pe * dr, x[k]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const int h = wave * HG + g;
      const float inv = e1 > e0 ? 1.f / l[g] : 0.f;
      const rsrc_t rr = make_rsrc(P.xbar + v * P.xbar_rs + h * P.xbar_hs, 4u * static_cast<uint32_t>(P.kp));
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        scale4(acc[g][k], inv);
        bstore4<kStream>(rr, 16u * static_cast<uint32_t>(lane + k * kWave), acc[g][k]);
      }
      if (lane == 0) {
        P.stats[(v * H + h) * 2 + 0] = m[g];
        P.stats[(v * H + h) * 2 + 1] = l[g];
      }
    }
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

__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

template <typename T>
__global__ __launch_bounds__(kBlock) void gather_rows(const T* tab, int64_t ld_tab, int64_t n_tab,
                                                     const int64_t* idx, int64_t n, int dim,
                                                     float* out, int64_t ld_out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (r >= n) return;
  const int64_t src = idx ? idx[r] : r;
  const bool ok = src >= 0 && src < n_tab;
  for (int c = lane_id(); c < dim; c += kWave)
    out[r * ld_out + c] = ok ? to_float(tab[src * ld_tab + c]) : 0.f;
}

// Float32 rows whole chunks wide (aligned, dim and both row strides multiples of 4): a
// half-wave per row, float4 loads and stores.
__global__ __launch_bounds__(kBlock) void gather_rows4(const float* tab, int64_t ld_tab, int64_t n_tab,
                                                      const int64_t* idx, int64_t n, int dim,
                                                      float* out, int64_t ld_out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (2 * kWavesPerBlock) + threadIdx.x / kHalf;
  if (r >= n) return;
  const int64_t src = idx ? idx[r] : r;
  const bool ok = src >= 0 && src < n_tab;
  const float4* row = reinterpret_cast<const float4*>(tab + (ok ? src : 0) * ld_tab);
  float4* dst = reinterpret_cast<float4*>(out + r * ld_out);
  for (int c = threadIdx.x & (kHalf - 1); c < dim / 4; c += kHalf) dst[c] = ok ? row[c] : f4_zero();
}

// ---------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------
int fill_params(const fa_tgat_graph* g, int heads, const float* qt, int64_t qt_rs, int64_t qt_hs,
                float slope,
                const float* drop, uint64_t drop_seed, float drop_p, TgatParams& P) {
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
  if ((g->node_dtype != FA_F32 && g->node_dtype != FA_BF16) ||
      (g->edge_dtype != FA_F32 && g->edge_dtype != FA_BF16))
    return FA_EINVAL;
  P.node_tab = static_cast<const char*>(g->node_tab); P.ld_node = g->ld_node;
  P.n_node = g->dn > 0 ? g->n_node : 0;
  P.dn = g->dn; P.node_idx = g->node_idx;
  P.edge_tab = static_cast<const char*>(g->edge_tab); P.ld_edge = g->ld_edge;
  P.n_erow = g->de > 0 ? g->n_edge_rows : 0;
  P.de = g->de; P.edge_idx = g->edge_idx;
  //   // Row chunks are read whole when every row start is chunk-aligned (16 bytes for float32,
  // 8 for bf16), else element by element.
  P.node_bf16 = g->node_dtype == FA_BF16;
  P.edge_bf16 = g->edge_dtype == FA_BF16;
  const uintptr_t nmask = P.node_bf16 ? 7u : 15u, emask = P.edge_bf16 ? 7u : 15u;
  const bool nal = !(g->ld_node & 3) && !(reinterpret_cast<uintptr_t>(g->node_tab) & nmask);
  const bool eal = !(g->ld_edge & 3) && !(reinterpret_cast<uintptr_t>(g->edge_tab) & emask);
  P.node_tail = g->dn <= 0 ? 0 : (!nal ? 2 : ((g->dn & 3) ? 1 : 0));
  P.edge_tail = g->de <= 0 ? 0 : (!eal ? 2 : ((g->de & 3) ? 1 : 0));
  const int64_t nes = P.node_bf16 ? 2 : 4, ees = P.edge_bf16 ? 2 : 4;
  // mode 1 reads up to the padded width (ld rounded down to whole chunks >= dn)
  P.node_stride = static_cast<uint64_t>(nes * g->ld_node);
  P.edge_stride = static_cast<uint64_t>(ees * g->ld_edge);
  P.node_row_bytes = static_cast<uint32_t>(nes * (P.node_tail == 1 ? round_up(g->dn, 4) : g->dn));
  P.edge_row_bytes = static_cast<uint32_t>(ees * (P.edge_tail == 1 ? round_up(g->de, 4) : g->de));
  P.dnode_dwords = (g->dn & 3) != 0;
  if (g->n_edges > 0 && ((g->dn > 0 && g->n_node <= 0) || (g->de > 0 && g->n_edge_rows <= 0)))
    return FA_EINVAL;
  // row ids travel as 32 bits (kNoRow marks a missing row)
  if (g->n_node >= static_cast<int64_t>(kNoRow) || g->n_edge_rows >= static_cast<int64_t>(kNoRow))
    return FA_EUNSUPPORTED;
  P.dt = g->dt; P.time_w = g->time_w; P.time_b = g->time_b; P.dt_dim = g->dt_dim;
  P.cn = static_cast<int>(ceil_div(g->dn, 4));
  P.ce = static_cast<int>(ceil_div(g->de, 4));
  P.ct = static_cast<int>(ceil_div(g->dt_dim, 4));
  P.cp = P.cn + P.ce + P.ct + 1;
  P.tvs = 4 * (P.ct + 2);
  P.kp = 4 * static_cast<int64_t>(P.cp);
  P.qt = qt; P.qt_rs = qt_rs; P.qt_hs = qt_hs; P.slope = slope; P.drop = drop;
  if (!(drop_p >= 0.f && drop_p < 1.f)) return FA_EINVAL;
  P.drop_seed = drop_seed;
  P.drop_p = drop_p;
  P.drop_scale = static_cast<float>(1.0 / (1.0 - static_cast<double>(drop_p)));
  P.drop_hash = (drop == nullptr && drop_p > 0.f) ? 1 : 0;
  if (!aligned16(qt) || (qt_rs & 3) || (qt_hs & 3)) return FA_EALIGN;
  if (qt_rs < 0 || qt_hs < 0) return FA_EINVAL;  // an input block may repeat (stride 0)
  return FA_OK;
}

// An output block: 16-byte aligned, strides multiples of 4, and no two (destination, head)
// rows overlap, i.e. destination-major ([n_dst][heads][Kp]-like) or head-major
// ([heads][n_dst][Kp]-like).
int check_out_rows(const void* p, int64_t rs, int64_t hs, int64_t kp, int heads, int64_t n_dst) {
  if (!aligned16(p) || (rs & 3) || (hs & 3)) return FA_EALIGN;
  const bool dst_major = rs >= kp && (heads == 1 || (hs >= kp && rs >= hs * heads));
  const bool head_major = hs >= kp && rs >= kp && hs >= rs * n_dst;
  return dst_major || head_major ? FA_OK : FA_EINVAL;
}

// An input block read alongside the outputs: aligned, non-negative strides.
int check_in_rows(const void* p, int64_t rs, int64_t hs) {
  if (!aligned16(p) || (rs & 3) || (hs & 3)) return FA_EALIGN;
  return rs < 0 || hs < 0 ? FA_EINVAL : FA_OK;
}

size_t fwd_lds_bytes(const TgatParams& P) {
  return sizeof(float) * static_cast<size_t>(kWavesPerBlock) * kBatch * P.tvs;
}

size_t bwd_lds_bytes(const TgatParams& P) {
  return sizeof(float) * static_cast<size_t>(kWavesPerBlock) * (2 * kBatch + 2) * P.tvs;
}

// Workgroups of a grid-stride launch over n_dst destinations (4 per workgroup pass).
int stride_grid(int64_t n_dst) {
  const int64_t want = ceil_div(n_dst, kWavesPerBlock);
  return static_cast<int>(want < kMaxBlocks ? (want < 1 ? 1 : want) : kMaxBlocks);
}

// Persistent launch: at most the resident workgroups, so every workgroup runs in the first
// (and only) round.
int persistent_grid(int64_t n_dst, const void* kernel, size_t lds) {
  const int want = stride_grid(n_dst);
  const int res = resident_blocks(kernel, lds);
  return want < res ? want : res;
}

// The pair kernels read both tables with one element type (a template parameter): a table
// without columns takes the other's.
bool pair_one_type(const TgatParams& P) { return P.dn == 0 || P.de == 0 || P.node_bf16 == P.edge_bf16; }
bool pair_bf16(const TgatParams& P) { return P.dn > 0 ? P.node_bf16 : P.edge_bf16; }

// The two-edge forward: whole-chunk rows (mode 0), up to 2 heads, up to 128 chunks for one
// head and 96 for two (beyond that its registers spill).
bool pair_fwd_fits(const TgatParams& P, int heads) {
  return heads <= 2 && P.node_tail == 0 && P.edge_tail == 0 && pair_one_type(P) &&
         P.cp <= (heads == 1 ? 4 : 3) * kHalf;
}

size_t pair_lds_bytes(const TgatParams& P, int heads) {
  return sizeof(float) * (static_cast<size_t>(pair_tile_base(P.dt_dim)) +
                          static_cast<size_t>(kWavesPerBlock) *
                              pair_wave_floats(P.tvs, heads, static_cast<int>(ceil_div(P.cp, kHalf))));
}

// The head-split forward: 4 or 8 heads, chunk loads (modes 0 and 1), at most 32 time chunks
// (the time table) and 192 chunks.
bool hs_fwd_fits(const TgatParams& P, int heads) {
  return (heads == 4 || heads == 8) && P.node_tail != 2 && P.edge_tail != 2 && P.ct <= 64 &&
         P.cp <= 3 * kWave;
}

size_t hs_lds_bytes(const TgatParams& P) {
  return sizeof(float4) * (2 * static_cast<size_t>(P.ct + 1) +
                           static_cast<size_t>(kHsBatch) * kWave * ceil_div(P.cp, kWave)) +
         sizeof(HsEdge) * kHsBatch;
}

template <int H>
int launch_fwd_h(const TgatParams& P, hipStream_t stream) {
  const int ns = static_cast<int>(ceil_div(P.cp, kWave));
  size_t lds = fwd_lds_bytes(P);
  void (*k)(TgatParams) = nullptr;
  if constexpr (H == 4 || H == 8) if (hs_fwd_fits(P, H)) {
    lds = hs_lds_bytes(P);
    switch (ns) {
      case 1: k = tgat_fwd_hs<H, 1>; break;
      case 2: k = tgat_fwd_hs<H, 2>; break;
      default: k = tgat_fwd_hs<H, 3>; break;
    }
    const void* kp = reinterpret_cast<const void*>(k);
    const int64_t res = resident_blocks(kp, lds);
    const dim3 grid(static_cast<unsigned>(P.n_dst < res ? (P.n_dst < 1 ? 1 : P.n_dst) : res));
    hipLaunchKernelGGL(k, grid, dim3(kBlock), lds, stream, P);
    return launch_status();
  }
  if constexpr (H <= 2) if (pair_fwd_fits(P, H)) {
    lds = pair_lds_bytes(P, H);
    const bool bf = pair_bf16(P);
    switch (ceil_div(P.cp, kHalf)) {
      case 1: k = bf ? tgat_fwd_pair<H, 1, true> : tgat_fwd_pair<H, 1, false>; break;
      case 2: k = bf ? tgat_fwd_pair<H, 2, true> : tgat_fwd_pair<H, 2, false>; break;
      case 3: k = bf ? tgat_fwd_pair<H, 3, true> : tgat_fwd_pair<H, 3, false>; break;
      default: k = bf ? tgat_fwd_pair<H, (H == 1 ? 4 : 3), true> : tgat_fwd_pair<H, (H == 1 ? 4 : 3), false>; break;
    }
    const dim3 grid(static_cast<unsigned>(persistent_grid(P.n_dst, reinterpret_cast<const void*>(k), lds)));
    hipLaunchKernelGGL(k, grid, dim3(kBlock), lds, stream, P);
    return launch_status();
  }
  switch (ns) {
    case 1: k = tgat_fwd<H, 1>; break;
    case 2: k = tgat_fwd<H, 2>; break;
    case 3: k = tgat_fwd<H, 3>; break;
    case 4: k = tgat_fwd<H, 4>; break;
    default: return FA_EUNSUPPORTED;
  }
  const dim3 grid(static_cast<unsigned>(persistent_grid(P.n_dst, reinterpret_cast<const void*>(k), lds)));
  hipLaunchKernelGGL(k, grid, dim3(kBlock), lds, stream, P);
  return launch_status();
}

constexpr size_t kMaxLds = 64 * 1024;  // dynamic LDS per workgroup used by the fused kernels

// The two-edge backward: the forward's conditions, at most 96 chunks, at most 32 time
// chunks (one per lane), and 16-byte node-gradient rows.
bool pair_bwd_fits(const TgatParams& P, int heads) {
  return pair_fwd_fits(P, heads) && P.cp <= 3 * kHalf && P.ct <= kHalf &&
         (!P.d_node || !P.dnode_dwords);
}

size_t pair_bwd_lds_bytes(const TgatParams& P, int heads) {
  const int ns = static_cast<int>(ceil_div(P.cp, kHalf));
  return sizeof(float) * (static_cast<size_t>(pair_tile_base(P.dt_dim)) +
                          static_cast<size_t>(kWavesPerBlock) * pair_bwd_wave_floats(P.tvs, heads, ns) +
                          static_cast<size_t>(kWavesPerBlock) * 2 * P.tvs);
}

int bwd_grid(int64_t n_dst) { return stride_grid(n_dst); }

template <int H, int NS>
auto pair_bwd_kernel(const TgatParams& P) -> void (*)(TgatParams) {
  if (P.d_node) return pair_bf16(P) ? tgat_bwd_pair<H, NS, true, true> : tgat_bwd_pair<H, NS, false, true>;
  return pair_bf16(P) ? tgat_bwd_pair<H, NS, true, false> : tgat_bwd_pair<H, NS, false, false>;
}

// `grid` returns the workgroups launched (rows of the time-gradient partials).
template <int H>
int launch_bwd_h(const TgatParams& P, int& grid, hipStream_t stream) {
  const int ns = static_cast<int>(ceil_div(P.cp, kWave));
  size_t lds = bwd_lds_bytes(P);
  void (*k)(TgatParams) = nullptr;
  switch (ns) {
    case 1: k = tgat_bwd<H, 1>; break;
    case 2: k = tgat_bwd<H, 2>; break;
    case 3: k = tgat_bwd<H, 3>; break;
    case 4: k = tgat_bwd<H, 4>; break;
    default: return FA_EUNSUPPORTED;
  }
  if constexpr (H <= 2) if (pair_bwd_fits(P, H)) {
    const int pns = static_cast<int>(ceil_div(P.cp, kHalf));
    lds = pair_bwd_lds_bytes(P, H);
    switch (pns) {
      case 1: k = pair_bwd_kernel<H, 1>(P); break;
      case 2: k = pair_bwd_kernel<H, 2>(P); break;
      default: k = pair_bwd_kernel<H, 3>(P); break;
    }
  }
  grid = persistent_grid(P.n_dst, reinterpret_cast<const void*>(k), lds);
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(kBlock), lds, stream, P);
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
                                    int64_t qt_rs, int64_t qt_hs, float slope, const float* drop,
                                    uint64_t drop_seed, float drop_p, float* xbar,
                                    int64_t xbar_rs, int64_t xbar_hs, float* scores, float* stats,
                                    hipStream_t stream) {
  TgatParams P;
  int st = fill_params(g, heads, qt, qt_rs, qt_hs, slope, drop, drop_seed, drop_p, P);
  if (st != FA_OK) return st;
  if (P.n_dst == 0) return FA_OK;
  if (fwd_lds_bytes(P) > kMaxLds) return FA_EUNSUPPORTED;
  if (!xbar || !stats || (P.n_edges > 0 && !scores)) return FA_EINVAL;
  st = check_out_rows(xbar, xbar_rs, xbar_hs, P.kp, heads, P.n_dst);
  if (st != FA_OK) return st;
  P.xbar = xbar; P.xbar_rs = xbar_rs; P.xbar_hs = xbar_hs; P.scores = scores; P.stats = stats;
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

// ---------------------------------------------------------------------------------
// The backward without allocation: its time-gradient partials live in `scratch`, a static
// device array (one copy per GPU, held until the process ends). Every workgroup the backward
// launches writes its whole partial row before the reduction reads it, so nothing has to be
// cleared between calls. Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------------
// Rows for the largest grid (kMaxBlocks workgroups) at the widest time encoding the backward
// takes (256): 4 MiB.
constexpr size_t kNoAllocScratchFloats = static_cast<size_t>(kMaxBlocks) * 2 * 256;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of the current device's copy of `scratch`, looked up once per device
// (the array's name is a host-side stand-in and must never reach a kernel).
static int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return FA_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return FA_ESCRATCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FA_OK;
}

// The backward behind both entry points: `partial` is the caller's time-gradient scratch;
// with `lib_scratch` the library's static array is used instead, looked up after every
// argument check.
static int tgat_bwd_impl(bool lib_scratch, const fa_tgat_graph* g, int32_t heads, const float* qt,
                         int64_t qt_rs, int64_t qt_hs, float slope, const float* drop, uint64_t drop_seed,
                         float drop_p, const float* xbar, int64_t xbar_rs, int64_t xbar_hs,
                         const float* tdot, const float* scores, const float* stats,
                         const float* dxbar, int64_t dxbar_rs, int64_t dxbar_hs, float* dqt,
                         int64_t dqt_rs, int64_t dqt_hs, float* d_node, int64_t ld_dnode,
                         float* d_time_w, float* d_time_b, void* partial, size_t partial_bytes,
                         hipStream_t stream) {
  TgatParams P;
  int st = fill_params(g, heads, qt, qt_rs, qt_hs, slope, drop, drop_seed, drop_p, P);
  if (st != FA_OK) return st;
  if (P.n_dst == 0) {
    if (P.dt_dim > 0 && d_time_w && d_time_b) {
      hipLaunchKernelGGL(fill_zero, dim3(1), dim3(kBlock), 0, stream, d_time_w, P.dt_dim);
      hipLaunchKernelGGL(fill_zero, dim3(1), dim3(kBlock), 0, stream, d_time_b, P.dt_dim);
    }
    return launch_status();
  }
  if (bwd_lds_bytes(P) > kMaxLds || P.ct > kWave) return FA_EUNSUPPORTED;
  if ((!xbar && !tdot) || !dxbar || !dqt || !stats || (P.n_edges > 0 && !scores)) return FA_EINVAL;
  if (!tdot && (st = check_in_rows(xbar, xbar_rs, xbar_hs)) != FA_OK) return st;
  if ((st = check_in_rows(dxbar, dxbar_rs, dxbar_hs)) != FA_OK) return st;
  if ((st = check_out_rows(dqt, dqt_rs, dqt_hs, P.kp, heads, P.n_dst)) != FA_OK) return st;
  if (d_node && (P.dn <= 0 || ld_dnode < P.dn)) return FA_EINVAL;
  if (d_node && P.node_bf16) return FA_EUNSUPPORTED;  // node gradients for float32 rows only
  if (P.dt_dim > 0 && (!d_time_w || !d_time_b)) return FA_EINVAL;
  int grid = bwd_grid(P.n_dst);   // the most workgroups a launch uses (scratch rows)
  if (lib_scratch && (st = noalloc_scratch(&partial)) != FA_OK) return st;
  if (P.dt_dim > 0 && (!partial || partial_bytes < fa_tgat_attn_bwd_scratch_bytes(P.n_dst, P.dt_dim)))
    return FA_ESCRATCH;
  P.xbar = const_cast<float*>(xbar); P.xbar_rs = xbar_rs; P.xbar_hs = xbar_hs; P.tdot = tdot;
  P.dxbar = dxbar; P.dxbar_rs = dxbar_rs; P.dxbar_hs = dxbar_hs;
  P.dqt = dqt; P.dqt_rs = dqt_rs; P.dqt_hs = dqt_hs;
  P.d_node = d_node; P.ld_dnode = ld_dnode; P.scores = const_cast<float*>(scores);
  // 16-byte node-gradient stores need 16-byte aligned gradient rows as well
  if (d_node && (!aligned16(d_node) || (ld_dnode & 3))) P.dnode_dwords = 1;
  P.stats = const_cast<float*>(stats); P.partial = static_cast<float*>(partial);
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

extern "C" int fa_tgat_attn_bwd_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                                    int64_t qt_rs, int64_t qt_hs, float slope, const float* drop,
                                    uint64_t drop_seed, float drop_p, const float* xbar,
                                    int64_t xbar_rs, int64_t xbar_hs, const float* tdot,
                                    const float* scores,
                                    const float* stats, const float* dxbar, int64_t dxbar_rs,
                                    int64_t dxbar_hs, float* dqt, int64_t dqt_rs, int64_t dqt_hs,
                                    float* d_node, int64_t ld_dnode,
                                    float* d_time_w, float* d_time_b, void* scratch,
                                    size_t scratch_bytes, hipStream_t stream) {
  return tgat_bwd_impl(false, g, heads, qt, qt_rs, qt_hs, slope, drop, drop_seed, drop_p, xbar,
                       xbar_rs, xbar_hs, tdot, scores, stats, dxbar, dxbar_rs, dxbar_hs, dqt,
                       dqt_rs, dqt_hs, d_node, ld_dnode, d_time_w, d_time_b, scratch,
                       scratch_bytes, stream);
}

extern "C" int fa_tgat_attn_bwd_noalloc_f32(const fa_tgat_graph* g, int32_t heads, const float* qt,
                                            int64_t qt_rs, int64_t qt_hs, float slope,
                                            const float* drop, uint64_t drop_seed, float drop_p,
                                            const float* xbar, int64_t xbar_rs, int64_t xbar_hs,
                                            const float* tdot, const float* scores,
                                            const float* stats, const float* dxbar,
                                            int64_t dxbar_rs, int64_t dxbar_hs, float* dqt,
                                            int64_t dqt_rs, int64_t dqt_hs, float* d_node,
                                            int64_t ld_dnode, float* d_time_w, float* d_time_b,
                                            hipStream_t stream) {
  // a shape whose partials exceed the array is refused (FA_ESCRATCH) by the size check in
  // tgat_bwd_impl, before any launch
  return tgat_bwd_impl(true, g, heads, qt, qt_rs, qt_hs, slope, drop, drop_seed, drop_p, xbar,
                       xbar_rs, xbar_hs, tdot, scores, stats, dxbar, dxbar_rs, dxbar_hs, dqt,
                       dqt_rs, dqt_hs, d_node, ld_dnode, d_time_w, d_time_b, nullptr,
                       sizeof(scratch), stream);
}

__global__ __launch_bounds__(kBlock) void dropout_mask(uint64_t seed, float p, float scale,
                                                      int64_t n, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n) out[i] = drop_mult(seed, static_cast<uint64_t>(i), p, scale);
}

extern "C" int fa_dropout_mask_f32(uint64_t seed, float p, int64_t n, float* out,
                                   hipStream_t stream) {
  if (n < 0 || !(p >= 0.f && p < 1.f)) return FA_EINVAL;
  if (n == 0) return FA_OK;
  if (!out) return FA_EINVAL;
  const float scale = static_cast<float>(1.0 / (1.0 - static_cast<double>(p)));
  hipLaunchKernelGGL(dropout_mask, dim3(static_cast<unsigned>(ceil_div(n, kBlock))), dim3(kBlock), 0,
                     stream, seed, p, scale, n, out);
  return launch_status();
}

template <typename T>
int gather_rows_launch(const T* tab, int64_t ld_tab, int64_t n_tab, const int64_t* idx, int64_t n,
                       int32_t dim, float* out, int64_t ld_out, hipStream_t stream) {
  if (n < 0 || dim < 0 || n_tab < 0) return FA_EINVAL;
  if (n == 0 || dim == 0) return FA_OK;
  if (!tab || !out || ld_tab < dim || ld_out < dim) return FA_EINVAL;
  if constexpr (std::is_same<T, float>::value) {
    if (aligned16(tab) && aligned16(out) && !(dim & 3) && !(ld_tab & 3) && !(ld_out & 3)) {
      hipLaunchKernelGGL(gather_rows4, dim3(static_cast<unsigned>(ceil_div(n, 2 * kWavesPerBlock))),
                         dim3(kBlock), 0, stream, tab, ld_tab, n_tab, idx, n, dim, out, ld_out);
      return launch_status();
    }
  }
  hipLaunchKernelGGL(gather_rows<T>, dim3(static_cast<unsigned>(ceil_div(n, kWavesPerBlock))), dim3(kBlock),
                     0, stream, tab, ld_tab, n_tab, idx, n, dim, out, ld_out);
  return launch_status();
}

extern "C" int fa_gather_rows_f32(const float* tab, int64_t ld_tab, int64_t n_tab,
                                  const int64_t* idx, int64_t n, int32_t dim, float* out,
                                  int64_t ld_out, hipStream_t stream) {
  return gather_rows_launch(tab, ld_tab, n_tab, idx, n, dim, out, ld_out, stream);
}

extern "C" int fa_gather_rows_bf16_f32(const uint16_t* tab, int64_t ld_tab, int64_t n_tab,
                                       const int64_t* idx, int64_t n, int32_t dim, float* out,
                                       int64_t ld_out, hipStream_t stream) {
  return gather_rows_launch(tab, ld_tab, n_tab, idx, n, dim, out, ld_out, stream);
}
