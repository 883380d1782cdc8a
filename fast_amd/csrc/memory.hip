// TGN node-memory path on gfx950 (reference memorys.py:6-304):
//   mail gather   the updater inputs of every source row gathered by node id
//                 (MailBox.prep_input_mails, memorys.py:57-71), the mails written straight
//                 into the rows of the recurrent cell's input;
//   time rows     cos(w (ts - mem_ts) + b) into those rows' time columns
//                 (GRUMemeoryUpdater.forward, memorys.py:288-290);
//   cell gates    the elementwise part of torch.nn.GRUCell / RNNCell (memorys.py:291, 332)
//                 forward and backward; the two input products stay library GEMMs;
//   time grad     dw, db of the time encoder: per-workgroup partial sums over row chunks,
//                 then a fixed-order sum of the partials (deterministic);
//   write-back    MailBox.update_memory / update_mailbox for deliver_to = 'self',
//                 mail_combine = 'last' (memorys.py:84-139): one winner per node id, the
//                 row that comes last in the reference's order. A 64-bit atomic max of
//                 (generation << 32 | row) per node picks it; the winner alone writes, so
//                 the result does not depend on scheduling. The generation grows with
//                 every call, so the per-node tags never need clearing.
//
// Rows are handled one wave per row (copies, 16-byte chunks where everything is aligned)
// or one thread per element (gates, time columns); every grid is grid-stride.
#include <hip/hip_runtime.h>

#include "fa_common.hpp"
#include "fastagg.h"

namespace fa {
namespace {

constexpr int kRowBlock = 256;                 // 4 waves
constexpr int kRowWaves = kRowBlock / kWave;
constexpr int kMaxRowBlocks = 8192;
constexpr int kEltBlock = 256;
constexpr int kMaxEltBlocks = 16384;

__device__ __forceinline__ int64_t load_id(const void* ids, int id64, int64_t i) {
  return id64 ? static_cast<const int64_t*>(ids)[i]
              : static_cast<int64_t>(static_cast<const int32_t*>(ids)[i]);
}

// dst[0, w) = valid ? src[0, w) : 0 by one wave (lane-strided, 16-byte chunks when V4);
// `valid` is the same in every lane, and src is not read when it is false.
template <bool V4>
__device__ __forceinline__ void wave_copy(const float* src, float* dst, int64_t w, bool valid,
                                          int lane) {
  if constexpr (V4) {
    const int64_t w4 = w >> 2;
    if (valid) {
      for (int64_t c = lane; c < w4; c += kWave)
        reinterpret_cast<float4*>(dst)[c] = reinterpret_cast<const float4*>(src)[c];
    } else {
      for (int64_t c = lane; c < w4; c += kWave) reinterpret_cast<float4*>(dst)[c] = f4_zero();
    }
  } else {
    if (valid) {
      for (int64_t c = lane; c < w; c += kWave) dst[c] = src[c];
    } else {
      for (int64_t c = lane; c < w; c += kWave) dst[c] = 0.f;
    }
  }
}

__device__ __forceinline__ float cos_time(float t, float w, float b) {
  const float a = time_arg(t, w, b);
  if (fabsf(a) > trig::kMaxArg) return cosf(a);  // outside the reduction's range
  float s, c;
  sincos_hw(a, s, c);
  return c;
}

__device__ __forceinline__ float sin_time(float t, float w, float b) {
  const float a = time_arg(t, w, b);
  if (fabsf(a) > trig::kMaxArg) return sinf(a);
  float s, c;
  sincos_hw(a, s, c);
  return s;
}

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

int row_grid(int64_t rows) {
  const int64_t b = (rows + kRowWaves - 1) / kRowWaves;
  return static_cast<int>(b < 1 ? 1 : (b > kMaxRowBlocks ? kMaxRowBlocks : b));
}

int elt_grid(int64_t n) {
  const int64_t b = (n + kEltBlock - 1) / kEltBlock;
  return static_cast<int>(b < 1 ? 1 : (b > kMaxEltBlocks ? kMaxEltBlocks : b));
}

bool al16(const void* p) { return p == nullptr || aligned16(p); }

// ---------------------------------------------------------------------------------
// Mail gather
// ---------------------------------------------------------------------------------
struct MailGatherParams {
  const void* ids;
  int id64;
  int64_t n, num_nodes;
  const float* memory;      // [num_nodes][ld_mem], m used
  int64_t ld_mem;
  int32_t m;
  const float* memory_ts;   // [num_nodes]
  const float* mailbox;     // [num_nodes][ld_mail], mail_w used
  int64_t ld_mail, mail_w;
  const float* mailbox_ts;  // [num_nodes][slots]
  int32_t slots;
  float* mem_out;           // [n][ld_mem_out]
  int64_t ld_mem_out;
  float* mem_ts_out;        // [n]
  float* x_out;             // [n][ldx], columns [0, mail_w)
  int64_t ldx;
  float* mail_ts_out;       // [n][slots]
};

template <bool V4>
__global__ __launch_bounds__(kRowBlock) void mail_gather(MailGatherParams P) {
  const int lane = lane_id();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kRowWaves;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave; i < P.n;
       i += waves) {
    const int64_t id = load_id(P.ids, P.id64, i);
    const bool ok = id >= 0 && id < P.num_nodes;
    const int64_t row = ok ? id : 0;
    wave_copy<V4>(P.memory + row * P.ld_mem, P.mem_out + i * P.ld_mem_out, P.m, ok, lane);
    wave_copy<V4>(P.mailbox + row * P.ld_mail, P.x_out + i * P.ldx, P.mail_w, ok, lane);
    if (ok) {
      for (int s = lane; s < P.slots; s += kWave)
        P.mail_ts_out[i * P.slots + s] = P.mailbox_ts[row * P.slots + s];
      if (lane == 0) P.mem_ts_out[i] = P.memory_ts[row];
    } else {
      for (int s = lane; s < P.slots; s += kWave) P.mail_ts_out[i * P.slots + s] = 0.f;
      if (lane == 0) P.mem_ts_out[i] = 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------
// Time columns and their gradient
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(kEltBlock) void time_rows(const float* ts, const float* mem_ts,
                                                       int64_t n, const float* w, const float* b,
                                                       int32_t dt, float* out, int64_t ld) {
  const int64_t total = n * dt;
  if (total <= 0xffffffffLL) {   // 32-bit index arithmetic (no 64-bit division per element)
    const uint32_t tot = static_cast<uint32_t>(total), d = static_cast<uint32_t>(dt);
    const uint32_t stride = gridDim.x * kEltBlock;
    for (uint32_t idx = blockIdx.x * kEltBlock + threadIdx.x; idx < tot; idx += stride) {
      const uint32_t i = idx / d;
      const uint32_t j = idx - i * d;
      const float t = mem_ts ? ts[i] - mem_ts[i] : ts[i];
      out[static_cast<int64_t>(i) * ld + j] = cos_time(t, w[j], b[j]);
      if (idx > tot - stride) break;   // the next index would wrap past 2^32
    }
    return;
  }
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kEltBlock + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kEltBlock) {
    const int64_t i = idx / dt;
    const int j = static_cast<int>(idx - i * dt);
    const float t = mem_ts ? ts[i] - mem_ts[i] : ts[i];
    out[i * ld + j] = cos_time(t, w[j], b[j]);
  }
}

// Row-chunk kernels: workgroup b owns rows [b*per, min(n, (b+1)*per)); its 256 threads are
// 128 column lanes x 2 row phases (phase p takes rows r0 + p, r0 + p + 2, ...), so each
// row's columns are read and written contiguously. Column sums are kept per thread in row
// order, the two phases added in a fixed order through LDS, and the workgroups' partials
// summed by col_finish in a fixed order: the sums do not depend on scheduling.
constexpr int kColLanes = 128;
constexpr int kRowPhases = 2;
constexpr int kColBlock = kColLanes * kRowPhases;
constexpr int kMaxChunkBlocks = 4096;
constexpr int kMinChunkRows = 64;

int chunk_blocks(int64_t n) {
  const int64_t b = (n + kMinChunkRows - 1) / kMinChunkRows;
  return static_cast<int>(b < 1 ? 1 : (b > kMaxChunkBlocks ? kMaxChunkBlocks : b));
}

struct RowChunk {
  int64_t r0, r1;
  int lane, phase;
};

__device__ __forceinline__ RowChunk row_chunk(int64_t n) {
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  RowChunk c;
  c.r0 = static_cast<int64_t>(blockIdx.x) * per;
  c.r1 = c.r0 + per < n ? c.r0 + per : n;
  c.lane = threadIdx.x % kColLanes;
  c.phase = threadIdx.x / kColLanes;
  return c;
}

// out[b][col] = sum of the two phases' values v (phase 0 first); every thread of the
// workgroup calls it with the same col0 (the column chunk), lanes past `cols` pass 0.
template <int K>
__device__ __forceinline__ void phase_sums(const float (&v)[K], const RowChunk& c, int64_t col,
                                           int64_t cols, int64_t stride, float* out) {
  __shared__ float red[kRowPhases][K][kColLanes];
#pragma unroll
  for (int k = 0; k < K; ++k) red[c.phase][k][c.lane] = v[k];
  __syncthreads();
  if (c.phase == 0 && col < cols) {
#pragma unroll
    for (int k = 0; k < K; ++k) out[k * stride + col] = red[0][k][c.lane] + red[1][k][c.lane];
  }
  __syncthreads();
}

// partial[blk][0][j] = sum over the workgroup's rows of -sin(a_ij) t_i g_ij, [1][j] the same
// without t_i.
__global__ __launch_bounds__(kColBlock) void time_rows_grad(
    const float* ts, const float* mem_ts, int64_t n, const float* w, const float* b, int32_t dt,
    const float* g, int64_t ldg, float* partial) {
  const RowChunk c = row_chunk(n);
  float* out = partial + static_cast<int64_t>(blockIdx.x) * 2 * dt;
  for (int j0 = 0; j0 < dt; j0 += kColLanes) {
    const int j = j0 + c.lane;
    float v[2] = {0.f, 0.f};
    if (j < dt) {
      const float wj = w[j], bj = b[j];
      for (int64_t i = c.r0 + c.phase; i < c.r1; i += kRowPhases) {
        const float t = mem_ts ? ts[i] - mem_ts[i] : ts[i];
        const float d = -sin_time(t, wj, bj) * g[i * ldg + j];
        v[0] = fmaf(d, t, v[0]);
        v[1] += d;
      }
    }
    phase_sums<2>(v, c, j, dt, dt, out);
  }
}

// Per output column c < cols: the sum over `blocks` partial rows [blocks][cols], one wave
// per column (lane-strided, then the wave's fixed reduction tree). Column c goes to
// out_a[c] when c < split, else out_b[c - split]; with dup > 0, columns c < dup also go to
// out_b[c].
__global__ __launch_bounds__(kRowBlock) void col_finish(const float* partial, int blocks,
                                                        int64_t cols, int64_t split, float* out_a,
                                                        float* out_b, int64_t dup) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
  if (col >= cols) return;
  const int lane = lane_id();
  float s = 0.f;
  for (int k = lane; k < blocks; k += kWave) s += partial[static_cast<int64_t>(k) * cols + col];
  s = wave_sum(s);
  if (lane == 0) {
    if (col < split) {
      out_a[col] = s;
      if (col < dup) out_b[col] = s;
    } else {
      out_b[col - split + dup] = s;
    }
  }
}

// ---------------------------------------------------------------------------------
// Recurrent cell gates
// ---------------------------------------------------------------------------------
// gi = x W_ih^T + b_ih, gh = h W_hh^T + b_hh, gate blocks [r | z | n] (torch.nn.GRUCell):
//   r = s(gi_r + gh_r), z = s(gi_z + gh_z), c = tanh(gi_n + r gh_n), h' = (1 - z) c + z h.
// With bi / bh the products come without their biases, added here (per column).
// ws keeps [r | z | c | gh_n] per row for the backward.
__global__ __launch_bounds__(kColBlock) void gru_fwd(int64_t n, int32_t m, const float* gi,
                                                     int64_t ldgi, const float* gh, int64_t ldgh,
                                                     const float* h, int64_t ldh, const float* bi,
                                                     const float* bh, float* hy, int64_t ldy,
                                                     float* ws) {
  const RowChunk c = row_chunk(n);
  for (int j = c.lane; j < m; j += kColLanes) {
    // the biases of this column's three gates (0 without)
    const float br = (bi ? bi[j] : 0.f) + (bh ? bh[j] : 0.f);
    const float bz = (bi ? bi[m + j] : 0.f) + (bh ? bh[m + j] : 0.f);
    const float bin = bi ? bi[2 * m + j] : 0.f, bhn = bh ? bh[2 * m + j] : 0.f;
    for (int64_t i = c.r0 + c.phase; i < c.r1; i += kRowPhases) {
      const float* a = gi + i * ldgi;
      const float* q = gh + i * ldgh;
      const float r = sigmoid(a[j] + q[j] + br);
      const float z = sigmoid(a[m + j] + q[m + j] + bz);
      const float hn = q[2 * m + j] + bhn;
      const float nc = tanhf(a[2 * m + j] + bin + r * hn);
      const float hv = h ? h[i * ldh + j] : 0.f;
      hy[i * ldy + j] = (1.f - z) * nc + z * hv;
      float* s = ws + i * 4 * m;
      s[j] = r;
      s[m + j] = z;
      s[2 * m + j] = nc;
      s[3 * m + j] = hn;
    }
  }
}

// dgi = [dr' | dz' | dn'], dgh = [dr' | dz' | dn' r] with dn' = dy (1 - z)(1 - c^2),
// dz' = dy (h - c) z (1 - z), dr' = dn' gh_n r (1 - r); dh = dy z (the direct path; the
// path through W_hh is the caller's product dgh W_hh). With partial, the workgroup's column
// sums of dr', dz', dn', dn' r go to partial[blk][4m] (the bias gradients).
__global__ __launch_bounds__(kColBlock) void gru_bwd(int64_t n, int32_t m, const float* dy,
                                                     int64_t ldd, const float* ws, const float* h,
                                                     int64_t ldh, float* dgi, int64_t ldgi,
                                                     float* dgh, int64_t ldgh, float* dh,
                                                     int64_t lddh, float* partial) {
  const RowChunk c = row_chunk(n);
  for (int j0 = 0; j0 < m; j0 += kColLanes) {
    const int j = j0 + c.lane;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (j < m) {
      for (int64_t i = c.r0 + c.phase; i < c.r1; i += kRowPhases) {
        const float* s = ws + i * 4 * m;
        const float r = s[j], z = s[m + j], nc = s[2 * m + j], hn = s[3 * m + j];
        const float g = dy[i * ldd + j];
        const float hv = h ? h[i * ldh + j] : 0.f;
        const float dn = g * (1.f - z) * (1.f - nc * nc);
        const float dz = g * (hv - nc) * z * (1.f - z);
        const float dr = dn * hn * r * (1.f - r);
        float* a = dgi + i * ldgi;
        float* q = dgh + i * ldgh;
        a[j] = dr;
        a[m + j] = dz;
        a[2 * m + j] = dn;
        q[j] = dr;
        q[m + j] = dz;
        q[2 * m + j] = dn * r;
        if (dh) dh[i * lddh + j] = g * z;
        v[0] += dr;
        v[1] += dz;
        v[2] += dn;
        v[3] += dn * r;
      }
    }
    if (partial) phase_sums<4>(v, c, j, m, m, partial + static_cast<int64_t>(blockIdx.x) * 4 * m);
  }
}

// torch.nn.RNNCell (tanh): h' = tanh(gi + gh) (+ the biases bi, bh when the products come
// without them); backward da = dy (1 - h'^2).
__global__ __launch_bounds__(kEltBlock) void rnn_fwd(int64_t n, int32_t m, const float* gi,
                                                     int64_t ldgi, const float* gh, int64_t ldgh,
                                                     const float* bi, const float* bh, float* hy,
                                                     int64_t ldy) {
  const int64_t total = n * m;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kEltBlock + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kEltBlock) {
    const int64_t i = idx / m;
    const int j = static_cast<int>(idx - i * m);
    const float b = (bi ? bi[j] : 0.f) + (bh ? bh[j] : 0.f);
    hy[i * ldy + j] = tanhf(gi[i * ldgi + j] + gh[i * ldgh + j] + b);
  }
}

__global__ __launch_bounds__(kEltBlock) void rnn_bwd(int64_t n, int32_t m, const float* dy,
                                                     int64_t ldd, const float* hy, int64_t ldy,
                                                     float* da, int64_t lda) {
  const int64_t total = n * m;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kEltBlock + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kEltBlock) {
    const int64_t i = idx / m;
    const int j = static_cast<int>(idx - i * m);
    const float y = hy[i * ldy + j];
    da[i * lda + j] = dy[i * ldd + j] * (1.f - y * y);
  }
}

// ---------------------------------------------------------------------------------
// Write-back: one winner per node id
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t row_tag(uint32_t gen, int64_t r) {
  return (static_cast<uint64_t>(gen) << 32) | static_cast<uint64_t>(r);
}

// Node id of write row r: ids[r] (memory), or the edge's source / destination for even /
// odd r (mailbox: rows interleaved src_0, dst_0, src_1, ...).
__device__ __forceinline__ int64_t write_row_id(const void* a, const void* b, int id64,
                                                int64_t r) {
  return b ? load_id((r & 1) ? b : a, id64, r >> 1) : load_id(a, id64, r);
}

__global__ __launch_bounds__(kEltBlock) void claim_rows(const void* a, const void* b, int id64,
                                                        int64_t rows, int64_t num_nodes,
                                                        unsigned long long* last, uint32_t gen) {
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kEltBlock + threadIdx.x; r < rows;
       r += static_cast<int64_t>(gridDim.x) * kEltBlock) {
    const int64_t id = write_row_id(a, b, id64, r);
    if (id >= 0 && id < num_nodes) atomicMax(last + id, static_cast<unsigned long long>(row_tag(gen, r)));
  }
}

struct MemoryWriteParams {
  const void* ids;
  int id64;
  int64_t rows, num_nodes;
  const float* mem;  // [rows][ldm]
  int64_t ldm;
  int32_t m;
  const float* ts;   // [rows]
  float* node_memory;
  int64_t ld_nm;
  float* node_ts;
  const unsigned long long* last;
  uint32_t gen;
};

template <bool V4>
__global__ __launch_bounds__(kRowBlock) void memory_winners(MemoryWriteParams P) {
  const int lane = lane_id();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kRowWaves;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave; r < P.rows;
       r += waves) {
    const int64_t id = load_id(P.ids, P.id64, r);
    if (id < 0 || id >= P.num_nodes || P.last[id] != row_tag(P.gen, r)) continue;
    wave_copy<V4>(P.mem + r * P.ldm, P.node_memory + id * P.ld_nm, P.m, true, lane);
    if (lane == 0) P.node_ts[id] = P.ts[r];
  }
}

struct MailboxWriteParams {
  const void* src;
  const void* dst;
  int id64;
  int64_t n, num_nodes;   // n edges: 2n write rows
  const float* mem;       // [2n][ldm]: rows 0..n-1 sources, n..2n-1 destinations
  int64_t ldm;
  int32_t m;
  const float* ef;        // [n][lde] or null
  int64_t lde;
  int32_t de;
  const float* ts;        // [2n], read at the write row's own index
  float* mailbox;         // [num_nodes][slots][2m + de] (rows of ld_mb)
  int64_t ld_mb;
  float* mailbox_ts;      // [num_nodes][slots]
  int64_t* next_pos;      // [num_nodes]
  int32_t slots;
  const unsigned long long* last;
  uint32_t gen;
};

template <bool V4>
__global__ __launch_bounds__(kRowBlock) void mailbox_winners(MailboxWriteParams P) {
  const int lane = lane_id();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kRowWaves;
  const int64_t mail = 2 * static_cast<int64_t>(P.m) + P.de;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave; r < 2 * P.n;
       r += waves) {
    const int64_t id = write_row_id(P.src, P.dst, P.id64, r);
    if (id < 0 || id >= P.num_nodes || P.last[id] != row_tag(P.gen, r)) continue;
    const int64_t pos = P.next_pos[id];
    if (pos < 0 || pos >= P.slots) continue;  // a corrupt position writes nothing
    const int64_t k = r >> 1;
    const bool odd = (r & 1) != 0;
    const float* self = P.mem + (odd ? P.n + k : k) * P.ldm;
    const float* other = P.mem + (odd ? k : P.n + k) * P.ldm;
    float* out = P.mailbox + id * P.ld_mb + pos * mail;
    wave_copy<V4>(self, out, P.m, true, lane);
    wave_copy<V4>(other, out + P.m, P.m, true, lane);
    if (P.de > 0) wave_copy<V4>(P.ef + k * P.lde, out + 2 * P.m, P.de, true, lane);
    if (lane == 0) {
      P.mailbox_ts[id * P.slots + pos] = P.ts[r];
      if (P.slots > 1) P.next_pos[id] = (pos + 1) % P.slots;
    }
  }
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_mail_gather_f32(int64_t n, const void* ids, int32_t ids_are_int64,
                                  int64_t num_nodes, const float* memory, int64_t ld_memory,
                                  int32_t dim_memory, const float* memory_ts,
                                  const float* mailbox, int64_t ld_mailbox, int64_t mail_width,
                                  const float* mailbox_ts, int32_t slots, float* mem_out,
                                  int64_t ld_mem_out, float* mem_ts_out, float* x_out,
                                  int64_t ld_x, float* mail_ts_out, hipStream_t stream) {
  if (n < 0 || num_nodes < 0 || dim_memory < 0 || mail_width < 0 || slots < 0) return FA_EINVAL;
  if (n == 0) return FA_OK;
  if (!ids || !mem_out || !mem_ts_out || !x_out || (slots > 0 && !mail_ts_out)) return FA_EINVAL;
  if (num_nodes > 0 && (!memory || !memory_ts || !mailbox || (slots > 0 && !mailbox_ts)))
    return FA_EINVAL;
  if (ld_memory < dim_memory || ld_mailbox < mail_width || ld_mem_out < dim_memory ||
      ld_x < mail_width)
    return FA_EINVAL;
  MailGatherParams P{ids, ids_are_int64 ? 1 : 0, n, num_nodes, memory, ld_memory, dim_memory,
                     memory_ts, mailbox, ld_mailbox, mail_width, mailbox_ts, slots, mem_out,
                     ld_mem_out, mem_ts_out, x_out, ld_x, mail_ts_out};
  const bool v4 = al16(memory) && al16(mailbox) && al16(mem_out) && al16(x_out) &&
                  ld_memory % 4 == 0 && ld_mailbox % 4 == 0 && ld_mem_out % 4 == 0 &&
                  ld_x % 4 == 0 && dim_memory % 4 == 0 && mail_width % 4 == 0;
  if (v4) mail_gather<true><<<row_grid(n), kRowBlock, 0, stream>>>(P);
  else mail_gather<false><<<row_grid(n), kRowBlock, 0, stream>>>(P);
  return launch_status();
}

extern "C" int fa_time_rows_f32(int64_t n, const float* ts, const float* mem_ts, const float* w,
                                const float* b, int32_t dt, float* out, int64_t ld_out,
                                hipStream_t stream) {
  if (n < 0 || dt < 0 || ld_out < dt) return FA_EINVAL;
  if (n == 0 || dt == 0) return FA_OK;
  if (!ts || !w || !b || !out) return FA_EINVAL;
  time_rows<<<elt_grid(n * dt), kEltBlock, 0, stream>>>(ts, mem_ts, n, w, b, dt, out, ld_out);
  return launch_status();
}

extern "C" size_t fa_time_rows_grad_scratch_bytes(int32_t dt) {
  return dt > 0 ? sizeof(float) * static_cast<size_t>(kMaxChunkBlocks) * 2 * dt : 0;
}

extern "C" int fa_time_rows_grad_f32(int64_t n, const float* ts, const float* mem_ts,
                                     const float* w, const float* b, int32_t dt, const float* g,
                                     int64_t ld_g, float* dw, float* db, void* scratch,
                                     size_t scratch_bytes, hipStream_t stream) {
  if (n < 0 || dt < 0 || ld_g < dt) return FA_EINVAL;
  if (dt == 0) return FA_OK;
  if (!w || !b || !dw || !db || (n > 0 && (!ts || !g))) return FA_EINVAL;
  if (!scratch || scratch_bytes < fa_time_rows_grad_scratch_bytes(dt)) return FA_ESCRATCH;
  float* partial = static_cast<float*>(scratch);
  const int blocks = n > 0 ? chunk_blocks(n) : 0;
  if (blocks > 0)
    time_rows_grad<<<blocks, kColBlock, 0, stream>>>(ts, mem_ts, n, w, b, dt, g, ld_g, partial);
  const int64_t cols = 2 * static_cast<int64_t>(dt);
  col_finish<<<static_cast<int>((cols + kRowWaves - 1) / kRowWaves), kRowBlock, 0, stream>>>(
      partial, blocks, cols, dt, dw, db, 0);
  return launch_status();
}

extern "C" int fa_gru_fwd_f32(int64_t n, int32_t m, const float* gi, int64_t ld_gi,
                              const float* gh, int64_t ld_gh, const float* h, int64_t ld_h,
                              const float* b_ih, const float* b_hh, float* hy, int64_t ld_hy,
                              float* workspace, hipStream_t stream) {
  if (n < 0 || m < 0 || ld_gi < 3 * static_cast<int64_t>(m) || ld_gh < 3 * static_cast<int64_t>(m) ||
      ld_hy < m || (h && ld_h < m))
    return FA_EINVAL;
  if (n == 0 || m == 0) return FA_OK;
  if (!gi || !gh || !hy || !workspace) return FA_EINVAL;
  gru_fwd<<<chunk_blocks(n), kColBlock, 0, stream>>>(n, m, gi, ld_gi, gh, ld_gh, h, ld_h, b_ih, b_hh,
                                                     hy, ld_hy, workspace);
  return launch_status();
}

extern "C" size_t fa_gru_bwd_scratch_bytes(int64_t n, int32_t m) {
  return n > 0 && m > 0 ? sizeof(float) * static_cast<size_t>(chunk_blocks(n)) * 4 * m : 0;
}

extern "C" int fa_gru_bwd_f32(int64_t n, int32_t m, const float* dhy, int64_t ld_dhy,
                              const float* workspace, const float* h, int64_t ld_h, float* dgi,
                              int64_t ld_dgi, float* dgh, int64_t ld_dgh, float* dh,
                              int64_t ld_dh, float* db_ih, float* db_hh, void* scratch,
                              size_t scratch_bytes, hipStream_t stream) {
  if (n < 0 || m < 0 || ld_dhy < m || ld_dgi < 3 * static_cast<int64_t>(m) ||
      ld_dgh < 3 * static_cast<int64_t>(m) || (h && ld_h < m) || (dh && ld_dh < m) ||
      (!db_ih != !db_hh))
    return FA_EINVAL;
  if (m == 0) return FA_OK;
  const bool sums = db_ih != nullptr;
  if (sums && n > 0 && (!scratch || scratch_bytes < fa_gru_bwd_scratch_bytes(n, m)))
    return FA_ESCRATCH;
  if (n > 0) {
    if (!dhy || !workspace || !dgi || !dgh) return FA_EINVAL;
    gru_bwd<<<chunk_blocks(n), kColBlock, 0, stream>>>(n, m, dhy, ld_dhy, workspace, h, ld_h, dgi,
                                                       ld_dgi, dgh, ld_dgh, dh, ld_dh,
                                                       sums ? static_cast<float*>(scratch) : nullptr);
  }
  if (sums) {
    // partial columns [dr' | dz' | dn' | dn' r]: db_ih = the first three, db_hh = the first
    // two and the fourth
    const int64_t cols = 4 * static_cast<int64_t>(m);
    col_finish<<<static_cast<int>((cols + kRowWaves - 1) / kRowWaves), kRowBlock, 0, stream>>>(
        static_cast<const float*>(scratch), n > 0 ? chunk_blocks(n) : 0, cols,
        3 * static_cast<int64_t>(m), db_ih, db_hh, 2 * static_cast<int64_t>(m));
  }
  return launch_status();
}

extern "C" int fa_rnn_fwd_f32(int64_t n, int32_t m, const float* gi, int64_t ld_gi,
                              const float* gh, int64_t ld_gh, const float* b_ih, const float* b_hh,
                              float* hy, int64_t ld_hy, hipStream_t stream) {
  if (n < 0 || m < 0 || ld_gi < m || ld_gh < m || ld_hy < m) return FA_EINVAL;
  if (n == 0 || m == 0) return FA_OK;
  if (!gi || !gh || !hy) return FA_EINVAL;
  rnn_fwd<<<elt_grid(n * m), kEltBlock, 0, stream>>>(n, m, gi, ld_gi, gh, ld_gh, b_ih, b_hh, hy,
                                                     ld_hy);
  return launch_status();
}

extern "C" int fa_rnn_bwd_f32(int64_t n, int32_t m, const float* dhy, int64_t ld_dhy,
                              const float* hy, int64_t ld_hy, float* da, int64_t ld_da,
                              hipStream_t stream) {
  if (n < 0 || m < 0 || ld_dhy < m || ld_hy < m || ld_da < m) return FA_EINVAL;
  if (n == 0 || m == 0) return FA_OK;
  if (!dhy || !hy || !da) return FA_EINVAL;
  rnn_bwd<<<elt_grid(n * m), kEltBlock, 0, stream>>>(n, m, dhy, ld_dhy, hy, ld_hy, da, ld_da);
  return launch_status();
}

extern "C" int fa_memory_update_f32(int64_t rows, const void* ids, int32_t ids_are_int64,
                                    const float* mem, int64_t ld_mem, int32_t dim_memory,
                                    const float* ts, float* node_memory, int64_t ld_node_memory,
                                    float* node_memory_ts, int64_t num_nodes,
                                    unsigned long long* last, uint32_t generation,
                                    hipStream_t stream) {
  if (rows < 0 || dim_memory < 0 || num_nodes < 0 || ld_mem < dim_memory ||
      ld_node_memory < dim_memory || rows >= (int64_t{1} << 32) || generation == 0)
    return FA_EINVAL;
  if (rows == 0 || num_nodes == 0) return FA_OK;
  if (!ids || !mem || !ts || !node_memory || !node_memory_ts || !last) return FA_EINVAL;
  const int id64 = ids_are_int64 ? 1 : 0;
  claim_rows<<<elt_grid(rows), kEltBlock, 0, stream>>>(ids, nullptr, id64, rows, num_nodes, last,
                                                       generation);
  MemoryWriteParams P{ids, id64, rows, num_nodes, mem, ld_mem, dim_memory, ts, node_memory,
                      ld_node_memory, node_memory_ts, last, generation};
  const bool v4 = al16(mem) && al16(node_memory) && ld_mem % 4 == 0 && ld_node_memory % 4 == 0 &&
                  dim_memory % 4 == 0;
  if (v4) memory_winners<true><<<row_grid(rows), kRowBlock, 0, stream>>>(P);
  else memory_winners<false><<<row_grid(rows), kRowBlock, 0, stream>>>(P);
  return launch_status();
}

extern "C" int fa_mailbox_update_f32(int64_t n, const void* src_ids, const void* dst_ids,
                                     int32_t ids_are_int64, const float* mem, int64_t ld_mem,
                                     int32_t dim_memory, const float* edge_feats, int64_t ld_edge,
                                     int32_t dim_edge, const float* ts, float* mailbox,
                                     int64_t ld_mailbox, float* mailbox_ts, int64_t* next_pos,
                                     int32_t slots, int64_t num_nodes, unsigned long long* last,
                                     uint32_t generation, hipStream_t stream) {
  if (n < 0 || dim_memory < 0 || dim_edge < 0 || slots < 1 || num_nodes < 0 ||
      ld_mem < dim_memory || (dim_edge > 0 && ld_edge < dim_edge) ||
      ld_mailbox < static_cast<int64_t>(slots) * (2 * static_cast<int64_t>(dim_memory) + dim_edge) ||
      2 * n >= (int64_t{1} << 32) || generation == 0)
    return FA_EINVAL;
  if (n == 0 || num_nodes == 0) return FA_OK;
  if (!src_ids || !dst_ids || !mem || !ts || !mailbox || !mailbox_ts || !next_pos || !last ||
      (dim_edge > 0 && !edge_feats))
    return FA_EINVAL;
  const int id64 = ids_are_int64 ? 1 : 0;
  claim_rows<<<elt_grid(2 * n), kEltBlock, 0, stream>>>(src_ids, dst_ids, id64, 2 * n, num_nodes,
                                                        last, generation);
  MailboxWriteParams P{src_ids, dst_ids, id64, n, num_nodes, mem, ld_mem, dim_memory, edge_feats,
                       ld_edge, dim_edge, ts, mailbox, ld_mailbox, mailbox_ts, next_pos, slots,
                       last, generation};
  const int64_t mail = 2 * static_cast<int64_t>(dim_memory) + dim_edge;
  const bool v4 = al16(mem) && al16(mailbox) && al16(edge_feats) && ld_mem % 4 == 0 &&
                  ld_mailbox % 4 == 0 && (dim_edge == 0 || ld_edge % 4 == 0) &&
                  dim_memory % 4 == 0 && dim_edge % 4 == 0 && mail % 4 == 0;
  if (v4) mailbox_winners<true><<<row_grid(2 * n), kRowBlock, 0, stream>>>(P);
  else mailbox_winners<false><<<row_grid(2 * n), kRowBlock, 0, stream>>>(P);
  return launch_status();
}
