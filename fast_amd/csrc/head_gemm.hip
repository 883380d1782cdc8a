// Per-head projections between the K-space blocks [G][N][C] of the fused kernels and the
// head-blocked feature rows [N][G*J] of the layer (G heads, J = dim_out/heads <= 64,
// C = Kp). The layer needs three products per weight W[g] ([J][C] per head):
//   proj   Y[g][n][:] = X[n][g*J : g*J+J] W[g]  (+ bias[g])     (q~ = Q W_k, dxbar = dagg W_v)
//   reduce Z[n][g*J : g*J+J] = Y[g][n][:] W[g]^T                (agg = xbar W_v^T, dQ = dq~ W_k^T)
//   wgrad  dW[g] = sum_n X[n][g-block]^T Y[g][n][:]  (+ sum_n Y[g][n][:] as row J)
// They are tall and skinny (N ~ 1e5 rows, J ~ 32..64, C ~ 400..700): their cost is the
// stream over the [G][N][C] block. proj (and reduce and wgrad for unaligned Y rows) runs on
// the fp32 matrix cores,
//   MFMA 16x16x4 f32, lane l: A[l%16][l/16], B[l/16][l%16], D[4*(l/16)+r][l%16], r < 4,
// and reduce and wgrad on the bf16 ones with split operands (head_reduce_bf, head_wgrad_bf),
// with every global access of the block a 16-byte-per-lane load or store (the texture
// unit takes one lane per clock whatever the width, so narrower accesses to the block
// would cap the bandwidth). The small operands are staged in LDS: the X rows of a tile,
// read with coalesced loads by the whole workgroup, and (reduce) the whole of W[g].
// Because a product does not depend on the order of the contraction, the k-slot of a
// lane may stand for any index as long as A and B agree; reduce uses that to read four
// consecutive columns of a row with one 16-byte load, and wgrad to give each lane four
// consecutive columns (tile t takes columns 4m + t).
#include "fa_common.hpp"

namespace fa {
namespace {

using f4 = __attribute__((ext_vector_type(4))) float;
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // raw (unformatted) 32-bit buffer
constexpr uint32_t kOob = 0x7ffffff0u;  // offset past every range used here (< 2 GiB)

// Buffer descriptor over [base, base + bytes): loads past the range return 0 and stores
// past it are dropped, which covers the ragged last tile without branches.
__device__ __forceinline__ rsrc_t rsrc(const void* base, int64_t bytes) {
  const int64_t b = bytes < 0 ? 0 : (bytes > 0xffffffffLL ? 0xffffffffLL : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(static_cast<uint32_t>(b)), kRsrcWord3);
}
__device__ __forceinline__ float ld1(rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0));
}
__device__ __forceinline__ void st1(rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ f4 ld4(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
  return f4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
            __uint_as_float(v[3])};
}
using f2 = __attribute__((ext_vector_type(2))) float;
__device__ __forceinline__ f2 ld2(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
  return f2{__uint_as_float(v[0]), __uint_as_float(v[1])};
}
__device__ __forceinline__ void st4(rsrc_t r, uint32_t off, f4 v) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  u4 u;
  u[0] = __float_as_uint(v[0]);
  u[1] = __float_as_uint(v[1]);
  u[2] = __float_as_uint(v[2]);
  u[3] = __float_as_uint(v[3]);
  __builtin_amdgcn_raw_buffer_store_b128(u, r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Keeps the instruction scheduler from moving anything across this point: a prefetch
// issued before it stays ahead of the work after it (the scheduler would otherwise sink
// the loads next to their first use, and the wait for them would expose their latency).
__device__ __forceinline__ void pin() { __builtin_amdgcn_sched_barrier(0); }

// Descriptor over rows [n0, n0+16) of a row-major array (row stride ld, width w): empty
// past the last row, so a prefetch beyond the end reads zeros.
__device__ __forceinline__ rsrc_t tile_rsrc(const float* base, int64_t n, int64_t n0, int64_t ld,
                                            int64_t w) {
  const int64_t rows = n - n0 < 16 ? n - n0 : 16;
  return rsrc(base + n0 * ld, rows > 0 ? 4 * ((rows - 1) * ld + w) : 0);
}

// ----- proj ------------------------------------------------------------------------------
struct ProjParams {
  int64_t n; int j, c, g;
  const float* x; int64_t ldx; int64_t xg;   // X row n, group g: x + n*ldx + g*xg
  const float* w; int64_t wg; int64_t ldw;   // W[g][j][c] = w[g*wg + j*ldw + c]
  const float* bias; int64_t bg;             // bias[g][c] = bias[g*bg + c] (may be null)
  float* y; int64_t yg; int64_t ldy;         // Y[g][n][c] = y[g*yg + n*ldy + c]
  int ncg4;                                  // workgroups per group along the columns
  int vec;                                   // Y rows 16-byte aligned and c % 4 == 0
};

constexpr int kProjCt = 6;   // 16-column tiles per wave (96 columns)
#ifndef FA_PROJ_RT
#define FA_PROJ_RT 2
#endif
constexpr int kProjRt = FA_PROJ_RT;  // 16-row tiles per workgroup step (one LDS sync each)

// Workgroup: one head g, four 96-column groups (one per wave), 16-row tiles grid-stride.
// The product is formed transposed, Y^T tile = W^T (A: registers for the whole kernel,
// KS = ceil(J/4) k-steps x CT tiles, zero past J and C) times X^T (B: from the tile's X
// rows in LDS), so that each lane ends up with four consecutive columns of one row and
// stores them as one float4. The workgroup loads the next tile's X rows (coalesced, one
// element per thread and load) while the current tile is multiplied and stored.
template <int KS, int CT, bool BIAS, bool VEC>
__global__ __launch_bounds__(kBlock) void head_proj(ProjParams P) {
  constexpr int RT = kProjRt;                          // 16-row tiles per step
  constexpr int XW = 4 * KS + 1;                       // odd LDS row: rows in distinct banks
  constexpr int XL = (RT * 16 * 4 * KS + kBlock - 1) / kBlock;
  __shared__ float xs[2][RT * 16][XW];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int g = blockIdx.y / P.ncg4;
  const int c0 = ((blockIdx.y - g * P.ncg4) * kWavesPerBlock + wave) * (16 * CT);
  const bool active = c0 < P.c;                         // idle waves still load X
  const int li = lane & 15, lk = lane >> 4;
  const float* w = P.w + g * P.wg;
  float wf[KS][CT];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int t = 0; t < CT; ++t) {
      const int jj = 4 * s + lk, cc = c0 + 16 * t + li;
      wf[s][t] = (active && jj < P.j && cc < P.c) ? w[jj * P.ldw + cc] : 0.f;
    }
  }
  // output of tile t: columns cb .. cb+3 (cb = c0 + 16t + 4lk) of row n0 + li
  f4 bias4[BIAS ? CT : 1];
  uint32_t yo[CT];
#pragma unroll
  for (int t = 0; t < CT; ++t) {
    const int cb = c0 + 16 * t + 4 * lk;
    if (BIAS) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bias4[t][r] = cb + r < P.c ? P.bias[g * P.bg + cb + r] : 0.f;
    }
    yo[t] = cb < P.c ? 4u * static_cast<uint32_t>(li * P.ldy + cb) : kOob;
  }
  // X elements of this thread: e = tid + kBlock*i of the RT*16 x J step block
  uint32_t xo[XL];
  int xl[XL];                                           // LDS slot (row*XW + col), -1: none
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int e = tid + kBlock * i;
    const int r = e / P.j, cc = e - r * P.j;
    const bool ok = e < RT * 16 * P.j;
    xo[i] = ok ? 4u * static_cast<uint32_t>(r * P.ldx + cc) : kOob;
    xl[i] = ok ? r * XW + cc : -1;
  }
  // columns J .. 4KS of both buffers stay zero
  for (int e = tid; e < 2 * RT * 16 * (XW - P.j); e += kBlock) {
    const int b = e / (RT * 16 * (XW - P.j)), rem = e - b * RT * 16 * (XW - P.j);
    const int r = rem / (XW - P.j);
    xs[b][r][P.j + (rem - r * (XW - P.j))] = 0.f;
  }
  const float* xbase = P.x + g * P.xg;
  float* ybase = P.y + g * P.yg;
  const int64_t tiles = (P.n + 16 * RT - 1) / (16 * RT);   // steps of RT*16 rows
  float xv[XL];
  auto gload = [&](int64_t tile) {
    const int64_t n0 = tile * 16 * RT;
    const int64_t rows = P.n - n0 < 16 * RT ? P.n - n0 : 16 * RT;
    const rsrc_t rx = rsrc(xbase + n0 * P.ldx, rows > 0 ? 4 * ((rows - 1) * P.ldx + P.j) : 0);
#pragma unroll
    for (int i = 0; i < XL; ++i) xv[i] = ld1(rx, xo[i]);
  };
  auto lstore = [&](int b) {
#pragma unroll
    for (int i = 0; i < XL; ++i)
      if (xl[i] >= 0) (&xs[b][0][0])[xl[i]] = xv[i];
  };
  int64_t tile = blockIdx.x;
  gload(tile);
  lstore(0);
  __syncthreads();
  int b = 0;
  for (; tile < tiles; tile += gridDim.x) {
    gload(tile + gridDim.x);
    pin();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (!active) break;
      // all of the tile's B values first: one LDS wait, not one per k-step
      float bx[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) bx[s] = xs[b][16 * rt + li][4 * s + lk];
      pin();
      f4 acc[CT];
#pragma unroll
      for (int t = 0; t < CT; ++t) acc[t] = BIAS ? bias4[t] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int t = 0; t < CT; ++t) acc[t] = mfma4(wf[s][t], bx[s], acc[t]);
      }
      const rsrc_t ry = tile_rsrc(ybase, P.n, (tile * RT + rt) * 16, P.ldy, P.c);
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        if (VEC) {
          st4(ry, yo[t], acc[t]);
        } else {
          const int cb = c0 + 16 * t + 4 * lk;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            st1(ry, (yo[t] == kOob || cb + r >= P.c) ? kOob : yo[t] + 4u * r, acc[t][r]);
        }
      }
    }
    lstore(b ^ 1);
    __syncthreads();
    b ^= 1;
  }
}

// ----- reduce ----------------------------------------------------------------------------
struct ReduceParams {
  int64_t n; int j, c, g;
  const float* y; int64_t yg; int64_t ldy;   // Y[g][n][c] = y[g*yg + n*ldy + c]
  const float* w; int64_t wg; int64_t ldw;   // W[g][j][c] = w[g*wg + j*ldw + c]
  float* z; int64_t ldz; int64_t zg;         // Z[n][g*J + j] = z[n*ldz + g*zg + j]
  int c16;                                   // 16-column groups of a row, rounded up to kRedDepth
  int kb, cp;                                // split-bf16 form: 32-column k-blocks (a multiple
                                             // of kRbDepth) and the LDS row in bf16
};

constexpr int kRedWaves = 8;                 // waves per reduce workgroup
#ifndef FA_RED_DEPTH
#define FA_RED_DEPTH 8
#endif
constexpr int kRedDepth = FA_RED_DEPTH;      // column groups of Y in flight per wave
constexpr int kRedBlock = kRedWaves * kWave;

// LDS bytes of reduce: W[g] as float4 rows [J+1][4*c16 + 1] (the extra float4 staggers
// the rows over the banks), row J zero.
size_t reduce_lds_bytes(int j, int c16) { return static_cast<size_t>(j + 1) * (4 * c16 + 1) * 16; }

// Workgroup: one head g, its W[g] in LDS; each wave takes whole 16-row tiles (grid-stride)
// and runs over all C columns, 16 at a time: k-step 4q + t of lane l stands for column
// 16q + 4*(l/16) + t, so a lane's A values for four k-steps are one float4 of its row and
// its B values one float4 of W[g][j] from LDS. Four column groups of Y are in flight
// ahead of the one multiplied (four register sets, named, so no copies between them).
template <int JT, bool VEC>
__global__ __launch_bounds__(kRedBlock) void head_reduce(ReduceParams P) {
  extern __shared__ f4 wl[];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int g = blockIdx.y;
  const int c4n = 4 * P.c16 + 1;               // LDS row stride in float4
  const float* w = P.w + g * P.wg;
  const bool wvec = !(P.ldw & 3) && !(reinterpret_cast<uintptr_t>(w) & 15);
  for (int i = tid; i < (P.j + 1) * c4n; i += kRedBlock) {
    const int jr = i / c4n, c4 = i - jr * c4n;
    f4 v = f4{0.f, 0.f, 0.f, 0.f};
    if (jr < P.j && wvec && 4 * c4 + 3 < P.c) {
      v = *reinterpret_cast<const f4*>(w + jr * P.ldw + 4 * c4);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (jr < P.j && 4 * c4 + t < P.c) v[t] = w[jr * P.ldw + 4 * c4 + t];
    }
    wl[i] = v;
  }
  __syncthreads();
  const int li = lane & 15, lk = lane >> 4;
  int wrow[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) wrow[jt] = (16 * jt + li < P.j ? 16 * jt + li : P.j) * c4n + lk;
  const float* ybase = P.y + g * P.yg;
  const int64_t tiles = (P.n + 15) / 16;
  const uint32_t yrow = 4u * static_cast<uint32_t>(li * P.ldy);
  for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kRedWaves + wave; tile < tiles;
       tile += static_cast<int64_t>(gridDim.x) * kRedWaves) {
    const int64_t n0 = tile * 16;
    const rsrc_t ry = tile_rsrc(ybase, P.n, n0, P.ldy, P.c);
    auto ly = [&](int q) -> f4 {
      const int cq = 16 * q + 4 * lk;
      if (VEC) return ld4(ry, cq < P.c ? yrow + 4u * cq : kOob);
      f4 a;
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = ld1(ry, cq + t < P.c ? yrow + 4u * (cq + t) : kOob);
      return a;
    };
    f4 acc[JT];
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) acc[jt] = f4{0.f, 0.f, 0.f, 0.f};
    // W values of column group q (clamped to the row), read one group ahead of their use
    auto lw = [&](int q, f4 (&wv)[JT]) {
      const int qq = q < P.c16 ? q : P.c16 - 1;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) wv[jt] = wl[wrow[jt] + 4 * qq];
    };
    auto mm = [&](const f4& a, const f4 (&wv)[JT]) {
      // consecutive products go to different accumulators
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) acc[jt] = mfma4(a[t], wv[jt][t], acc[jt]);
      }
    };
    // issued in order (the loop's waits count on ay[0] being the oldest); kRedDepth column
    // groups are in flight ahead of the one multiplied
    f4 ay[kRedDepth];
#pragma unroll
    for (int d = 0; d < kRedDepth; ++d) {
      ay[d] = ly(d);
      pin();
    }
    f4 wa[JT], wb[JT];
    lw(0, wa);
    for (int q = 0; q < P.c16; q += kRedDepth) {   // c16 is a multiple of kRedDepth
#pragma unroll
      for (int d = 0; d < kRedDepth; d += 2) {
        lw(q + d + 1, wb);
        mm(ay[d], wa);
        pin();
        ay[d] = ly(q + d + kRedDepth);
        pin();
        lw(q + d + 2, wa);
        mm(ay[d + 1], wb);
        pin();
        ay[d + 1] = ly(q + d + 1 + kRedDepth);
        pin();
      }
    }
    // D row 4lk + r, column 16jt + li
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      const int jj = 16 * jt + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = n0 + 4 * lk + r;
        if (jj < P.j && row < P.n) P.z[row * P.ldz + g * P.zg + jj] = acc[jt][r];
      }
    }
  }
}

// ----- wgrad -----------------------------------------------------------------------------
struct WgradParams {
  int64_t n; int j, c, g, jr;                // jr = j (+1 with the ones row)
  const float* x; int64_t ldx; int64_t xg;   // X row n, group g: x + n*ldx + g*xg
  const float* y; int64_t yg; int64_t ldy;   // Y[g][n][c] = y[g*yg + n*ldy + c]
  float* part;                               // [chunks][g][jr][c]
  int64_t rows;                              // rows per chunk (multiple of 16)
  int ncw4, njg;                             // column and j workgroups per head (the fp32
                                             // kernel's j workgroups are 64-row j groups)
  int vec;                                   // Y rows 16-byte aligned and c % 4 == 0
};

constexpr int kWcols = 64;  // columns per wave in wgrad
// Waves per SIMD the register budget of wgrad is held to (nw waves per workgroup)
constexpr int wgrad_min_waves(int nw, bool vec) { return nw >= 2 && vec ? 4 : 3; }
// LDS row of the staged X block: 80 floats, so the four rows a k-step reads (one per lane
// quarter) start 16 banks apart and the 64 lanes of a read hit distinct banks
constexpr int kWgradLdsRow = 80;
constexpr int kWgradStage = 16;  // rows per LDS stage (one k-block of four MFMA k-steps)

// Workgroup (chunk, g, j group, column quad): each wave accumulates X^T Y over the chunk's
// rows for 16*NJT rows j and 64 columns, 16 rows (4 k-steps, k-slot of lane l = row
// l/16) at a time. The A values come from the block's X rows, staged in LDS by the whole
// workgroup (coalesced loads; the ones row is a column of ones over the valid rows). Tile
// t of the wave stands for the columns cw + 4m + t (m < 16), so the four B values of a
// lane in a k-step are one float4, Y[row][cw + 4*(l%16) .. +3]. The next block's X and Y
// are loaded while the current one is multiplied.
template <int NJT, bool VEC, int NW, int XV>
__global__ __launch_bounds__(NW * kWave, wgrad_min_waves(NW, VEC)) void head_wgrad(WgradParams P) {
  constexpr int XW = kWgradLdsRow;
  constexpr int SR = kWgradStage;              // rows per stage
  constexpr int KK = SR / 4;                   // k-steps per stage
  constexpr int XL = kWave / XV;               // lanes per 64-column X row
  constexpr int XR = NW * kWave / XL;          // stage rows covered by one pass of the threads
  constexpr int XE = (SR + XR - 1) / XR;       // X vectors per thread and stage
  __shared__ __align__(16) float xs[2][SR][XW];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int per_g = P.njg * P.ncw4;
  const int g = blockIdx.y / per_g;
  const int rem = blockIdx.y - g * per_g;
  const int jg = rem / P.ncw4;
  const int cw = ((rem - jg * P.ncw4) * NW + wave) * kWcols;
  const bool active = cw < P.c;
  const int j0 = jg * 64;
  const int li = lane & 15, lk = lane >> 4;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * P.rows;
  const int64_t r1 = P.n < r0 + P.rows ? P.n : r0 + P.rows;
  const float* xbase = P.x + g * P.xg;
  const float* ybase = P.y + g * P.yg;
  // X vectors of this thread: columns xc .. xc+XV-1 (of the 64-column j group) of the stage
  // rows xr + XR*i. j % XV == 0, so a vector lies wholly inside X or wholly past column j.
  const int xr = tid / XL, xc = (tid % XL) * XV;
  const int xj = j0 + xc;
  const uint32_t xo = xj < P.j ? 4u * static_cast<uint32_t>(xr * P.ldx + xj) : kOob;
  const uint32_t xstep = 4u * static_cast<uint32_t>(XR * P.ldx);
  const int cl = cw + 4 * li;                  // first of this lane's four B columns
  const uint32_t yo = (active && cl < P.c) ? 4u * static_cast<uint32_t>(lk * P.ldy + cl) : kOob;
  const uint32_t ystep = 16u * static_cast<uint32_t>(P.ldy);   // 4 rows
  // a stage's rows [nb, nb + SR) of X (rows past r1 read 0)
  auto stage_rsrc = [&](const float* base, int64_t nb, int64_t ld, int64_t w) {
    const int64_t rows = r1 - nb < SR ? r1 - nb : SR;
    return rsrc(base + nb * ld, rows > 0 ? 4 * ((rows - 1) * ld + w) : 0);
  };
  float xv[XE][XV];
  auto xload = [&](int64_t nb) {
    const rsrc_t rx = stage_rsrc(xbase, nb, P.ldx, P.j);
#pragma unroll
    for (int i = 0; i < XE; ++i) {
      const uint32_t off = (xo == kOob || xr + XR * i >= SR) ? kOob : xo + i * xstep;
      if constexpr (XV == 4) {
        const f4 v = ld4(rx, off);
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[i][e] = v[e];
      } else if constexpr (XV == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rx, static_cast<int>(off), 0, 0);
        xv[i][0] = __uint_as_float(v[0]);
        xv[i][1] = __uint_as_float(v[1]);
      } else {
        xv[i][0] = ld1(rx, off);
      }
    }
  };
  auto xstore = [&](int b, int64_t nb) {
    const int64_t left = r1 - nb;              // rows of the stage inside the chunk
    const int valid = left < SR ? static_cast<int>(left) : SR;
#pragma unroll
    for (int i = 0; i < XE; ++i) {
      const int r = xr + XR * i;
      if (XE * XR > SR && r >= SR) continue;
      float v[XV];
#pragma unroll
      for (int e = 0; e < XV; ++e) {
        // past column j: the ones row (with ones) over the rows inside the chunk, else 0
        const float one = (xj + e >= P.j && xj + e < P.jr && r < valid) ? 1.f : 0.f;
        v[e] = xo == kOob ? one : xv[i][e];
      }
      if constexpr (XV == 4) {
        *reinterpret_cast<f4*>(&xs[b][r][xc]) = f4{v[0], v[1], v[2], v[3]};
      } else if constexpr (XV == 2) {
        *reinterpret_cast<float2*>(&xs[b][r][xc]) = make_float2(v[0], v[1]);
      } else {
        xs[b][r][xc] = v[0];
      }
    }
  };
  auto yload = [&](int64_t nb, f4 (&bv)[KK]) {
    const rsrc_t ry = stage_rsrc(ybase, nb, P.ldy, P.c);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (VEC) {
        bv[kk] = ld4(ry, yo == kOob ? kOob : yo + kk * ystep);
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          bv[kk][t] = ld1(ry, (yo == kOob || cl + t >= P.c) ? kOob : yo + kk * ystep + 4u * t);
      }
    }
  };
  f4 acc[NJT][4];
#pragma unroll
  for (int a = 0; a < NJT; ++a)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[a][t] = f4{0.f, 0.f, 0.f, 0.f};
  auto stage = [&](int b, const f4 (&bv)[KK]) {
    // the A values of k-step kk + 1 are read from LDS while k-step kk is multiplied
    float av[2][NJT];
#pragma unroll
    for (int a = 0; a < NJT; ++a) av[0][a] = xs[b][lk][16 * a + li];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) {
#pragma unroll
        for (int a = 0; a < NJT; ++a) av[(kk + 1) & 1][a] = xs[b][4 * (kk + 1) + lk][16 * a + li];
      }
      pin();
#pragma unroll
      for (int a = 0; a < NJT; ++a) {
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[a][t] = mfma4(av[kk & 1][a], bv[kk][t], acc[a][t]);
      }
      pin();
    }
  };
  f4 ba[KK], bb[KK];
  int64_t nb = r0;
  xload(nb);
  yload(nb, ba);
  xstore(0, nb);
  __syncthreads();
  int b = 0;
  while (nb < r1) {
    xload(nb + SR);
    yload(nb + SR, bb);
    pin();
    if (active) stage(b, ba);
    xstore(b ^ 1, nb + SR);
    __syncthreads();
    b ^= 1;
    nb += SR;
    if (nb >= r1) break;
    xload(nb + SR);
    yload(nb + SR, ba);
    pin();
    if (active) stage(b, bb);
    xstore(b ^ 1, nb + SR);
    __syncthreads();
    b ^= 1;
    nb += SR;
  }
  if (!active) return;
  // D[i][m] of tile t: row j0 + 16a + 4lk + r, column cw + 4*li + t
  float* part = P.part + (static_cast<int64_t>(blockIdx.x) * P.g + g) * P.jr * P.c;
#pragma unroll
  for (int a = 0; a < NJT; ++a) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int jj = j0 + 16 * a + 4 * lk + r;
      if (jj < P.jr) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (cl + t < P.c) part[static_cast<int64_t>(jj) * P.c + cl + t] = acc[a][t][r];
      }
    }
  }
}

// ----- wgrad on the bf16 matrix cores -----------------------------------------------------
// The same product with every fp32 operand split into three bf16 parts whose sum is the
// operand exactly (hi = bf16(x), mid = bf16(x - hi), lo = x - hi - mid: 8 + 8 + 8 bits of
// the 24-bit significand), multiplied as the six part products whose order is at most
// 2^-16 of the whole (hi.hi, hi.mid, mid.hi, hi.lo, lo.hi, mid.mid) on MFMA 16x16x32 bf16
// with fp32 accumulation. The three products left out are below 2^-24 of |x y| together,
// the size of the rounding of one fp32 product, and six bf16 products cost less than half
// the matrix-core time of one fp32 product.
//   MFMA 16x16x32 bf16, lane l: A[l%16][8*(l/16) + s], B[8*(l/16) + s][l%16] (s < 8, the
//   same k for A and B), D[4*(l/16)+r][l%16].
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef float fl2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(fl2_t{a, b}, bf2_t));
}
__device__ __forceinline__ float bf16_low(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_high(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats as three bf16 pairs (hi, mid, lo) with x = hi + mid + lo per element.
__device__ __forceinline__ void split3(float x0, float x1, uint32_t (&part)[3]) {
  part[0] = pack_bf16(x0, x1);
  const float r0 = x0 - bf16_low(part[0]), r1 = x1 - bf16_high(part[0]);
  part[1] = pack_bf16(r0, r1);
  part[2] = pack_bf16(r0 - bf16_low(part[1]), r1 - bf16_high(part[1]));
}

__device__ __forceinline__ f4 mfma_bf(const u4_t& a, const u4_t& b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, a),
                                                 __builtin_bit_cast(bf8_t, b), c, 0, 0, 0);
}

constexpr int kBfStage = 32;  // rows per stage: one k-block of the bf16 product
constexpr int kBfXp = 40;     // bf16 per LDS row of the transposed X parts (32 rows + 8)

// Column tiles (16 columns) per wave of the split-bf16 wgrad, and waves per workgroup at
// most: 32-column waves small enough (about 110 VGPRs) for four per SIMD.
constexpr int kWbCt = 2;
constexpr int kWbCols = 16 * kWbCt;
#ifndef FA_WB_MAXW
#define FA_WB_MAXW 12
#endif
#ifndef FA_WB_SIMDW
#define FA_WB_SIMDW 3
#endif
constexpr int kWbMaxWaves = FA_WB_MAXW;
// LDS of the split-bf16 wgrad's X stages, and the waves per SIMD it is held to (its launch
// bound): FA_WB_SIMDW (3: about 170 VGPRs a wave), less where the LDS keeps fewer resident
// (asking for more than the LDS allows would void the bound).
constexpr int wgrad_bf_span(int njt) { return njt > 4 ? 128 : 64; }   // j rows of a wave
constexpr int wgrad_bf_lds(int njg, int njt) { return 2 * 3 * wgrad_bf_span(njt) * njg * kBfXp * 2; }
constexpr int wgrad_bf_min_waves(int waves, int njg, int njt) {
  const int per_simd = (160 * 1024 / wgrad_bf_lds(njg, njt)) * waves / 4;
  const int want = njt > 4 ? 2 : FA_WB_SIMDW;   // 128-row waves: about 250 VGPRs
  return per_simd >= want ? want : (per_simd >= 1 ? per_simd : 1);
}

// The workgroup covers NJG j groups of a head (wave jl*NW + w: j group jl, 32 columns; a j
// group is 64 rows, or 128 for a single group of more than four 16-row tiles) so that every
// X element is staged once per workgroup and every Y element is
// fetched from HBM once per workgroup (the NJG waves of one column read it through the L1).
// X staged in LDS already split and transposed, [part][j][row], so a lane's A operand of a
// tile and part is one 16-byte LDS read; each lane's Y values of a stage are eight float2
// rows (rows 8*(l/16) + s, columns cw + 2*(l%16), +1), split in registers into the B
// operands of its two column tiles. Two stages of X and Y are in flight: a stage's
// registers are reloaded with the stage after next as soon as they are consumed (Y split
// into B operands, X stored into LDS).
template <int NJT, int NW, int NJG>
__global__ __launch_bounds__(NJG * NW * kWave, wgrad_bf_min_waves(NJG * NW, NJG, NJT)) void head_wgrad_bf(WgradParams P) {
  constexpr int SR = kBfStage;
  constexpr int CT = kWbCt;
  constexpr int JW = wgrad_bf_span(NJT);       // j rows of a wave
  static_assert(NJT <= 4 || NJG == 1, "128-row j groups come one to a workgroup");
  constexpr int XC = JW * NJG;                 // X columns the workgroup stages
  // X staging: thread t takes column t % XC of the workgroup's j range and the 8-row groups
  // t / XC, t / XC + NT / XC, ... of a stage (written to LDS as one 16-byte run per part)
  constexpr int NT = NJG * NW * kWave;
  constexpr int XG = NT / XC < 4 ? 4 / (NT / XC) : 1;   // 8-row groups per thread
  constexpr int XE = 8 * XG;                   // X elements per thread and stage
  static_assert(NT / XC >= 4 || 4 % (NT / XC) == 0, "X row groups must cover the stage");
  __shared__ __align__(16) uint16_t xp[2][3][XC][kBfXp];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int jl = wave / NW;
  const int per_g = P.njg * P.ncw4;            // j workgroups x column workgroups per head
  const int g = blockIdx.y / per_g;
  const int rem = blockIdx.y - g * per_g;
  const int jw = rem / P.ncw4;
  const int cw = ((rem - jw * P.ncw4) * NW + (wave - jl * NW)) * kWbCols;
  const int jbase = jw * XC;                   // first j of the workgroup
  const int j0 = jbase + JW * jl;              // first j of the wave
  const bool active = cw < P.c && j0 < P.jr;
  const int li = lane & 15, lq = lane >> 4;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * P.rows;
  const int64_t r1 = P.n < r0 + P.rows ? P.n : r0 + P.rows;
  const float* xbase = P.x + g * P.xg;
  const float* ybase = P.y + g * P.yg;
  const int xc = tid % XC;                     // column
  const int xg0 = uniform(tid / XC);           // first 8-row group (XC is a multiple of 64)
  const bool xbusy = xg0 < 4;                  // threads past the stage's four groups idle
  const int xj = jbase + xc;
  const uint32_t xo = xbusy && xj < P.j ? 4u * static_cast<uint32_t>(8 * xg0 * P.ldx + xj) : kOob;
  const uint32_t xrow = 4u * static_cast<uint32_t>(P.ldx);                       // next row
  const uint32_t xgrp = 4u * static_cast<uint32_t>(8 * (NT / XC) * P.ldx);      // next group
  const bool xones = xbusy && xj >= P.j && xj < P.jr;   // this thread's column is the ones row
  const int cl = cw + CT * li;                 // first of this lane's CT B columns
  const uint32_t yo =
      (active && cl < P.c) ? 4u * static_cast<uint32_t>(8 * lq * P.ldy + cl) : kOob;
  const uint32_t ystep = 4u * static_cast<uint32_t>(P.ldy);   // one row
  auto stage_rsrc = [&](const float* base, int64_t nb, int64_t ld, int64_t w) {
    const int64_t rows = r1 - nb < SR ? r1 - nb : SR;
    return rsrc(base + nb * ld, rows > 0 ? 4 * ((rows - 1) * ld + w) : 0);
  };
  // one offset expression per element, no select: a thread without X (column past j, or
  // idle) starts at kOob, and its offsets stay past every range without wrapping (the
  // stage offsets are below 2^31, checked on the host); the thread's groups are all < 4
  auto xload = [&](float (&xv)[XE], int64_t nb) {
    const rsrc_t rx = stage_rsrc(xbase, nb, P.ldx, P.j);
#pragma unroll
    for (int k = 0; k < XG; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[8 * k + e] = ld1(rx, xo + k * xgrp + e * xrow);
  };
  auto xstore = [&](int b, const float (&xv)[XE], int64_t nb) {
    const int64_t left = r1 - nb;
    const int valid = left < SR ? static_cast<int>(left) : SR;
#pragma unroll
    for (int k = 0; k < XG; ++k) {
      const int grp = xg0 + k * (NT / XC);
      if (grp < 4) {
        u4_t part4[3];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const int ra = 8 * grp + e;
          const float va = xo == kOob ? ((xones && ra < valid) ? 1.f : 0.f) : xv[8 * k + e];
          const float vb = xo == kOob ? ((xones && ra + 1 < valid) ? 1.f : 0.f) : xv[8 * k + e + 1];
          uint32_t part[3];
          split3(va, vb, part);
#pragma unroll
          for (int q = 0; q < 3; ++q) part4[q][e / 2] = part[q];
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) *reinterpret_cast<u4_t*>(&xp[b][q][xc][8 * grp]) = part4[q];
      }
    }
  };
  auto yload = [&](f2 (&raw)[8], int64_t nb) {
    const rsrc_t ry = stage_rsrc(ybase, nb, P.ldy, P.c);
#pragma unroll
    for (int s = 0; s < 8; ++s) raw[s] = ld2(ry, yo == kOob ? kOob : yo + s * ystep);
  };
  f4 acc[NJT][CT];
#pragma unroll
  for (int a = 0; a < NJT; ++a)
#pragma unroll
    for (int t = 0; t < CT; ++t) acc[a][t] = f4{0.f, 0.f, 0.f, 0.f};
  float xa[XE], xb[XE];
  f2 ra[8], rb[8];
  xload(xa, r0);
  yload(ra, r0);
  xload(xb, r0 + SR);
  yload(rb, r0 + SR);
  xstore(0, xa, r0);
  __syncthreads();
  int buf = 0;
  auto step = [&](f2 (&rc)[8], float (&xc_)[XE], const float (&xn)[XE], int64_t at) {
    // this stage's B operands: tile t, part q, k-slots s = rows 8*(l/16) + s
    u4_t bp[3][CT];
#pragma unroll
    for (int t = 0; t < CT; ++t) {
#pragma unroll
      for (int s = 0; s < 8; s += 2) {
        uint32_t part[3];
        split3(rc[s][t], rc[s + 1][t], part);
#pragma unroll
        for (int q = 0; q < 3; ++q) bp[q][t][s / 2] = part[q];
      }
    }
    xload(xc_, at + 2 * SR);
    yload(rc, at + 2 * SR);
    pin();
    if (active) {
      // the six part products by A part (A0 x B0..B2, A1 x B0..B1, A2 x B0), each over
      // every (a, t): consecutive products go to different accumulators
#pragma unroll
      for (int qa = 0; qa < 3; ++qa) {
        u4_t ap[NJT];
#pragma unroll
        for (int a = 0; a < NJT; ++a)
          ap[a] = *reinterpret_cast<const u4_t*>(&xp[buf][qa][JW * jl + 16 * a + li][8 * lq]);
#pragma unroll
        for (int qb = 0; qb < 3 - qa; ++qb) {
#pragma unroll
          for (int a = 0; a < NJT; ++a) {
#pragma unroll
            for (int t = 0; t < CT; ++t) acc[a][t] = mfma_bf(ap[a], bp[qb][t], acc[a][t]);
          }
        }
      }
    }
    xstore(buf ^ 1, xn, at + SR);
    __syncthreads();
    buf ^= 1;
  };
  for (int64_t nb = r0; nb < r1; nb += 2 * SR) {
    step(ra, xa, xb, nb);
    if (nb + SR >= r1) break;
    step(rb, xb, xa, nb + SR);
  }
  if (!active) return;
  // D[i][m] of tile t: row j0 + 16a + 4lq + r, column cw + CT*li + t
  float* part = P.part + (static_cast<int64_t>(blockIdx.x) * P.g + g) * P.jr * P.c;
#pragma unroll
  for (int a = 0; a < NJT; ++a) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int jj = j0 + 16 * a + 4 * lq + r;
      if (jj < P.jr) {
#pragma unroll
        for (int t = 0; t < CT; ++t)
          if (cl + t < P.c) part[static_cast<int64_t>(jj) * P.c + cl + t] = acc[a][t][r];
      }
    }
  }
}

// ----- reduce on the bf16 matrix cores ----------------------------------------------------
#ifndef FA_RB_WAVES
#define FA_RB_WAVES 12
#endif
#ifndef FA_RB_MINW
#define FA_RB_MINW 3
#endif
constexpr int kRbWaves = FA_RB_WAVES;  // waves per workgroup (one per CU: W's parts fill LDS)
constexpr int kRbBlock = kRbWaves * kWave;
#ifndef FA_RB_DEPTH
#define FA_RB_DEPTH 4
#endif
constexpr int kRbDepth = FA_RB_DEPTH;  // k-blocks of Y in flight ahead of the one multiplied
constexpr int kRbQuads = 4;    // W quads per thread in flight while W is staged in LDS

// LDS row (bf16) of the split W[g]: the k-blocks, plus 8 so that the rows of a 16-lane read
// start 4 banks apart.
int reduce_bf_row(int c) { return static_cast<int>(round_up(ceil_div(c, 32), kRbDepth)) * 32 + 8; }
size_t reduce_bf_lds_bytes(int j, int c) {
  return static_cast<size_t>(3) * (j + 1) * reduce_bf_row(c) * sizeof(uint16_t);
}

// head_reduce with the split-bf16 product (see head_wgrad_bf): W[g]'s three parts in LDS
// ([part][J+1][cp], row J zero). Each wave streams its 16-row tiles as one sequence of
// (tile, k-block) steps, kRbDepth k-blocks of Y in flight across tile ends; its first loads
// are issued before W is staged. k-slot s
// of lane l stands for column 32kb + 4*(l/16) + s (s < 4) or 32kb + 16 + 4*(l/16) + s - 4,
// so that a lane's A values are two float4 loads whose 16 lanes of a row read 64
// contiguous bytes; W is stored in LDS in that order.
template <int JT>
__global__ __launch_bounds__(kRbBlock, FA_RB_MINW) void head_reduce_bf(ReduceParams P) {
  extern __shared__ __align__(16) uint16_t wlb[];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int g = blockIdx.y;
  const int cp = P.cp, rows = P.j + 1;
  const int li = lane & 15, lq = lane >> 4;
  const float* ybase = P.y + g * P.yg;
  // this wave's 16-row tiles: gw, gw + (all waves), ... with the waves dealt to the
  // workgroups first, so that a launch with fewer tiles than resident waves still spreads
  // them over every CU (and the tiles in flight at one time are neighbours in memory)
  const int64_t gw = static_cast<int64_t>(wave) * gridDim.x + blockIdx.x;
  const int64_t nw_all = static_cast<int64_t>(gridDim.x) * kRbWaves;
  const int64_t t16 = (P.n + 15) / 16;
  const int tiles = gw < t16 ? static_cast<int>((t16 - gw + nw_all - 1) / nw_all) : 0;
  auto tile_row = [&](int t) { return (gw + t * nw_all) * 16; };
  auto tile_end = [&](int64_t n0) { return P.n < n0 + 16 ? P.n : n0 + 16; };
  const int64_t rb = tile_row(0);
  const uint32_t yrow = 4u * static_cast<uint32_t>(li * P.ldy);
  auto range_rsrc = [&](int t) {
    if (t >= tiles) return rsrc(ybase, 0);   // past the wave's last tile: reads zeros
    const int64_t n0 = tile_row(t);
    const int64_t left = tile_end(n0) - n0;
    const int64_t rr = left < 16 ? left : 16;
    return rsrc(ybase + (rr > 0 ? n0 : 0) * P.ldy, rr > 0 ? 4 * ((rr - 1) * P.ldy + P.c) : 0);
  };
  // load cursor: tile lt, k-block lk (wave-uniform)
  int lt = 0, lk = 0;
  rsrc_t lr = range_rsrc(0);
  auto ly = [&](f4 (&v)[2]) {
    const int c0 = 32 * lk + 4 * lq, c1 = c0 + 16;
    const bool in = lt < tiles;
    const uint32_t o0 = in && c0 < P.c ? yrow + 4u * c0 : kOob;
    const uint32_t o1 = in && c1 < P.c ? yrow + 4u * c1 : kOob;
    v[0] = ld4(lr, o0);
    v[1] = ld4(lr, o1);
    if (++lk == P.kb) {
      lk = 0;
      ++lt;
      lr = range_rsrc(lt);
    }
  };
  // issued in order: ya[0] is the oldest; kRbDepth k-blocks in flight
  f4 ya[kRbDepth][2];
#pragma unroll
  for (int d = 0; d < kRbDepth; ++d) {
    ly(ya[d]);
    pin();
  }
  const float* w = P.w + g * P.wg;
  {
    // W[g] in quads of LDS columns: LDS columns 4i..4i+3 of a row hold four consecutive
    // columns of W (k-slots 0-3 or 4-7 of one lane group), so each quad is four loads issued
    // together and one 8-byte LDS store per part; kRbQuads quads per thread in flight.
    const int cq = cp >> 2, quads = rows * cq;
    for (int q0 = tid; q0 < quads; q0 += kRbBlock * kRbQuads) {
      float v[kRbQuads][4];
#pragma unroll
      for (int u = 0; u < kRbQuads; ++u) {
        const int i = q0 + u * kRbBlock;
        const int jr = i / cq, cc = 4 * (i - jr * cq);
        const int src = 32 * (cc >> 5) + ((cc & 4) ? 16 : 0) + 4 * ((cc >> 3) & 3);
        const bool ok = i < quads && jr < P.j && cc < 32 * P.kb && src < P.c;
        const float* wp = w + static_cast<int64_t>(ok ? jr : 0) * P.ldw + (ok ? src : 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = ok ? wp[e] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kRbQuads; ++u) {
        const int i = q0 + u * kRbBlock;
        if (i < quads) {
          const int jr = i / cq, cc = 4 * (i - jr * cq);
          uint32_t lo[3], hi[3];
          split3(v[u][0], v[u][1], lo);
          split3(v[u][2], v[u][3], hi);
#pragma unroll
          for (int pp = 0; pp < 3; ++pp)
            *reinterpret_cast<uint2*>(&wlb[(pp * rows + jr) * cp + cc]) = make_uint2(lo[pp], hi[pp]);
        }
      }
    }
  }
  __syncthreads();
  int wrow[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) wrow[jt] = (16 * jt + li < P.j ? 16 * jt + li : P.j) * cp + 8 * lq;
  const int plane = rows * cp;
  f4 acc[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) acc[jt] = f4{0.f, 0.f, 0.f, 0.f};
  auto mm = [&](int kb, const f4 (&v)[2]) {
    u4_t ap[3];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        uint32_t part[3];
        split3(v[h][e], v[h][e + 1], part);
#pragma unroll
        for (int pp = 0; pp < 3; ++pp) ap[pp][2 * h + e / 2] = part[pp];
      }
    }
    u4_t bp[3][JT];
#pragma unroll
    for (int pp = 0; pp < 3; ++pp)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
        bp[pp][jt] = *reinterpret_cast<const u4_t*>(&wlb[pp * plane + wrow[jt] + 32 * kb]);
    constexpr int kPa[6] = {0, 0, 1, 0, 2, 1};
    constexpr int kPb[6] = {0, 1, 0, 2, 0, 1};
#pragma unroll
    for (int q = 0; q < 6; ++q) {
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[jt] = mfma_bf(ap[kPa[q]], bp[kPb[q]][jt], acc[jt]);
    }
  };
  int kb = 0, ct = 0;
  int64_t n0 = rb;
  const int steps = tiles * P.kb;   // a multiple of kRbDepth (P.kb is)
  for (int st = 0; st < steps; st += kRbDepth) {
#pragma unroll
    for (int d = 0; d < kRbDepth; ++d) {
      mm(kb + d, ya[d]);
      pin();
      ly(ya[d]);
      pin();
    }
    kb += kRbDepth;
    if (kb == P.kb) {
      // D row 4lq + r of the tile, column 16jt + li
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const int jj = 16 * jt + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t row = n0 + 4 * lq + r;
          if (jj < P.j && row < tile_end(n0)) P.z[row * P.ldz + g * P.zg + jj] = acc[jt][r];
        }
        acc[jt] = f4{0.f, 0.f, 0.f, 0.f};
      }
      kb = 0;
      n0 = tile_row(++ct);
    }
  }
}

// ----- proj on the bf16 matrix cores ------------------------------------------------------
constexpr int kPbWaves = 8;                  // waves per workgroup (48 columns each)
constexpr int kPbBlock = kPbWaves * kWave;
constexpr int kPbCt = 3;                     // 16-column tiles per wave
#ifndef FA_PB_ROWS
#define FA_PB_ROWS 32
#endif
constexpr int kPbRows = FA_PB_ROWS;          // rows per workgroup step (one LDS sync each)
constexpr int kPbXp = 72;                    // bf16 per LDS row of the split X: 64 j + 8

// head_proj with the split-bf16 product (see head_wgrad_bf), formed transposed as head_proj:
// Y^T tile = W^T (A: W's three parts for the wave's 48 columns and KB k-blocks of 32 j, in
// registers for the whole kernel) times X^T (B: the tile's X rows, split into parts in LDS,
// [part][row][j]). The bias rides in the product as row J of W^T against an X column of
// ones. Each lane ends with four consecutive columns of one row and stores one float4.
template <int KB, bool BIAS>
__global__ __launch_bounds__(kPbBlock, 2) void head_proj_bf(ProjParams P) {
  __shared__ __align__(16) uint16_t xp[2][3][kPbRows][kPbXp];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = uniform(tid / kWave);
  const int g = blockIdx.y / P.ncg4;
  const int c0 = ((blockIdx.y - g * P.ncg4) * kPbWaves + wave) * (16 * kPbCt);
  const bool active = c0 < P.c;                         // idle waves still stage X
  const int li = lane & 15, lq = lane >> 4;
  const float* w = P.w + g * P.wg;
  // A operands: tile t, k-block kb, part q; k-slot s of lane l is j = 32kb + 8*(l/16) + s
  u4_t wa[3][kPbCt][KB];
#pragma unroll
  for (int t = 0; t < kPbCt; ++t) {
    const int cc = c0 + 16 * t + li;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int s = 0; s < 8; s += 2) {
        float v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int jj = 32 * kb + 8 * lq + s + e;
          v[e] = 0.f;
          if (active && cc < P.c) {
            if (jj < P.j) v[e] = w[jj * P.ldw + cc];
            else if (BIAS && jj == P.j) v[e] = P.bias[g * P.bg + cc];
          }
        }
        uint32_t part[3];
        split3(v[0], v[1], part);
#pragma unroll
        for (int q = 0; q < 3; ++q) wa[q][t][kb][s / 2] = part[q];
      }
    }
  }
  // output of tile t: columns cb .. cb+3 (cb = c0 + 16t + 4lq) of row n0 + li
  uint32_t yo[kPbCt];
#pragma unroll
  for (int t = 0; t < kPbCt; ++t) {
    const int cb = c0 + 16 * t + 4 * lq;
    yo[t] = (active && cb < P.c) ? 4u * static_cast<uint32_t>(li * P.ldy + cb) : kOob;
  }
  // X elements of this thread: column `lane` of the step rows wave + kPbWaves*i; columns
  // J .. 32KB hold the ones column (with a bias) and zeros
  constexpr int XE = kPbRows / kPbWaves;
  const bool xin = lane < P.j;
  const float xpad = (BIAS && lane == P.j) ? 1.f : 0.f;
  const uint32_t xo = xin ? 4u * static_cast<uint32_t>(wave * P.ldx + lane) : kOob;
  const uint32_t xstep = 4u * static_cast<uint32_t>(kPbWaves * P.ldx);
  const float* xbase = P.x + g * P.xg;
  float* ybase = P.y + g * P.yg;
  const int64_t steps = (P.n + kPbRows - 1) / kPbRows;
  float xv[XE];
  auto gload = [&](int64_t step) {
    const int64_t n0 = step * kPbRows;
    const int64_t rows = P.n - n0 < kPbRows ? P.n - n0 : kPbRows;
    const rsrc_t rx = rsrc(xbase + n0 * P.ldx, rows > 0 ? 4 * ((rows - 1) * P.ldx + P.j) : 0);
#pragma unroll
    for (int i = 0; i < XE; ++i) xv[i] = ld1(rx, xo == kOob ? kOob : xo + i * xstep);
  };
  auto lstore = [&](int b) {
#pragma unroll
    for (int i = 0; i < XE; i += 2) {
      uint32_t part[3];
      split3(xin ? xv[i] : xpad, xin ? xv[i + 1] : xpad, part);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        xp[b][q][wave + kPbWaves * i][lane] = static_cast<uint16_t>(part[q] & 0xffffu);
        xp[b][q][wave + kPbWaves * (i + 1)][lane] = static_cast<uint16_t>(part[q] >> 16);
      }
    }
  };
  // the k-blocks past 64 j (KB = 3: j = 64 with the bias row) read LDS columns 64 .. 95,
  // which this layout does not hold: KB is at most 2 here
  static_assert(KB <= 2, "head_proj_bf covers j + bias <= 64");
  int64_t step = blockIdx.x;
  gload(step);
  lstore(0);
  __syncthreads();
  int b = 0;
  constexpr int kPa[6] = {0, 0, 1, 0, 2, 1};
  constexpr int kPb[6] = {0, 1, 0, 2, 0, 1};
  for (; step < steps; step += gridDim.x) {
    gload(step + gridDim.x);
    pin();
    if (active) {
#pragma unroll
      for (int rt = 0; rt < kPbRows / 16; ++rt) {
        u4_t xb[3][KB];
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
            xb[q][kb] = *reinterpret_cast<const u4_t*>(&xp[b][q][16 * rt + li][32 * kb + 8 * lq]);
        f4 acc[kPbCt];
#pragma unroll
        for (int t = 0; t < kPbCt; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pr = 0; pr < 6; ++pr) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int t = 0; t < kPbCt; ++t)
              acc[t] = mfma_bf(wa[kPa[pr]][t][kb], xb[kPb[pr]][kb], acc[t]);
          }
        }
        const rsrc_t ry = tile_rsrc(ybase, P.n, step * kPbRows + 16 * rt, P.ldy, P.c);
#pragma unroll
        for (int t = 0; t < kPbCt; ++t) st4(ry, yo[t], acc[t]);
      }
    }
    lstore(b ^ 1);
    __syncthreads();
    b ^= 1;
  }
}

// out[i] = sum over chunks k of part[k*stride + i], in chunk order: 32 outputs per
// workgroup, 8 threads per output each summing every 8th chunk, then the 8 partial sums
// in order through LDS.
__global__ __launch_bounds__(kBlock) void chunk_sums(const float* part, int chunks, int64_t stride,
                                                     float* out) {
  __shared__ float red[8][33];
  const int o = threadIdx.x & 31, kg = threadIdx.x >> 5;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 32 + o;
  float s = 0.f;
  if (i < stride)
    for (int k = kg; k < chunks; k += 8) s += part[k * stride + i];
  red[kg][o] = s;
  __syncthreads();
  if (kg == 0 && i < stride) {
    float t = red[0][o];
#pragma unroll
    for (int q = 1; q < 8; ++q) t += red[q][o];
    out[i] = t;
  }
}

// The same, four consecutive outputs per thread (stride and out 16-byte aligned, stride a
// multiple of 4): 32 outputs per workgroup (8 threads of float4), 32 threads per output
// each summing every 32nd chunk, then the 32 partial sums in order through LDS.
constexpr int kSumOut4 = 8;                  // float4 outputs per workgroup
constexpr int kSumGroups = kBlock / kSumOut4;  // chunk groups

__global__ __launch_bounds__(kBlock) void chunk_sums4(const float* part, int chunks, int64_t stride,
                                                      float* out) {
  __shared__ float4 red[kSumGroups][kSumOut4];
  const int o = threadIdx.x % kSumOut4, kg = threadIdx.x / kSumOut4;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * kSumOut4 + o) * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < stride)
    for (int k = kg; k < chunks; k += kSumGroups) {
      const float4 v = *reinterpret_cast<const float4*>(part + k * stride + i);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
  red[kg][o] = s;
  __syncthreads();
  if (kg == 0 && i < stride) {
    float4 t = red[0][o];
    for (int q = 1; q < kSumGroups; ++q) {
      const float4 v = red[q][o];
      t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
    }
    *reinterpret_cast<float4*>(out + i) = t;
  }
}

constexpr int kGemmBlocks = 1024;  // workgroups of the row-tile launches
constexpr size_t kMaxReduceLds = 160 * 1024;
#ifndef FA_PROJ_BF
#define FA_PROJ_BF 1
#endif
constexpr bool kProjBf = FA_PROJ_BF != 0;  // proj on the split-bf16 kernel (j + bias <= 64)
#ifndef FA_REDUCE_BF
#define FA_REDUCE_BF 1
#endif
constexpr bool kReduceBf = FA_REDUCE_BF != 0;  // reduce on the split-bf16 kernel where it fits

// Byte offsets inside a 16-row tile stay below the out-of-range marker.
bool tile_fits(int64_t ld) { return ld >= 0 && 17 * ld * 4 < static_cast<int64_t>(kOob); }

// Workgroups per grid row of the persistent proj launch: the resident workgroups shared
// out over the grid rows, at most one per step of 16*kProjRt rows.
int row_grid(int64_t n, int per_tile_groups, const void* kernel) {
  const int64_t tiles = ceil_div(n, 16 * kProjRt);
  const int64_t want = resident_blocks(kernel, 0) / (per_tile_groups > 0 ? per_tile_groups : 1);
  const int64_t g = tiles < want ? tiles : want;
  return static_cast<int>(g < 1 ? 1 : g);
}

#ifndef FA_WGRAD_MIN_ROWS
#define FA_WGRAD_MIN_ROWS 64
#endif
constexpr int kWgradMinRows = FA_WGRAD_MIN_ROWS;  // rows of a wgrad chunk, at least

// Chunks of the wgrad reduction: one per resident workgroup row (the launch runs in one
// round, with no tail of late workgroups), at least kWgradMinRows rows each.
int64_t wgrad_chunks(int64_t n, int groups, int64_t resident) {
  int64_t chunks = resident / (groups > 0 ? groups : 1);
  if (chunks < 1) chunks = 1;
  const int64_t by_rows = ceil_div(n, kWgradMinRows);
  return chunks < by_rows ? chunks : (by_rows < 1 ? 1 : by_rows);
}

// Waves per wgrad workgroup: the 64-column waves a head needs, shared out evenly over at
// most 4 per workgroup (no idle waves for C = 100, 376, 708, ...).
int wgrad_waves(int c) {
  const int ncw = static_cast<int>(ceil_div(c, kWcols));
  return static_cast<int>(ceil_div(ncw, ceil_div(ncw, kWavesPerBlock)));
}

// Workgroup rows of a wgrad launch: groups x 64-row j groups x column workgroups.
int wgrad_groups(int j, int c, int groups, int ones) {
  const int jr = j + (ones ? 1 : 0);
  const int ncwg = static_cast<int>(ceil_div(ceil_div(c, kWcols), wgrad_waves(c)));
  return groups * static_cast<int>(ceil_div(jr, 64)) * ncwg;
}

using WgradKernel = void (*)(WgradParams);

// The wgrad kernel for njt 16-row j tiles, nw waves per workgroup and X read xv floats
// at a time (1 with scalar-column Y).
WgradKernel wgrad_kernel(int njt, int nw, bool vec, int xv) {
#define FA_WG_NW(NJ, NWV)                                                                  \
  if (njt == NJ && nw == NWV) {                                                            \
    if (!vec) return head_wgrad<NJ, false, NWV, 1>;                                        \
    return xv == 4 ? head_wgrad<NJ, true, NWV, 4>                                          \
                   : (xv == 2 ? head_wgrad<NJ, true, NWV, 2> : head_wgrad<NJ, true, NWV, 1>); \
  }
#define FA_WG(NJ) FA_WG_NW(NJ, 1) FA_WG_NW(NJ, 2) FA_WG_NW(NJ, 3) FA_WG_NW(NJ, 4)
  FA_WG(1) FA_WG(2) FA_WG(3) FA_WG(4)
#undef FA_WG
#undef FA_WG_NW
  return nullptr;
}

// The split-bf16 wgrad launch shape: njg 64-row j groups and nw 32-column waves per
// workgroup (nw one of the compiled counts, at least the waves the columns need), njw j
// workgroups and ncwg column workgroups per head, njt 16-row j tiles per wave.
struct WgradBfShape {
  int njg, nw, njw, ncwg, njt;
};

WgradBfShape wgrad_bf_shape(int jr, int c) {
  WgradBfShape s;
  const int jg = static_cast<int>(ceil_div(jr, 64));
  const bool wide = jg == 2;   // 65..128 rows: one 128-row j group (5 to 8 tiles a wave)
  s.njg = wide ? 1 : (jg < 4 ? jg : 4);
  s.njw = wide ? 1 : static_cast<int>(ceil_div(jg, s.njg));
  const int ncw = static_cast<int>(ceil_div(c, kWbCols));
  // column-wave counts compiled (128-row groups: 4 or 8, two waves per SIMD)
  static const int kCounts[] = {2, 4, 6, 8, 12};
  static const int kWideCounts[] = {4, 4, 8, 8, 8};
  const int* counts = wide ? kWideCounts : kCounts;
  int cap = 0;   // the most column waves a workgroup of njg j groups takes
  for (int i = 0; i < 5; ++i)
    if (counts[i] * s.njg <= kWbMaxWaves) cap = counts[i];
  s.ncwg = static_cast<int>(ceil_div(ncw, cap));
  const int need = static_cast<int>(ceil_div(ncw, s.ncwg));
  s.nw = cap;
  for (int i = 0; i < 5; ++i)
    if (counts[i] >= need && counts[i] < s.nw) s.nw = counts[i];
  s.njt = jg == 1 || wide ? static_cast<int>(ceil_div(jr, 16)) : 4;
  return s;
}

// The split-bf16 wgrad kernel for a launch shape.
WgradKernel wgrad_bf_kernel(const WgradBfShape& s) {
#define FA_WGB(NJ, NWV, NG) \
  if (s.njt == NJ && s.nw == NWV && s.njg == NG) return head_wgrad_bf<NJ, NWV, NG>;
#define FA_WGB1(NJ) FA_WGB(NJ, 2, 1) FA_WGB(NJ, 4, 1) FA_WGB(NJ, 6, 1) FA_WGB(NJ, 8, 1) \
  FA_WGB(NJ, 12, 1)
  FA_WGB1(1) FA_WGB1(2) FA_WGB1(3) FA_WGB1(4)
  FA_WGB(5, 4, 1) FA_WGB(5, 8, 1) FA_WGB(6, 4, 1) FA_WGB(6, 8, 1)
  FA_WGB(7, 4, 1) FA_WGB(7, 8, 1) FA_WGB(8, 4, 1) FA_WGB(8, 8, 1)
  FA_WGB(4, 2, 2) FA_WGB(4, 4, 2) FA_WGB(4, 6, 2)
  FA_WGB(4, 2, 3) FA_WGB(4, 4, 3)
  FA_WGB(4, 2, 4)
#undef FA_WGB1
#undef FA_WGB
  return nullptr;
}

int wgrad_njt(int jr) {
  return jr > 64 ? 4 : static_cast<int>(ceil_div(jr, 16));
}

#ifndef FA_WGRAD_BF
#define FA_WGRAD_BF 1
#endif
// Y blocks with 16-byte rows go to the split-bf16 kernel
constexpr bool kWgradBf = FA_WGRAD_BF != 0;

// Row chunks of a wgrad launch: the resident workgroups of its kernel (the fp32 kernel with
// 16-byte Y rows and single X loads, or the split-bf16 one), shared out over the workgroup
// rows.
int64_t wgrad_plan_chunks(int64_t n, int j, int c, int groups, int ones, bool bf) {
  const int jr = j + (ones ? 1 : 0);
  if (bf) {
    const WgradBfShape s = wgrad_bf_shape(jr, c);
    const WgradKernel k = wgrad_bf_kernel(s);
    const int64_t resident =
        k ? resident_blocks(reinterpret_cast<const void*>(k), 0, s.njg * s.nw * kWave) : 1;
    int64_t chunks = wgrad_chunks(n, groups * s.njw * s.ncwg, resident);
    // a multiple of the 8 XCDs (workgroups go to XCDs in turn by linear id), so that the
    // workgroups of one chunk (its heads, j and column blocks, which read the same rows)
    // share one XCD's L2
    if (chunks >= 16) chunks -= chunks % 8;
    return chunks;
  }
  const int nw = wgrad_waves(c);
  const WgradKernel k = wgrad_kernel(wgrad_njt(jr), nw, true, 1);
  const int64_t resident =
      k ? resident_blocks(reinterpret_cast<const void*>(k), 0, nw * kWave) : 1;
  return wgrad_chunks(n, wgrad_groups(j, c, groups, ones), resident);
}

void launch_proj(void (*k)(ProjParams), int64_t n, int gy, const ProjParams& P,
                 hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(row_grid(n, gy, reinterpret_cast<const void*>(k))),
                  static_cast<unsigned>(gy));
  hipLaunchKernelGGL(k, grid, dim3(kBlock), 0, stream, P);
}

}  // namespace
}  // namespace fa

using namespace fa;

extern "C" int fa_head_proj_f32(int64_t n, int32_t j, int32_t c, int32_t groups, const float* x,
                                int64_t ldx, int64_t xg, const float* w, int64_t wg, int64_t ldw,
                                const float* bias, int64_t bg, float* y, int64_t yg, int64_t ldy,
                                hipStream_t stream) {
  if (n < 0 || j <= 0 || c <= 0 || groups <= 0 || j > 64) return j > 64 ? FA_EUNSUPPORTED : FA_EINVAL;
  if (n == 0) return FA_OK;
  if (!x || !w || !y || ldx < j || ldw < c || ldy < c) return FA_EINVAL;
  if (!tile_fits(ldx) || !tile_fits(ldy)) return FA_EUNSUPPORTED;
  ProjParams P;
  P.n = n; P.j = j; P.c = c; P.g = groups;
  P.x = x; P.ldx = ldx; P.xg = xg; P.w = w; P.wg = wg; P.ldw = ldw;
  P.bias = bias; P.bg = bg; P.y = y; P.yg = yg; P.ldy = ldy;
  P.vec = aligned16(y) && !(ldy & 3) && !(yg & 3) && !(c & 3);
  const int jb = j + (bias ? 1 : 0);   // k rows with the bias row
  if (kProjBf && P.vec && jb <= 64) {
    // split-bf16 kernel: 8 waves of 48 columns per workgroup
    P.ncg4 = static_cast<int>(ceil_div(ceil_div(c, 16 * kPbCt), kPbWaves));
    const int gyb = groups * P.ncg4;
    void (*k)(ProjParams) = nullptr;
    if (jb <= 32) k = bias ? head_proj_bf<1, true> : head_proj_bf<1, false>;
    else k = bias ? head_proj_bf<2, true> : head_proj_bf<2, false>;
    const int64_t steps = ceil_div(n, kPbRows);
    int64_t gx = resident_blocks(reinterpret_cast<const void*>(k), 0, kPbBlock) / gyb;
    if (gx > steps) gx = steps;
    if (gx < 1) gx = 1;
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gyb)),
                       dim3(kPbBlock), 0, stream, P);
    return launch_status();
  }
  const int ncg = static_cast<int>(ceil_div(c, 16 * kProjCt));
  P.ncg4 = static_cast<int>(ceil_div(ncg, kWavesPerBlock));
  const int gy = groups * P.ncg4;
  switch (static_cast<int>(ceil_div(j, 4))) {
#define FA_PROJ_CASE(K)                                                                    \
  case K:                                                                                  \
    if (bias && P.vec)                                                                     \
      launch_proj(head_proj<K, kProjCt, true, true>, n, gy, P, stream);                    \
    else if (bias)                                                                         \
      launch_proj(head_proj<K, kProjCt, true, false>, n, gy, P, stream);                   \
    else if (P.vec)                                                                        \
      launch_proj(head_proj<K, kProjCt, false, true>, n, gy, P, stream);                   \
    else                                                                                   \
      launch_proj(head_proj<K, kProjCt, false, false>, n, gy, P, stream);                  \
    break;
    FA_PROJ_CASE(1) FA_PROJ_CASE(2) FA_PROJ_CASE(3) FA_PROJ_CASE(4) FA_PROJ_CASE(5)
    FA_PROJ_CASE(6) FA_PROJ_CASE(7) FA_PROJ_CASE(8) FA_PROJ_CASE(9) FA_PROJ_CASE(10)
    FA_PROJ_CASE(11) FA_PROJ_CASE(12) FA_PROJ_CASE(13) FA_PROJ_CASE(14) FA_PROJ_CASE(15)
    FA_PROJ_CASE(16)
#undef FA_PROJ_CASE
    default: return FA_EUNSUPPORTED;
  }
  return launch_status();
}

// Which path a head_reduce call would take (0: none, FA_EUNSUPPORTED; 1: the float32 kernel;
// 2: the split-bf16 kernel), from the same tests fa_head_reduce_f32 makes.
static int head_reduce_path(int32_t j, int32_t c, int64_t ldy, bool vec) {
  if (j <= 0 || c <= 0 || j > 64 || ldy < c || !tile_fits(ldy)) return 0;
  if (kReduceBf && vec && reduce_bf_lds_bytes(j, c) <= kMaxReduceLds) return 2;
  const int c16 = static_cast<int>(round_up(ceil_div(c, 16), kRedDepth));
  return reduce_lds_bytes(j, c16) <= kMaxReduceLds ? 1 : 0;
}

extern "C" int fa_head_reduce_supported(int32_t j, int32_t c, int64_t ldy, int32_t rows16) {
  return head_reduce_path(j, c, ldy, rows16 != 0);
}

extern "C" int fa_head_reduce_f32(int64_t n, int32_t j, int32_t c, int32_t groups,
                                  const float* y, int64_t yg, int64_t ldy, const float* w,
                                  int64_t wg, int64_t ldw, float* z, int64_t ldz, int64_t zg,
                                  hipStream_t stream) {
  if (n < 0 || j <= 0 || c <= 0 || groups <= 0) return FA_EINVAL;
  if (j > 64) return FA_EUNSUPPORTED;
  if (n == 0) return FA_OK;
  if (!y || !w || !z || ldy < c || ldw < c || ldz < 0 || zg < 0) return FA_EINVAL;
  if (!tile_fits(ldy)) return FA_EUNSUPPORTED;
  ReduceParams P;
  P.n = n; P.j = j; P.c = c; P.g = groups;
  P.y = y; P.yg = yg; P.ldy = ldy; P.w = w; P.wg = wg; P.ldw = ldw;
  P.z = z; P.ldz = ldz; P.zg = zg;
  P.c16 = static_cast<int>(round_up(ceil_div(c, 16), kRedDepth));
  const bool vec = aligned16(y) && !(ldy & 3) && !(yg & 3) && !(c & 3);
  // 16-byte Y rows go to the split-bf16 kernel when W's three parts fit in LDS
  if (kReduceBf && vec && reduce_bf_lds_bytes(j, c) <= kMaxReduceLds) {
    P.kb = static_cast<int>(round_up(ceil_div(c, 32), kRbDepth));
    P.cp = reduce_bf_row(c);
    const size_t lds = reduce_bf_lds_bytes(j, c);
    void (*k)(ReduceParams) = nullptr;
    switch (static_cast<int>(ceil_div(j, 16))) {
      case 1: k = head_reduce_bf<1>; break;
      case 2: k = head_reduce_bf<2>; break;
      case 3: k = head_reduce_bf<3>; break;
      default: k = head_reduce_bf<4>; break;
    }
    const void* kp = reinterpret_cast<const void*>(k);
    if (hipFuncSetAttribute(kp, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return launch_status();
    const int64_t tiles = ceil_div(n, 16);
    int64_t gx = resident_blocks(kp, lds, kRbBlock) / groups;
    // heads that share Y rows: a multiple of the 8 XCDs, so that the workgroups of one grid
    // column (the same tiles) run on one XCD and its L2 serves the other heads' reads
    if (groups > 1 && gx >= 16) gx -= gx % 8;
    if (gx > tiles) gx = tiles;
    if (gx < 1) gx = 1;
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(groups)),
                       dim3(kRbBlock), lds, stream, P);
    return launch_status();
  }
  const size_t lds = reduce_lds_bytes(j, P.c16);
  if (lds > kMaxReduceLds) return FA_EUNSUPPORTED;
  void (*k)(ReduceParams) = nullptr;
  switch (static_cast<int>(ceil_div(j, 16))) {
    case 1: k = vec ? head_reduce<1, true> : head_reduce<1, false>; break;
    case 2: k = vec ? head_reduce<2, true> : head_reduce<2, false>; break;
    case 3: k = vec ? head_reduce<3, true> : head_reduce<3, false>; break;
    default: k = vec ? head_reduce<4, true> : head_reduce<4, false>; break;
  }
  const void* kp = reinterpret_cast<const void*>(k);
  if (hipFuncSetAttribute(kp, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(lds)) != hipSuccess)
    return launch_status();
  const int64_t tiles = ceil_div(n, 16);
  int64_t gx = resident_blocks(kp, lds, kRedBlock) / groups;
  if (gx > ceil_div(tiles, kRedWaves)) gx = ceil_div(tiles, kRedWaves);
  if (gx < 1) gx = 1;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(groups)),
                     dim3(kRedBlock), lds, stream, P);
  return launch_status();
}

extern "C" size_t fa_head_wgrad_scratch_bytes(int64_t n, int32_t j, int32_t c, int32_t groups,
                                              int32_t ones) {
  if (n <= 0 || j <= 0 || c <= 0 || groups <= 0) return 0;
  const int jr = j + (ones ? 1 : 0);
  // enough for either kernel (which one runs depends on the alignment of Y)
  int64_t chunks = wgrad_plan_chunks(n, j, c, groups, ones, false);
  if (kWgradBf && !(c & 3) && wgrad_waves(c) >= 2) {
    const int64_t bf = wgrad_plan_chunks(n, j, c, groups, ones, true);
    chunks = bf > chunks ? bf : chunks;
  }
  return static_cast<size_t>(chunks) * groups * jr * c * sizeof(float);
}

extern "C" int fa_head_wgrad_f32(int64_t n, int32_t j, int32_t c, int32_t groups,
                                 const float* x, int64_t ldx, int64_t xg, const float* y,
                                 int64_t yg, int64_t ldy, int32_t ones, float* dw,
                                 void* scratch, size_t scratch_bytes, hipStream_t stream) {
  if (n < 0 || j <= 0 || c <= 0 || groups <= 0 || !dw) return FA_EINVAL;
  const int jr = j + (ones ? 1 : 0);
  const int64_t out = static_cast<int64_t>(groups) * jr * c;
  if (n == 0) {
    hipLaunchKernelGGL(fill_zero, dim3(static_cast<unsigned>(ceil_div(out, kBlock))), dim3(kBlock),
                       0, stream, dw, out);
    return launch_status();
  }
  if (!x || !y || ldx < j || ldy < c) return FA_EINVAL;
  WgradParams P;
  P.n = n; P.j = j; P.c = c; P.g = groups; P.jr = jr;
  P.x = x; P.ldx = ldx; P.xg = xg; P.y = y; P.yg = yg; P.ldy = ldy;
  P.vec = aligned16(y) && !(ldy & 3) && !(yg & 3) && !(c & 3);
  const int nw = wgrad_waves(c);
  const bool bf = kWgradBf && P.vec && nw >= 2;   // one-wave shapes (c <= 64) stay fp32
  WgradKernel k = nullptr;
  int gy = 0, threads = 0;
  if (bf) {
    const WgradBfShape s = wgrad_bf_shape(jr, c);
    P.ncw4 = s.ncwg;
    P.njg = s.njw;
    gy = groups * s.njw * s.ncwg;
    threads = s.njg * s.nw * kWave;
    k = wgrad_bf_kernel(s);
  } else {
    P.ncw4 = static_cast<int>(ceil_div(ceil_div(c, kWcols), nw));
    P.njg = static_cast<int>(ceil_div(jr, 64));
    gy = wgrad_groups(j, c, groups, ones);
    threads = nw * kWave;
  }
  const int64_t chunks = wgrad_plan_chunks(n, j, c, groups, ones, bf);
  P.rows = round_up(ceil_div(n, chunks), bf ? kBfStage : kWgradStage);
  // byte offsets inside a chunk (and its one-block prefetch) stay below the marker
  if ((P.rows + 64) * (ldx > ldy ? ldx : ldy) * 4 >= static_cast<int64_t>(kOob)) return FA_EUNSUPPORTED;
  // the split-bf16 grid keeps every planned chunk (trailing ones past n add zeros), so that
  // its width stays a multiple of 8
  const int64_t used = bf ? chunks : ceil_div(n, P.rows);
  if (!scratch || scratch_bytes < fa_head_wgrad_scratch_bytes(n, j, c, groups, ones))
    return FA_ESCRATCH;
  P.part = static_cast<float*>(scratch);
  const dim3 grid(static_cast<unsigned>(used), static_cast<unsigned>(gy));
  // X read 4 or 2 floats at a time where j, the strides and the base allow it
  int xv = 1;
  if (!(j & 3) && !(ldx & 3) && !(xg & 3) && aligned16(x))
    xv = 4;
  else if (!(j & 1) && !(ldx & 1) && !(xg & 1) && !(reinterpret_cast<uintptr_t>(x) & 7))
    xv = 2;
  if (!bf) k = wgrad_kernel(wgrad_njt(jr), nw, P.vec != 0, xv);
  if (!k) return FA_EUNSUPPORTED;
  hipLaunchKernelGGL(k, grid, dim3(static_cast<unsigned>(threads)), 0, stream, P);
  if (!(out & 3) && aligned16(dw) && aligned16(scratch)) {
    hipLaunchKernelGGL(chunk_sums4, dim3(static_cast<unsigned>(ceil_div(out, 4 * kSumOut4))), dim3(kBlock), 0,
                       stream, static_cast<const float*>(P.part), static_cast<int>(used), out, dw);
    return launch_status();
  }
  hipLaunchKernelGGL(chunk_sums, dim3(static_cast<unsigned>(ceil_div(out, 32))), dim3(kBlock), 0,
                     stream, static_cast<const float*>(P.part), static_cast<int>(used), out, dw);
  return launch_status();
}
