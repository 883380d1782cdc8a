// Shared device/host helpers for the gfx950 kernels of libfastagg_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <tuple>

#include "fastagg.h"

namespace fa {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kBlock = 256;        // 4 waves per workgroup for the row kernels
constexpr int kWavesPerBlock = kBlock / kWave;

// ---------------------------------------------------------------------------
// Wave64 reductions. Lanes are combined inside each row of 16 with DPP (quad_perm,
// row_half_mirror, row_mirror), then the four row results are read with readlane and
// added in a fixed order, so every lane gets the same, order-deterministic value.
// All 64 lanes must be active.
// ---------------------------------------------------------------------------
namespace dpp {
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
}  // namespace dpp

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<dpp::kQuadSwap1>(v);
  v += dpp_mov<dpp::kQuadSwap2>(v);
  v += dpp_mov<dpp::kRowHalfMirror>(v);
  v += dpp_mov<dpp::kRowMirror>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<dpp::kQuadSwap1>(v));
  v = fmaxf(v, dpp_mov<dpp::kQuadSwap2>(v));
  v = fmaxf(v, dpp_mov<dpp::kRowHalfMirror>(v));
  v = fmaxf(v, dpp_mov<dpp::kRowMirror>(v));
  return v;
}

__device__ __forceinline__ float lane_read(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Cross-row step of a wave reduction: rows 1 and 3 receive lane 15 of the row below
// (row_bcast:15), then rows 2 and 3 receive lane 31 (row_bcast:31); lane 63 then holds
// (S3 + S2) + (S1 + S0) for row results S0..S3.
constexpr int kRowBcast15 = 0x142;
constexpr int kRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_bcast<kRowBcast15, 0xA>(v);
  v += dpp_bcast<kRowBcast31, 0xC>(v);
  return lane_read(v, 63);
}

constexpr int kHalf = 32;  // lanes of a half-wave

// Sum over each half-wave: every lane of rows 1 / 3 ends with its half's total; lanes 31
// and 63 are read back, so the result is uniform per half.
__device__ __forceinline__ float half_sum(float v) {
  v = row16_sum(v);
  v += dpp_bcast<kRowBcast15, 0xA>(v);
  const float s0 = lane_read(v, 31), s1 = lane_read(v, 63);
  return (threadIdx.x & (kWave - 1)) < kHalf ? s0 : s1;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)),
               fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Orders this wave's LDS accesses across lanes (a wave-level barrier with workgroup-scope
// release/acquire fences on LDS only); enough when only this wave touches the LDS region.
// The fences name the local address space: a fence over every address space would also
// wait for the wave's outstanding global loads (s_waitcnt vmcnt(0)), draining every load a
// kernel has put in flight ahead of its use.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Adds a row held as float4 chunks (lane l: columns 4l.. of slot k at 4(l + 64k)) into
// out[0, dim) with atomics issued lane-consecutively (one 256-byte span per instruction),
// transposing through this wave's LDS staging row `stage` (>= 4*64*NS floats).
template <int NS>
__device__ __forceinline__ void atomic_add_row(float* out, int dim, const float4 (&v)[NS],
                                               float* stage) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < NS; ++k)
    *reinterpret_cast<float4*>(stage + 4 * (lane + k * kWave)) = v[k];
  lds_sync();
  for (int c = lane; c < dim; c += kWave) atomicAdd(out + c, stage[c]);
  lds_sync();
}

// Broadcast a wave-uniform integer into a scalar register.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ __forceinline__ float dot4(const float4& a, const float4& b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

__device__ __forceinline__ void fma4(float4& acc, float s, const float4& x) {
  acc.x = fmaf(s, x.x, acc.x);
  acc.y = fmaf(s, x.y, acc.y);
  acc.z = fmaf(s, x.z, acc.z);
  acc.w = fmaf(s, x.w, acc.w);
}

__device__ __forceinline__ void scale4(float4& acc, float s) {
  acc.x *= s;
  acc.y *= s;
  acc.z *= s;
  acc.w *= s;
}

__device__ __forceinline__ float leaky(float z, float slope) { return z > 0.f ? z : z * slope; }

// Time-encoding argument w*t + b with the product and the sum rounded separately,
// matching an unfused multiply followed by an add. HIP's __fmul_rn/__fadd_rn are plain
// operators that -ffp-contract=fast would fuse into one FMA (a different rounding of an
// argument of size ~1e4), so contraction is switched off here.
__device__ __forceinline__ float time_arg(float t, float w, float b) {
#pragma clang fp contract(off)
  return t * w + b;
}

// exp(x) as 2^(x log2 e) on the hardware exp2 (a couple of ulp; used for softmax weights,
// whose arguments are <= 0).
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// sin and cos of x (radians) for |x| <= 2^22 on the hardware sin/cos, whose argument is in
// revolutions: f = x/(2 pi) - k with k = rint(x c_hi), evaluated as
// fma(x, c_lo, fma(x, c_hi, -k)) where c_hi + c_lo = 1/(2 pi) (float32 split); the inner
// FMA forms x c_hi - k exactly before its one rounding, so |f| <= 1/2 carries an error of
// about 3e-8 revolutions. The hardware functions are accurate to about 1.3e-7 absolute on
// [-1/2, 1/2]. Contraction is off: fusing x*c_hi into a later step would change the
// algorithm.
namespace trig {
constexpr float kInvTwoPiHi = 0.15915493667125701904296875f;   // float32(1/(2 pi))
constexpr float kInvTwoPiLo = 6.4206383e-09f;                   // 1/(2 pi) - kInvTwoPiHi
constexpr float kMaxArg = 4194304.0f;                           // 2^22
}  // namespace trig

__device__ __forceinline__ void sincos_hw(float x, float& s, float& c) {
#pragma clang fp contract(off)
  const float k = rintf(x * trig::kInvTwoPiHi);
  const float f = fmaf(x, trig::kInvTwoPiLo, fmaf(x, trig::kInvTwoPiHi, -k));
  s = __builtin_amdgcn_sinf(f);
  c = __builtin_amdgcn_cosf(f);
}

// Counter-based dropout: keep entry i with probability 1-p, decided by a 32-bit hash of
// (seed, i) (two rounds of the murmur3 finaliser). u = top 24 bits / 2^24 in [0, 1);
// kept when u >= p. The same function runs on the host side of the tests.
__host__ __device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  return x;
}

__host__ __device__ inline uint32_t drop_hash(uint64_t seed, uint64_t i) {
  uint32_t x = mix32(static_cast<uint32_t>(i) ^ static_cast<uint32_t>(seed));
  return mix32(x + static_cast<uint32_t>(seed >> 32) + static_cast<uint32_t>(i >> 32) * 0x9e3779b9u);
}

__host__ __device__ inline float drop_mult(uint64_t seed, uint64_t i, float p, float scale) {
  const float u = static_cast<float>(drop_hash(seed, i) >> 8) * (1.0f / 16777216.0f);
  return u >= p ? scale : 0.f;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

namespace {
// Zero fill by a kernel rather than hipMemsetAsync, so the call is safe under graph capture.
__global__ __launch_bounds__(kBlock) void fill_zero(float* p, int64_t n) {
  for (int64_t i = threadIdx.x + static_cast<int64_t>(blockIdx.x) * kBlock; i < n;
       i += static_cast<int64_t>(gridDim.x) * kBlock)
    p[i] = 0.f;
}
}  // namespace

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : static_cast<int>(e);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Workgroups of `kernel` (`block` threads, `lds` bytes of dynamic LDS) that the current
// device holds at once: a grid-stride (persistent) launch of exactly this many runs in
// one round, with no partly filled last round. Cached per (kernel, device, lds).
inline int resident_blocks(const void* kernel, size_t lds, int block = kBlock) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(kernel, dev, lds);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 1;
  (void)hipGetLastError();
  const int n = per_cu * cus;
  cache.emplace(key, n);
  return n;
}

}  // namespace fa
