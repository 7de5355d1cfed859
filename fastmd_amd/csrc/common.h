// Shared helpers of the gfx950 kernels: status codes, launch checks, wave-level reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastmd_hip.h"

#define FMD_WAVE 64

#define FMD_CHECK_LAUNCH()                        \
  do {                                            \
    hipError_t _e = hipGetLastError();            \
    if (_e != hipSuccess) return (int)_e;         \
  } while (0)

#define FMD_REQUIRE(cond)                         \
  do {                                            \
    if (!(cond)) return FMD_EINVAL;               \
  } while (0)

__host__ __device__ static inline int64_t fmd_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// XCD-aware block order: the hardware hands workgroups to the 8 XCDs round-robin (workgroup w to
// XCD w % 8), and each XCD has its own L2. The logical block of workgroup w of g is chosen so
// that every XCD walks one contiguous run of logical blocks (a bijection of [0, g)): blocks that
// read the same rows (neighbouring atoms, the tiles of one GEMM row) then share an L2.
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t fmd_xcd_block(int64_t w, int64_t g) {
  const int64_t xcd = w % kXcds, slot = w / kXcds, q = g / kXcds, r = g % kXcds;
  return xcd * q + (xcd < r ? xcd : r) + slot;
}

// gfx950 cross-lane moves that bypass the LDS crossbar: v_permlane32_swap / v_permlane16_swap
// trade the upper half of every 64 / 32 lanes of one register with the lower half of another, and
// DPP reads a partner lane inside a row of 16 as an operand of the consuming instruction.
__device__ __forceinline__ void swap_halves32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void swap_halves16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

constexpr int kDppQuadXor1 = 0xB1;    // quad_perm [1,0,3,2]: lane l reads l ^ 1
constexpr int kDppQuadXor2 = 0x4E;    // quad_perm [2,3,0,1]: lane l reads l ^ 2
constexpr int kDppRowRor8 = 0x128;    // row_ror:8: lane l reads (l + 8) mod 16 of its row = l ^ 8
constexpr int kDppHalfMirror = 0x141; // row_half_mirror: lane l reads 7 - l of its 8 (bit 2 flips)

template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Wavefront (64 lanes) reductions in a fixed butterfly order: every lane ends with the same
// value, and the order depends on nothing but the lane layout (deterministic). Called with the
// whole wave active.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, FMD_WAVE);
  return v;
}

// float: lanes l and l ^ 32, then l ^ 16 (half swaps of the value with itself), then l ^ 8, the
// mirror lane in 8, l ^ 1 and l ^ 2 (DPP) - 64 lanes in six steps without the LDS crossbar
template <>
__device__ __forceinline__ float wave_sum<float>(float v) {
  float w = v;
  swap_halves32(v, w);
  v = v + w;
  w = v;
  swap_halves16(v, w);
  v = v + w;
  v = v + dpp_read<kDppRowRor8>(v);
  v = v + dpp_read<kDppHalfMirror>(v);
  v = v + dpp_read<kDppQuadXor1>(v);
  v = v + dpp_read<kDppQuadXor2>(v);
  return v;
}

// double: the same six lane moves on both 32-bit halves (the same fixed order; no LDS crossbar)
__device__ __forceinline__ double f64_from(uint32_t lo, uint32_t hi) { return __hiloint2double((int)hi, (int)lo); }

template <int CTRL>
__device__ __forceinline__ double dpp_read_f64(double v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xf, 0xf, false);
  return __hiloint2double(hi, lo);
}

template <>
__device__ __forceinline__ double wave_sum<double>(double v) {
  const uint32_t l0 = (uint32_t)__double2loint(v), h0 = (uint32_t)__double2hiint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(l0, l0, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(h0, h0, false, false);
  v = f64_from(a[0], b[0]) + f64_from(a[1], b[1]);
  const uint32_t l1 = (uint32_t)__double2loint(v), h1 = (uint32_t)__double2hiint(v);
  const auto c = __builtin_amdgcn_permlane16_swap(l1, l1, false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(h1, h1, false, false);
  v = f64_from(c[0], d[0]) + f64_from(c[1], d[1]);
  v = v + dpp_read_f64<kDppRowRor8>(v);
  v = v + dpp_read_f64<kDppHalfMirror>(v);
  v = v + dpp_read_f64<kDppQuadXor1>(v);
  v = v + dpp_read_f64<kDppQuadXor2>(v);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    T o = __shfl_xor(v, off, FMD_WAVE);
    v = o > v ? o : v;
  }
  return v;
}

// Eight wave sums at once: a transposing butterfly (each of the first three exchanges halves the
// value set: a lane keeps one half and adds its partner's copy of it, the partner keeps the other
// half), then a full sum of the last value over the remaining 8 lanes. On return every lane holds
// the total of value index 4*b5 + 2*b4 + b3 (b_i: bit i of the lane), see wave_sum8_index. The
// order of additions is fixed by the lane layout (deterministic).
__device__ __forceinline__ float wave_sum8(const float (&v)[8]) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const bool h3 = lane & 8;
  float a[4], b[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // lanes with bit 5 set keep index i + 4
    float x = v[i], y = v[i + 4];
    swap_halves32(x, y);
    a[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // bit 4 set: index i + 2
    float x = a[i], y = a[i + 2];
    swap_halves16(x, y);
    b[i] = x + y;
  }
  float t = (h3 ? b[1] : b[0]) + dpp_read<kDppRowRor8>(h3 ? b[0] : b[1]);
  t = t + dpp_read<kDppHalfMirror>(t);
  t = t + dpp_read<kDppQuadXor1>(t);
  t = t + dpp_read<kDppQuadXor2>(t);
  return t;
}

__device__ __forceinline__ int wave_sum8_index(int lane) {
  return ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
}

// Sixteen wave sums at once (the same transposing butterfly over four halving exchanges, the
// fourth with the mirror lane in 8, then l ^ 1 and l ^ 2): on return every lane holds the total of
// value index 8*b5 + 4*b4 + 2*b3 + b2 (wave_sum16_index). Fixed order (deterministic).
__device__ __forceinline__ float wave_sum16(const float (&v)[16]) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const bool h3 = lane & 8, h2 = lane & 4;
  float a[8], b[4], c[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // bit 5 set: index i + 8
    float x = v[i], y = v[i + 8];
    swap_halves32(x, y);
    a[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // bit 4 set: index i + 4
    float x = a[i], y = a[i + 4];
    swap_halves16(x, y);
    b[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // bit 3 set: index i + 2 (partner l ^ 8)
    const float keep = h3 ? b[i + 2] : b[i], send = h3 ? b[i] : b[i + 2];
    c[i] = keep + dpp_read<kDppRowRor8>(send);
  }
  // bit 2 set: index 1 (partner: the mirror lane in 8, whose bit 2 is the other)
  float t = (h2 ? c[1] : c[0]) + dpp_read<kDppHalfMirror>(h2 ? c[0] : c[1]);
  t = t + dpp_read<kDppQuadXor1>(t);
  t = t + dpp_read<kDppQuadXor2>(t);
  return t;
}

__device__ __forceinline__ int wave_sum16_index(int lane) {
  return ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
}

// Sixteen sums over each half-wave (lanes 0-31 and 32-63 separately, each reducing its own
// values): the transposing butterfly over l ^ 16 (half swap), l ^ 8 (row_ror:8), the mirror lane
// in 8 and l ^ 2, then a full sum with l ^ 1. On return lanes l and l ^ 1 of a half hold the total
// of value index 8*b4 + 4*b3 + 2*b2 + b1 (half_sum16_index). Fixed order (deterministic).
__device__ __forceinline__ float half_sum16(const float (&v)[16]) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const bool h3 = lane & 8, h2 = lane & 4, h1 = lane & 2;
  float a[8], b[4], c[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // bit 4 set: index i + 8
    float x = v[i], y = v[i + 8];
    swap_halves16(x, y);
    a[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // bit 3 set: index i + 4 (partner l ^ 8)
    const float keep = h3 ? a[i + 4] : a[i], send = h3 ? a[i] : a[i + 4];
    b[i] = keep + dpp_read<kDppRowRor8>(send);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // bit 2 set: index i + 2 (partner: the mirror lane in 8)
    const float keep = h2 ? b[i + 2] : b[i], send = h2 ? b[i] : b[i + 2];
    c[i] = keep + dpp_read<kDppHalfMirror>(send);
  }
  float t = (h1 ? c[1] : c[0]) + dpp_read<kDppQuadXor2>(h1 ? c[0] : c[1]);  // bit 1 set: index 1
  t = t + dpp_read<kDppQuadXor1>(t);
  return t;
}

__device__ __forceinline__ int half_sum16_index(int lane) {
  return ((lane >> 4) & 1) * 8 + ((lane >> 3) & 1) * 4 + ((lane >> 2) & 1) * 2 + ((lane >> 1) & 1);
}

// x of lane l plus x of lane l ^ 32, the same value (same order of the two terms) in both lanes
__device__ __forceinline__ float add_halves(float x) {
  float y = x;
  swap_halves32(x, y);
  return x + y;
}

// Streaming stores (the `nt` bit): outputs written once and not re-read by the same kernel. On
// gfx950 they sustain ~5.9 TB/s for a gather-and-write stream against ~3.4 TB/s for plain
// stores, which keep the lines in L2 and the last-level cache on their way out.
__device__ __forceinline__ void store_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_stream(float4* p, float4 v) {
  __builtin_nontemporal_store(v.x, &p->x);
  __builtin_nontemporal_store(v.y, &p->y);
  __builtin_nontemporal_store(v.z, &p->z);
  __builtin_nontemporal_store(v.w, &p->w);
}

// NaN-propagating maximum (torch.max semantics).
__device__ __forceinline__ float nan_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

__device__ __forceinline__ float wave_nan_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = nan_max(v, __shfl_xor(v, off, FMD_WAVE));
  return v;
}

// Lane rank among the active-and-true lanes below it (prefix popcount of a ballot).
__device__ __forceinline__ int lane_prefix(uint64_t mask) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  return __popcll(mask & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
}

// Exclusive prefix sum of one integer per thread over the workgroup (blockDim a multiple of
// 64, at most 1024): wave inclusive scans by shuffles, then a scan of the wave totals by wave 0.
// Returns the thread's exclusive prefix; *total receives the block total in every thread.
// `s_wave` is LDS scratch of at least 16 entries. Integer sums are exact: the result does not
// depend on the order.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* s_wave, T* total) {
  const int lane = threadIdx.x & (FMD_WAVE - 1), wave = threadIdx.x / FMD_WAVE;
  const int nw = blockDim.x / FMD_WAVE;
  T incl = v;
#pragma unroll
  for (int off = 1; off < FMD_WAVE; off <<= 1) {
    const T o = __shfl_up(incl, off, FMD_WAVE);
    if (lane >= off) incl += o;
  }
  __syncthreads();  // s_wave may be in use by a previous call
  if (lane == FMD_WAVE - 1) s_wave[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    T w = lane < nw ? s_wave[lane] : T(0);
    T wi = w;
#pragma unroll
    for (int off = 1; off < FMD_WAVE; off <<= 1) {
      const T o = __shfl_up(wi, off, FMD_WAVE);
      if (lane >= off) wi += o;
    }
    if (lane < nw) s_wave[lane] = wi - w;  // exclusive offsets of the waves
    if (lane == nw - 1) s_wave[FMD_WAVE / 4] = wi;  // total (slot 16)
  }
  __syncthreads();
  *total = s_wave[FMD_WAVE / 4];
  return s_wave[wave] + incl - v;
}
