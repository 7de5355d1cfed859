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

// Wavefront (64 lanes) reductions in a fixed butterfly order: every lane ends with the same
// value, and the order depends on nothing but the lane layout (deterministic).
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, FMD_WAVE);
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

// Eight wave sums at once: a transposing butterfly (halve the value set at each of the first three
// exchanges, then reduce the last value over the remaining three) uses 10 exchanges instead of 48.
// On return every lane holds the total of value index 4*b5 + 2*b4 + b3 (b_i: bit i of the lane),
// see wave_sum8_index. The order of additions is fixed by the lane layout (deterministic).
__device__ __forceinline__ float wave_sum8(const float (&v)[8]) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8;
  float w[4], x[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = h5 ? v[i + 4] : v[i], send = h5 ? v[i] : v[i + 4];
    w[i] = keep + __shfl_xor(send, 32, FMD_WAVE);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = h4 ? w[i + 2] : w[i], send = h4 ? w[i] : w[i + 2];
    x[i] = keep + __shfl_xor(send, 16, FMD_WAVE);
  }
  float y = (h3 ? x[1] : x[0]) + __shfl_xor(h3 ? x[0] : x[1], 8, FMD_WAVE);
#pragma unroll
  for (int off = 4; off >= 1; off >>= 1) y += __shfl_xor(y, off, FMD_WAVE);
  return y;
}

__device__ __forceinline__ int wave_sum8_index(int lane) {
  return ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
}

// Sixteen wave sums at once (the same transposing butterfly over four halving exchanges, then two
// full ones): 17 exchanges instead of 96. On return every lane holds the total of value index
// 8*b5 + 4*b4 + 2*b3 + b2 (wave_sum16_index). Fixed order (deterministic).
__device__ __forceinline__ float wave_sum16(const float (&v)[16]) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8, h2 = lane & 4;
  float a[8], b[4], c[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float keep = h5 ? v[i + 8] : v[i], send = h5 ? v[i] : v[i + 8];
    a[i] = keep + __shfl_xor(send, 32, FMD_WAVE);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = h4 ? a[i + 4] : a[i], send = h4 ? a[i] : a[i + 4];
    b[i] = keep + __shfl_xor(send, 16, FMD_WAVE);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = h3 ? b[i + 2] : b[i], send = h3 ? b[i] : b[i + 2];
    c[i] = keep + __shfl_xor(send, 8, FMD_WAVE);
  }
  float y = (h2 ? c[1] : c[0]) + __shfl_xor(h2 ? c[0] : c[1], 4, FMD_WAVE);
  y += __shfl_xor(y, 2, FMD_WAVE);
  y += __shfl_xor(y, 1, FMD_WAVE);
  return y;
}

__device__ __forceinline__ int wave_sum16_index(int lane) {
  return ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
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
