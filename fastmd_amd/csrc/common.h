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
