// fp32 operands as three bf16 planes for the bf16 matrix cores (shared by the edge GEMM and the
// fused node kernels): x = x0 + x1 + x2 with each plane rounded to nearest from the remainder of
// the previous ones, so the three planes hold x's 24 significand bits; a product is the sum of
// the six plane products xi*yj with i + j <= 2 (the dropped ones are below 2^-24 relative).
#pragma once

#include "common.h"

typedef float fmd_f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 fmd_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 fmd_bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void x3_split(float4 v, fmd_bf16x4& p0, fmd_bf16x4& p1, fmd_bf16x4& p2) {
  const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const __bf16 h0 = (__bf16)x[e];
    const float r1 = x[e] - (float)h0;  // exact
    const __bf16 h1 = (__bf16)r1;
    const float r2 = r1 - (float)h1;    // exact
    p0[e] = h0;
    p1[e] = h1;
    p2[e] = (__bf16)r2;
  }
}

// acc += a * b over the six plane products, the small ones first: (0,2) (1,1) (2,0) (0,1) (1,0) (0,0)
__device__ __forceinline__ fmd_f32x16 x3_mfma(const fmd_bf16x8 (&a)[3], const fmd_bf16x8 (&b)[3], fmd_f32x16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  return acc;
}

// LDS tile of 128 rows x 16 k (one plane): the two 8-k chunks of row r swap places when bit 3 of
// r is set, so the sixteen 16-byte operand reads of a quarter wave hit distinct bank groups.
__device__ __forceinline__ int x3_lds_offset(int row, int k) {
  return row * 16 + ((((k >> 3) ^ ((row >> 3) & 1))) * 8) + (k & 7);
}
