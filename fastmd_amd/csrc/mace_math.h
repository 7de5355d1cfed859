// Per-(node, channel) arithmetic of the MACE-like symmetric contraction (correlation order 3,
// L <= 1), shared by the standalone kernels and the fused node kernels:
//   n1 = |P1|^2;  B0 = c1 P0 + c2 P0^2 + c3 n1 + c4 P0^3 + c5 P0 n1
//   B1_x = (d1 + d2 P0 + d3 P0^2 + d4 n1) P1_x
// c points at Wc[elem, 0, ch] (stride C between the five coefficients), d at Wd[elem, 0, ch].
#pragma once

#include "common.h"

__device__ __forceinline__ float symcon_b0(float p0, float n1, const float* c, int C) {
  return c[0] * p0 + c[C] * p0 * p0 + c[2 * C] * n1 + c[3 * C] * p0 * p0 * p0 + c[4 * C] * p0 * n1;
}

__device__ __forceinline__ float symcon_q(float p0, float n1, const float* d, int C) {
  return d[0] + d[C] * p0 + d[2 * C] * p0 * p0 + d[3 * C] * n1;
}

// VJP: (gb0, gb1 when has_vec, else no vector output) -> (gp0, gp[3])
__device__ __forceinline__ void symcon_vjp(float p0, const float (&p)[3], const float* c, const float* d, int C,
                                           float gb0, bool has_vec, const float (&gb1)[3], float& gp0,
                                           float (&gp)[3]) {
  const float n1 = p[0] * p[0] + p[1] * p[1] + p[2] * p[2];
  gp0 = gb0 * (c[0] + 2.0f * c[C] * p0 + 3.0f * c[3 * C] * p0 * p0 + c[4 * C] * n1);
  float gn1 = gb0 * (c[2 * C] + c[4 * C] * p0);
  gp[0] = gp[1] = gp[2] = 0.f;
  if (has_vec) {
    const float q = symcon_q(p0, n1, d, C);
    float gq = 0.f;
#pragma unroll
    for (int x = 0; x < 3; ++x) {
      gp[x] = gb1[x] * q;
      gq += gb1[x] * p[x];
    }
    gp0 += gq * (d[C] + 2.0f * d[2 * C] * p0);
    gn1 += gq * d[3 * C];
  }
#pragma unroll
  for (int x = 0; x < 3; ++x) gp[x] = gp[x] + 2.0f * gn1 * p[x];
}
