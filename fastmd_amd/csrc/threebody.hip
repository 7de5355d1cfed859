// Three-body Fourier angle basis over the line graph (triton_threebody_fourier.py:1-17, 45-80):
// for triplet t with bond rows (r1, r2) (the target and source bond vectors),
//   cos = (u[r1] . u[r2]) * (1 - 1e-6),  theta = acos(cos),
//   out[t] = [1/sqrt(2), sin(theta f_1..F), cos(theta f_1..F)] / scale     (1 + 2F columns)
// VJP (explicit, deterministic): d out / d theta, d theta / d cos = -1 / sqrt(max(1 - cos^2,
// 1e-24)), g_u[r1] += d * u[r2], g_u[r2] += d * u[r1] with d = g_cos * (1 - 1e-6). The angle
// itself is taken in float64 (angle_of), the basis and the VJP terms in float32. On the line
// graph the triplets of an atom are its ordered pairs of distinct short bonds: one wave per
// atom takes them (lane = triplet, up to 64 at a time), and the bond sums are formed in LDS in
// triplet order, without atomics. Padding triplets (the all-loop pair) are written in the
// forward; the VJP covers the real triplets. An overflowed build (its flag passed) has the
// all-loop topology in every row: the forward reads them all from line_graph, the VJP is zero.
#include "common.h"

namespace {

constexpr int kMaxFreq = 16;
constexpr float kEps = 0.999999f;

// The angle of two bond vectors. The dot product, the (1 - 1e-6) scaling, acos and 1 - c^2 are
// taken in float64 (the float products are exact there): near-(anti)parallel bonds, where
// acos' = -1 / sin(theta) magnifies the rounding of c, come out as accurate as the float inputs
// allow instead of carrying float32 rounding of c (the reference's kernel rounds c to float32).
struct Angle {
  float theta;    // acos(c)
  float inv_sin;  // 1 / sqrt(max(1 - c^2, 1e-24))
};

__device__ __forceinline__ Angle angle_of(const float (&a)[3], const float (&b)[3]) {
  const double d = ((double)a[0] * (double)b[0] + (double)a[1] * (double)b[1]) + (double)a[2] * (double)b[2];
  const double c = d * (1.0 - 1.0e-6);
  const double s2 = (1.0 - c) * (1.0 + c);
  return Angle{(float)acos(c), 1.0f / sqrtf((float)fmax(s2, 1.0e-24))};
}

__device__ __forceinline__ void basis_row(float theta, const float* freqs, int nf, float inv_scale, float* o) {
  o[0] = 0.70710678118654752f * inv_scale;
  for (int k = 0; k < nf; ++k) {
    const float a = theta * freqs[k];
    o[1 + k] = sinf(a) * inv_scale;
    o[1 + nf + k] = cosf(a) * inv_scale;
  }
}

__device__ __forceinline__ void unit_of(const float* u, int64_t ld, int64_t r, float (&v)[3]) {
  v[0] = u[r * ld];
  v[1] = u[r * ld + 1];
  v[2] = u[r * ld + 2];
}

// general rows: out[t] from (tgt[t], src[t])
__global__ void fourier_rows_kernel(const float* u, int64_t ld, const int32_t* tgt, const int32_t* src, int64_t rows,
                                    const float* freqs, int nf, float inv_scale, float* out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows) return;
  float a[3], b[3];
  unit_of(u, ld, tgt[t], a);
  unit_of(u, ld, src[t], b);
  basis_row(angle_of(a, b).theta, freqs, nf, inv_scale, out + t * (1 + 2 * nf));
}

// per-row contributions of the general VJP: contrib[t] = (d u[src], d u[tgt]) (6 floats)
__global__ void fourier_rows_bwd_kernel(const float* gout, const float* u, int64_t ld, const int32_t* tgt,
                                        const int32_t* src, int64_t rows, const float* freqs, int nf, float inv_scale,
                                        float* contrib) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows) return;
  float a[3], b[3];
  unit_of(u, ld, tgt[t], a);
  unit_of(u, ld, src[t], b);
  const Angle an = angle_of(a, b);
  const float* g = gout + t * (1 + 2 * nf);
  float dth = 0.f;
  for (int k = 0; k < nf; ++k) {
    const float f = freqs[k], x = an.theta * f;
    dth += g[1 + k] * cosf(x) * f - g[1 + nf + k] * sinf(x) * f;
  }
  dth *= inv_scale;
  const float d = -dth * an.inv_sin * kEps;
  float* o = contrib + t * 6;
  o[0] = d * b[0];  // to the target row
  o[1] = d * b[1];
  o[2] = d * b[2];
  o[3] = d * a[0];  // to the source row
  o[4] = d * a[1];
  o[5] = d * a[2];
}

struct LineArgs {
  const int64_t* pair_offsets;
  const int64_t* short_counts;
  const int32_t* sem;
  int32_t bmax;
  int64_t n;
  int64_t t_cap;
  const int32_t* line_graph;  // [t_cap, 5] (padding rows)
  const uint8_t* overflow;    // null or the build's flag: an overflowed build's rows are all padding
};

__device__ __forceinline__ bool line_overflowed(const LineArgs& la) { return la.overflow && *la.overflow; }

// forward over the line graph: blocks [0, atom_blocks) one wave per atom (its triplets),
// the rest the padding rows
__global__ void __launch_bounds__(256) fourier_line_kernel(LineArgs la, const float* u, int64_t ld, const float* freqs,
                                                            int nf, float inv_scale, float* out, int64_t atom_blocks) {
  const int lane = threadIdx.x & 63;
  const bool ovf = line_overflowed(la);
  const int64_t t_real_all = ovf ? 0 : la.pair_offsets[la.n];
  const int64_t t_real = t_real_all < la.t_cap ? t_real_all : la.t_cap;
  const int width = 1 + 2 * nf;
  if (blockIdx.x >= atom_blocks) {
    const int64_t t = t_real + (int64_t)(blockIdx.x - atom_blocks) * blockDim.x + threadIdx.x;
    for (int64_t r = t; r < la.t_cap; r += (int64_t)(gridDim.x - atom_blocks) * blockDim.x) {
      float a[3], b[3];
      unit_of(u, ld, la.line_graph[r * 5 + 2], a);
      unit_of(u, ld, la.line_graph[r * 5 + 4], b);
      basis_row(angle_of(a, b).theta, freqs, nf, inv_scale, out + r * width);
    }
    return;
  }
  const int64_t i = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (i >= la.n || ovf) return;
  const int64_t s = la.short_counts[i], p0 = la.pair_offsets[i];
  const int64_t npairs = s * (s - 1), den = s > 1 ? s - 1 : 1;
  const int32_t* row = la.sem + i * la.bmax;
  for (int64_t base = 0; base < npairs; base += 64) {
    const int64_t l = base + lane;
    const int64_t t = p0 + l;
    if (l < npairs && t < la.t_cap) {
      const int64_t first = l / den, second_raw = l - first * den, second = second_raw + (second_raw >= first ? 1 : 0);
      float a[3], b[3];
      unit_of(u, ld, row[first < la.bmax - 1 ? first : la.bmax - 1], a);
      unit_of(u, ld, row[second < la.bmax - 1 ? second : la.bmax - 1], b);
      basis_row(angle_of(a, b).theta, freqs, nf, inv_scale, out + t * width);
    }
  }
}

// VJP over the line graph: one wave per atom; per 64 triplets the contributions go to LDS, then
// lane k (a bond of the atom) adds those of its triplets in triplet order
__global__ void __launch_bounds__(256) fourier_line_bwd_kernel(LineArgs la, const float* gout, const float* u,
                                                                int64_t ld, const float* freqs, int nf,
                                                                float inv_scale, float* gu, int64_t ldg,
                                                                int accumulate) {
  __shared__ float s_c[4][64][6];
  __shared__ int s_f[4][64][2];
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64;
  const int64_t i = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (i >= la.n) return;
  const int64_t s = la.short_counts[i], p0 = la.pair_offsets[i];
  // an overflowed build has no real triplets: its short rows get a zero gradient
  const int64_t npairs = line_overflowed(la) ? 0 : s * (s - 1), den = s > 1 ? s - 1 : 1;
  const int32_t* row = la.sem + i * la.bmax;
  const int width = 1 + 2 * nf;
  const int64_t sb = s < la.bmax ? s : la.bmax;
  // bonds in chunks of 64 (lane k: the bond of rank kb + k), triplets in chunks of 64
  for (int64_t kb = 0; kb < sb; kb += 64) {
    float acc[3] = {0.f, 0.f, 0.f};
    for (int64_t base = 0; base < npairs; base += 64) {
      const int64_t l = base + lane;
      const int64_t t = p0 + l;
      int first = -1, second = -1;
      float ct[3] = {0.f, 0.f, 0.f}, cs[3] = {0.f, 0.f, 0.f};
      if (l < npairs && t < la.t_cap) {
        const int64_t f = l / den, sr = l - f * den, sc = sr + (sr >= f ? 1 : 0);
        first = (int)f;
        second = (int)sc;
        float a[3], b[3];
        unit_of(u, ld, row[f < la.bmax - 1 ? f : la.bmax - 1], a);
        unit_of(u, ld, row[sc < la.bmax - 1 ? sc : la.bmax - 1], b);
        const Angle an = angle_of(a, b);
        const float* g = gout + t * width;
        float dth = 0.f;
        for (int k = 0; k < nf; ++k) {
          const float fr = freqs[k], x = an.theta * fr;
          dth += g[1 + k] * cosf(x) * fr - g[1 + nf + k] * sinf(x) * fr;
        }
        dth *= inv_scale;
        const float d = -dth * an.inv_sin * kEps;
#pragma unroll
        for (int x = 0; x < 3; ++x) {
          ct[x] = d * b[x];  // to the first (target) bond
          cs[x] = d * a[x];  // to the second (source) bond
        }
      }
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        s_c[w][lane][x] = ct[x];
        s_c[w][lane][3 + x] = cs[x];
      }
      s_f[w][lane][0] = first;
      s_f[w][lane][1] = second;
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      const int64_t k = kb + lane;
      if (k < sb) {
        const int m = (int)(npairs - base < 64 ? npairs - base : 64);
        for (int q = 0; q < m; ++q) {
          if (s_f[w][q][0] == k) {
            acc[0] += s_c[w][q][0];
            acc[1] += s_c[w][q][1];
            acc[2] += s_c[w][q][2];
          }
          if (s_f[w][q][1] == k) {
            acc[0] += s_c[w][q][3];
            acc[1] += s_c[w][q][4];
            acc[2] += s_c[w][q][5];
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    const int64_t k = kb + lane;
    if (k < sb) {
      float* d = gu + (int64_t)row[k] * ldg;
#pragma unroll
      for (int x = 0; x < 3; ++x) d[x] = accumulate ? d[x] + acc[x] : acc[x];
    }
  }
}

}  // namespace

extern "C" {

int fmd_threebody_fourier_f32(const float* unit_vec, int64_t ld_unit, const int32_t* target_index,
                              const int32_t* source_index, int64_t rows, const float* freqs, int32_t n_freq,
                              float scale, float* out, hipStream_t stream) {
  FMD_REQUIRE(rows >= 0 && n_freq > 0 && n_freq <= kMaxFreq && ld_unit >= 3 && scale != 0.f);
  if (rows == 0) return FMD_OK;
  FMD_REQUIRE(unit_vec && target_index && source_index && freqs && out);
  hipLaunchKernelGGL(fourier_rows_kernel, dim3((unsigned)fmd_cdiv(rows, 256)), dim3(256), 0, stream, unit_vec, ld_unit,
                     target_index, source_index, rows, freqs, n_freq, 1.0f / scale, out);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_threebody_fourier_bwd_rows_f32(const float* gout, const float* unit_vec, int64_t ld_unit,
                                       const int32_t* target_index, const int32_t* source_index, int64_t rows,
                                       const float* freqs, int32_t n_freq, float scale, float* contrib,
                                       hipStream_t stream) {
  FMD_REQUIRE(rows >= 0 && n_freq > 0 && n_freq <= kMaxFreq && ld_unit >= 3 && scale != 0.f);
  if (rows == 0) return FMD_OK;
  FMD_REQUIRE(gout && unit_vec && target_index && source_index && freqs && contrib);
  hipLaunchKernelGGL(fourier_rows_bwd_kernel, dim3((unsigned)fmd_cdiv(rows, 256)), dim3(256), 0, stream, gout, unit_vec,
                     ld_unit, target_index, source_index, rows, freqs, n_freq, 1.0f / scale, contrib);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_threebody_fourier_line_f32(const float* unit_vec, int64_t ld_unit, const int64_t* pair_offsets,
                                   const int64_t* short_counts, const int32_t* short_edge_matrix, int32_t bmax,
                                   const int32_t* line_graph, const uint8_t* overflow, int64_t n_atoms, int64_t t_cap,
                                   const float* freqs, int32_t n_freq, float scale, float* out, hipStream_t stream) {
  FMD_REQUIRE(n_atoms > 0 && t_cap > 0 && bmax > 0 && n_freq > 0 && n_freq <= kMaxFreq && ld_unit >= 3 &&
              scale != 0.f);
  FMD_REQUIRE(unit_vec && pair_offsets && short_counts && short_edge_matrix && line_graph && freqs && out);
  LineArgs la{pair_offsets, short_counts, short_edge_matrix, bmax, n_atoms, t_cap, line_graph, overflow};
  const int64_t atom_blocks = fmd_cdiv(n_atoms, 4);
  int64_t pad_blocks = fmd_cdiv(t_cap, 256 * 8);
  pad_blocks = pad_blocks < 1 ? 1 : (pad_blocks > 1024 ? 1024 : pad_blocks);
  hipLaunchKernelGGL(fourier_line_kernel, dim3((unsigned)(atom_blocks + pad_blocks)), dim3(256), 0, stream, la,
                     unit_vec, ld_unit, freqs, n_freq, 1.0f / scale, out, atom_blocks);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_threebody_fourier_line_bwd_f32(const float* gout, const float* unit_vec, int64_t ld_unit,
                                       const int64_t* pair_offsets, const int64_t* short_counts,
                                       const int32_t* short_edge_matrix, int32_t bmax, const uint8_t* overflow,
                                       int64_t n_atoms, int64_t t_cap, const float* freqs, int32_t n_freq, float scale,
                                       float* grad_unit, int64_t ld_grad, int32_t accumulate, hipStream_t stream) {
  FMD_REQUIRE(n_atoms > 0 && t_cap > 0 && bmax > 0 && n_freq > 0 && n_freq <= kMaxFreq && ld_unit >= 3 &&
              ld_grad >= 3 && scale != 0.f);
  FMD_REQUIRE(gout && unit_vec && pair_offsets && short_counts && short_edge_matrix && freqs && grad_unit);
  LineArgs la{pair_offsets, short_counts, short_edge_matrix, bmax, n_atoms, t_cap, nullptr, overflow};
  hipLaunchKernelGGL(fourier_line_bwd_kernel, dim3((unsigned)fmd_cdiv(n_atoms, 4)), dim3(256), 0, stream, la, gout,
                     unit_vec, ld_unit, freqs, n_freq, 1.0f / scale, grad_unit, ld_grad, accumulate);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
