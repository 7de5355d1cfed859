// Kernels of the three-body (CHGNet/MatRIS-style) model: the bond envelope of the line graph,
// the gated segment sum that forms both of its updates (angles -> bonds, edges -> atoms) and
// its VJP, the linear per-atom readout and the geometry VJP that folds every radial gradient.
//
// Gated sum: out[s] (+)= scale * sum_{r in run s} silu(z[r]) * w(r), with the runs of a CSR
// whose rows are the identity (the rows of each segment contiguous: the edges of a centre, the
// triplets of a first bond) and w(r) a per-row weight: w[r], w[i1[r]], or w[i1[r]] w[i2[r]]
// (the two bonds' envelopes of a triplet). One wave per segment, channels across the lanes,
// rows summed in row order: deterministic, no atomics.
#include "common.h"

namespace {

__device__ __forceinline__ float tb_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

__device__ __forceinline__ int64_t tb_real_rows(const int64_t* n_edges, int64_t e_cap) {
  const int64_t e = n_edges[0];
  return e < e_cap ? e : e_cap;
}

// the polynomial cutoff 1 - 21x^5 + 35x^6 - 15x^7 (x = r / rc) and its r-derivative
__device__ __forceinline__ void poly_cutoff(float r, float rc, float& f, float& df) {
  const float x = r / rc;
  f = 0.f;
  df = 0.f;
  if (x < 1.0f) {
    const float x2 = x * x, x4 = x2 * x2, x5 = x4 * x;
    f = 1.0f - 21.0f * x5 + 35.0f * x5 * x - 15.0f * x5 * x2;
    const float omx = 1.0f - x;
    df = -105.0f * x4 * omx * omx / rc;
  }
}

// geo rows [u_x, u_y, u_z, r, fc, dfc, s, ds]: s = the bond envelope of a short real row
__global__ void tb_envelope_kernel(float* geo, const uint8_t* short_flags, const int64_t* n_edges, int64_t e_cap,
                                   float rb) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= e_cap) return;
  float s = 0.f, ds = 0.f;
  if (e < tb_real_rows(n_edges, e_cap) && short_flags[e]) poly_cutoff(geo[8 * e + 3], rb, s, ds);
  geo[8 * e + 6] = s;
  geo[8 * e + 7] = ds;
}

struct RowWeight {
  const float* w;
  int64_t ldw;
  const int32_t* i1;  // null: w[r]
  const int32_t* i2;  // null: w[i1[r]]
  int64_t ld_idx;
  __device__ __forceinline__ float w1(int64_t r) const { return i1 ? w[(int64_t)i1[r * ld_idx] * ldw] : w[r * ldw]; }
  __device__ __forceinline__ float w2(int64_t r) const { return i2 ? w[(int64_t)i2[r * ld_idx] * ldw] : 1.0f; }
};

__device__ __forceinline__ void run_of(const int64_t* off, int64_t s, int64_t rows, int64_t& lo, int64_t& hi) {
  lo = off[s];
  hi = off[s + 1];
  hi = hi < rows ? hi : rows;
  lo = lo < hi ? lo : hi;
}

__global__ void __launch_bounds__(256) tb_gated_sum_kernel(const float* z, int64_t ldz, int64_t rows, int C,
                                                            RowWeight rw, const int64_t* off, int64_t n_seg,
                                                            float scale, float* out, int64_t ldo, int accumulate) {
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (s >= n_seg) return;
  int64_t lo, hi;
  run_of(off, s, rows, lo, hi);
  for (int c = lane; c < C; c += 64) {
    float acc = 0.f;
    // four rows' loads in flight before their arithmetic (the sum stays in row order)
    for (int64_t r = lo; r < hi; r += 4) {
      const int m = hi - r >= 4 ? 4 : (int)(hi - r);
      float x[4], w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < m) {
          x[j] = z[(r + j) * ldz + c];
          w[j] = rw.w1(r + j) * rw.w2(r + j);
        }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < m) acc += x[j] * tb_sigmoid(x[j]) * w[j];
    }
    float* o = out + s * ldo + c;
    *o = accumulate ? *o + scale * acc : scale * acc;
  }
}

// VJP: per row of run s, with g = scale * gout[s]: gz[r] = g w(r) silu'(z[r]) and
// gw(r) = sum_c g silu(z[r]) (the weight's gradient; with two indices written as the two
// envelopes' terms (gw w2, gw w1); added to gw with acc_gw); gsum[s] = sum_r gz[r]. Rows past the
// last run: gz = 0, gw = 0 (left as they are with acc_gw).
__global__ void __launch_bounds__(256) tb_gated_sum_bwd_kernel(const float* gout, int64_t ldg, const float* z,
                                                                int64_t ldz, int64_t rows, int C, RowWeight rw,
                                                                const int64_t* off, int64_t n_seg, float scale,
                                                                float* gz, int64_t ldgz, float* gsum, int64_t ldgs,
                                                                float* gw, int64_t ldgw, int acc_gw,
                                                                int64_t seg_blocks) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if ((int64_t)blockIdx.x >= seg_blocks) {
    // the rows of no segment
    const int64_t tail = off[n_seg] < rows ? off[n_seg] : rows;
    const int64_t step = ((int64_t)gridDim.x - seg_blocks) * 4;
    for (int64_t r = tail + ((int64_t)blockIdx.x - seg_blocks) * 4 + wave; r < rows; r += step) {
      for (int c = lane; c < C; c += 64) gz[r * ldgz + c] = 0.f;
      if (gw && !acc_gw && lane < (rw.i2 ? 2 : 1)) gw[r * ldgw + lane] = 0.f;
    }
    return;
  }
  const int64_t s = (int64_t)blockIdx.x * 4 + wave;
  if (s >= n_seg) return;
  int64_t lo, hi;
  run_of(off, s, rows, lo, hi);
  // C <= 256: up to four channels per lane
  float g[4], acc[4];
  const int nc = (C + 63) / 64;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = lane + 64 * k;
    g[k] = (k < nc && c < C) ? scale * gout[s * ldg + c] : 0.f;
    acc[k] = 0.f;
  }
  for (int64_t r0 = lo; r0 < hi; r0 += 4) {
    // four rows' loads in flight before their arithmetic (rows still handled in order)
    const int m = hi - r0 >= 4 ? 4 : (int)(hi - r0);
    float xs[4][4], wa[4], wb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < m) {
        wa[j] = rw.w1(r0 + j);
        wb[j] = rw.w2(r0 + j);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = lane + 64 * k;
          xs[j][k] = (k < nc && c < C) ? z[(r0 + j) * ldz + c] : 0.f;
        }
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j >= m) break;
      const int64_t r = r0 + j;
      const float a = wa[j], b = wb[j], w = a * b;
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c = lane + 64 * k;
        if (k < nc && c < C) {
          const float x = xs[j][k];
          const float sg = tb_sigmoid(x);
          const float si = x * sg;
          const float v = g[k] * w * (sg + si * (1.0f - sg));
          gz[r * ldgz + c] = v;
          acc[k] += v;
          p += g[k] * si;
        }
      }
      if (gw) {
        const float t = wave_sum(p);
        if (lane == 0) {
          if (rw.i2) {
            gw[r * ldgw] = (acc_gw ? gw[r * ldgw] : 0.f) + t * b;
            gw[r * ldgw + 1] = (acc_gw ? gw[r * ldgw + 1] : 0.f) + t * a;
          } else {
            gw[r * ldgw] = (acc_gw ? gw[r * ldgw] : 0.f) + t;
          }
        }
      }
    }
  }
  if (gsum) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = lane + 64 * k;
      if (k < nc && c < C) gsum[s * ldgs + c] = acc[k];
    }
  }
}

// E_i = e0[elem_i] + h_i . wr
__global__ void __launch_bounds__(256) tb_readout_kernel(const float* h, int64_t ldh, int C, const float* wr,
                                                          const int32_t* elem, const float* e0, int64_t n,
                                                          float* energy) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (i >= n) return;
  float p = 0.f;
  for (int c = lane; c < C; c += 64) p += h[i * ldh + c] * wr[c];
  p = wave_sum(p);
  if (lane == 0) energy[i] = e0[elem[i]] + p;
}

// gh_i = g_i wr (g_i = gE[i], or `sign` without gE)
__global__ void tb_readout_bwd_kernel(const float* ge, float sign, const float* wr, int C, int64_t n, float* gh,
                                      int64_t ldgh) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * C) return;
  const int64_t i = t / C;
  const int c = (int)(t - i * C);
  gh[i * ldgh + c] = (ge ? ge[i] : sign) * wr[c];
}

// gvec = gr u + (gu - (gu . u) u) / r with gr = sum_n gef def + gfc dfc + gs ds
__global__ void tb_geometry_bwd_kernel(const float* geo, const float* def, int nb, const float* gef, int64_t ldgef,
                                       const float* gu, int64_t ldgu, const float* gfc, const float* gs,
                                       const uint8_t* bond_flags, const int64_t* n_edges, int64_t e_cap,
                                       float* gvec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= e_cap) return;
  if (e >= tb_real_rows(n_edges, e_cap)) {
    gvec[3 * e] = gvec[3 * e + 1] = gvec[3 * e + 2] = 0.f;
    return;
  }
  const float* g = geo + 8 * e;
  float gr = 0.f;
  if (gef)
    for (int n = 0; n < nb; ++n) gr += gef[e * ldgef + n] * def[e * nb + n];
  if (gfc) gr += gfc[e] * g[5];
  // gs and gu hold values on the bond rows only (with bond_flags; else on every row)
  const bool bond = bond_flags ? bond_flags[e] != 0 : true;
  if (gs && bond) gr += gs[e] * g[7];
  float v[3] = {0.f, 0.f, 0.f};
  if (gu && bond) {
    v[0] = gu[e * ldgu];
    v[1] = gu[e * ldgu + 1];
    v[2] = gu[e * ldgu + 2];
  }
  const float inv_r = 1.0f / g[3];
  const float gdotu = v[0] * g[0] + v[1] * g[1] + v[2] * g[2];
#pragma unroll
  for (int k = 0; k < 3; ++k) gvec[3 * e + k] = gr * g[k] + (v[k] - gdotu * g[k]) * inv_r;
}

// ---- angle -> bond sums over the line graph. The work is a few bonds and triplets per atom, far
// fewer than the edge rows: each kernel runs a fixed grid of waves that strides over the real
// bonds (bond_rows[0, short_offsets[n])) or triplets ([0, pair_offsets[n])), counts read on the
// device, one bond or triplet per wave at a time (channels across the lanes). A bond's triplets
// as first bond are the run [eto[b], eto[b+1]) of the line graph (contiguous), as second bond
// the same run through second_perm.
struct LineCsr {
  const int64_t* short_offsets;  // [n + 1]: the bond count at [n]
  const int32_t* bond_rows;      // [e_cap]
  const int64_t* eto;            // edge_triplet_offsets [e_cap + 1]
  const int32_t* second_perm;    // [t_cap]
  const int32_t* line;           // line_graph [t_cap, 5]: (atom, pair 1, row 1, pair 2, row 2)
  const int64_t* pair_offsets;   // [n + 1]: the triplet count at [n]
  int64_t n;
  int64_t t_cap;
};

constexpr int kStrideBlocks = 1024;  // 4096 waves (about four per SIMD)

__device__ __forceinline__ int64_t wave_id() {
  return (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
}

// eps[b] += scale * sum over b's triplets (first bond), in order, of silu(z3[k]) s_b s_b2
__global__ void __launch_bounds__(256) tb_bond_sum_kernel(LineCsr lc, const float* z3, int64_t ldz, int C,
                                                           const float* geo, float scale, float* eps, int64_t lde) {
  const int lane = threadIdx.x & 63;
  const int nc = (C + 63) / 64;
  const int64_t nb = lc.short_offsets[lc.n];
  for (int64_t j = wave_id(); j < nb; j += (int64_t)gridDim.x * 4) {
    const int64_t b = lc.bond_rows[j];
    const float w1 = geo[8 * b + 6];
    int64_t lo = lc.eto[b], hi = lc.eto[b + 1];
    hi = hi < lc.t_cap ? hi : lc.t_cap;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    // four triplets' loads in flight before their arithmetic (the sum stays in triplet order)
    for (int64_t k0 = lo; k0 < hi; k0 += 4) {
      const int m = hi - k0 >= 4 ? 4 : (int)(hi - k0);
      float x[4][4], w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < m) {
          w[q] = w1 * geo[8 * (int64_t)lc.line[5 * (k0 + q) + 4] + 6];
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            const int c = lane + 64 * cc;
            x[q][cc] = (cc < nc && c < C) ? z3[(k0 + q) * ldz + c] : 0.f;
          }
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < m)
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) acc[cc] += x[q][cc] * tb_sigmoid(x[q][cc]) * w[q];
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = lane + 64 * cc;
      if (cc < nc && c < C) eps[b * lde + c] += scale * acc[cc];
    }
  }
}

// Per triplet k (one wave): with g = scale geps[b1], gz3[k] = g s_b1 s_b2 silu'(z3[k]) and
// gw = sum_c g silu(z3[k]), stored as the envelope terms gsw[k] = (gw s_b2, gw s_b1). Rows past
// the real triplets: gz3 = 0.
__global__ void __launch_bounds__(256) tb_triplet_bwd_kernel(LineCsr lc, const float* geps, int64_t ldg,
                                                              const float* z3, int64_t ldz, int C, const float* geo,
                                                              float scale, float* gz3, int64_t ldgz, float* gsw) {
  const int lane = threadIdx.x & 63;
  const int nc = (C + 63) / 64;
  const int64_t t_all = lc.pair_offsets[lc.n];
  const int64_t t_real = t_all < lc.t_cap ? t_all : lc.t_cap;
  for (int64_t k = wave_id(); k < lc.t_cap; k += (int64_t)gridDim.x * 4) {
    if (k >= t_real) {
      for (int c = lane; c < C; c += 64) gz3[k * ldgz + c] = 0.f;
      continue;
    }
    const int64_t b1 = lc.line[5 * k + 2], b2 = lc.line[5 * k + 4];
    const float w1 = geo[8 * b1 + 6], w2 = geo[8 * b2 + 6], w = w1 * w2;
    float g[4], x[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = lane + 64 * cc;
      const bool ok = cc < nc && c < C;
      g[cc] = ok ? scale * geps[b1 * ldg + c] : 0.f;
      x[cc] = ok ? z3[k * ldz + c] : 0.f;
    }
    float p = 0.f;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = lane + 64 * cc;
      if (cc < nc && c < C) {
        const float sg = tb_sigmoid(x[cc]);
        const float si = x[cc] * sg;
        gz3[k * ldgz + c] = g[cc] * w * (sg + si * (1.0f - sg));
        p += g[cc] * si;
      }
    }
    const float gw = wave_sum(p);
    if (lane == 0) {
      gsw[2 * k] = gw * w2;
      gsw[2 * k + 1] = gw * w1;
    }
  }
}

// Per bond b (one wave): geps[b] += sum over b's triplets as first bond of ga3[k, 0:C], then as
// second bond of ga3[k, C:2C]; gs[b] (+)= the same sums of gsw[k, 0] and gsw[k, 1] (stored, or
// added with acc_gs).
__global__ void __launch_bounds__(256) tb_bond_reduce_kernel(LineCsr lc, const float* ga3, int64_t lda, int C,
                                                              const float* gsw, float* geps, int64_t ldg, float* gs,
                                                              int acc_gs) {
  const int lane = threadIdx.x & 63;
  const int nc = (C + 63) / 64;
  const int64_t nb = lc.short_offsets[lc.n];
  for (int64_t j = wave_id(); j < nb; j += (int64_t)gridDim.x * 4) {
    const int64_t b = lc.bond_rows[j];
    int64_t lo = lc.eto[b], hi = lc.eto[b + 1];
    hi = hi < lc.t_cap ? hi : lc.t_cap;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float gsum = 0.f;
    for (int role = 0; role < 2; ++role) {
      for (int64_t p0 = lo; p0 < hi; p0 += 4) {
        const int m = hi - p0 >= 4 ? 4 : (int)(hi - p0);
        int64_t kk[4];
        float x[4][4], sw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q < m) kk[q] = role == 0 ? p0 + q : (int64_t)lc.second_perm[p0 + q];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q < m) {
            const bool real = kk[q] >= 0;
            sw[q] = real ? gsw[2 * kk[q] + role] : 0.f;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
              const int c = lane + 64 * cc;
              x[q][cc] = (real && cc < nc && c < C) ? ga3[kk[q] * lda + role * C + c] : 0.f;
            }
          }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q < m) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) acc[cc] += x[q][cc];
            gsum += sw[q];
          }
      }
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int c = lane + 64 * cc;
      if (cc < nc && c < C) geps[b * ldg + c] += acc[cc];
    }
    if (lane == 0) gs[b] = (acc_gs ? gs[b] : 0.f) + gsum;
  }
}

RowWeight make_weight(const float* w, int64_t ldw, const int32_t* i1, const int32_t* i2, int64_t ld_idx) {
  return RowWeight{w, ldw, i1, i2, ld_idx};
}

}  // namespace

extern "C" {

int fmd_tb_bond_envelope_f32(float* geo, const uint8_t* short_flags, const int64_t* n_edges, int64_t e_cap, float rb,
                             hipStream_t stream) {
  FMD_REQUIRE(e_cap >= 0 && rb > 0.f);
  if (e_cap == 0) return FMD_OK;
  FMD_REQUIRE(geo && short_flags && n_edges);
  hipLaunchKernelGGL(tb_envelope_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, geo, short_flags,
                     n_edges, e_cap, rb);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_gated_sum_f32(const float* z, int64_t ldz, int64_t rows, int32_t channels, const float* w, int64_t ldw,
                         const int32_t* index1, const int32_t* index2, int64_t ld_index, const int64_t* offsets,
                         int64_t n_segments, float scale, float* out, int64_t ldo, int32_t accumulate,
                         hipStream_t stream) {
  FMD_REQUIRE(rows >= 0 && n_segments >= 0 && channels > 0 && channels <= 256 && ldz >= channels &&
              ldo >= channels && (index1 || !index2));
  if (n_segments == 0) return FMD_OK;
  FMD_REQUIRE(z && w && offsets && out);
  hipLaunchKernelGGL(tb_gated_sum_kernel, dim3((unsigned)fmd_cdiv(n_segments, 4)), dim3(256), 0, stream, z, ldz, rows,
                     channels, make_weight(w, ldw, index1, index2, ld_index), offsets, n_segments, scale, out, ldo,
                     accumulate);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_gated_sum_bwd_f32(const float* gout, int64_t ldg, const float* z, int64_t ldz, int64_t rows,
                             int32_t channels, const float* w, int64_t ldw, const int32_t* index1,
                             const int32_t* index2, int64_t ld_index, const int64_t* offsets, int64_t n_segments,
                             float scale, float* gz, int64_t ldgz, float* gsum, int64_t ldgs, float* gw, int64_t ldgw,
                             int32_t accumulate_gw, hipStream_t stream) {
  FMD_REQUIRE(rows >= 0 && n_segments >= 0 && channels > 0 && channels <= 256 && ldz >= channels &&
              ldgz >= channels && (index1 || !index2));
  if (rows == 0 && n_segments == 0) return FMD_OK;
  FMD_REQUIRE(gout && z && w && offsets && gz);
  FMD_REQUIRE(!gsum || ldgs >= channels);
  FMD_REQUIRE(!gw || ldgw >= (index2 ? 2 : 1));
  const int64_t seg_blocks = fmd_cdiv(n_segments, 4);
  int64_t tail_blocks = fmd_cdiv(rows, 4);
  tail_blocks = tail_blocks < 1 ? 1 : (tail_blocks > 512 ? 512 : tail_blocks);
  hipLaunchKernelGGL(tb_gated_sum_bwd_kernel, dim3((unsigned)(seg_blocks + tail_blocks)), dim3(256), 0, stream, gout,
                     ldg, z, ldz, rows, channels, make_weight(w, ldw, index1, index2, ld_index), offsets, n_segments,
                     scale, gz, ldgz, gsum, ldgs, gw, ldgw, accumulate_gw, seg_blocks);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_bond_sum_f32(const float* z3, int64_t ldz, int32_t channels, const float* geo, const int64_t* short_offsets,
                        const int32_t* bond_rows, const int64_t* edge_triplet_offsets, const int32_t* line_graph,
                        int64_t n_atoms, int64_t t_cap, float scale, float* eps, int64_t lde, hipStream_t stream) {
  FMD_REQUIRE(n_atoms >= 0 && t_cap >= 0 && channels > 0 && channels <= 256 && ldz >= channels && lde >= channels);
  if (n_atoms == 0 || t_cap == 0) return FMD_OK;
  FMD_REQUIRE(z3 && geo && short_offsets && bond_rows && edge_triplet_offsets && line_graph && eps);
  LineCsr lc{short_offsets, bond_rows, edge_triplet_offsets, nullptr, line_graph, nullptr, n_atoms, t_cap};
  hipLaunchKernelGGL(tb_bond_sum_kernel, dim3(kStrideBlocks), dim3(256), 0, stream, lc, z3, ldz, channels, geo, scale,
                     eps, lde);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_triplet_bwd_f32(const float* geps, int64_t ldg, const float* z3, int64_t ldz, int32_t channels,
                           const float* geo, const int32_t* line_graph, const int64_t* pair_offsets, int64_t n_atoms,
                           int64_t t_cap, float scale, float* gz3, int64_t ldgz, float* gsw, hipStream_t stream) {
  FMD_REQUIRE(n_atoms >= 0 && t_cap >= 0 && channels > 0 && channels <= 256 && ldg >= channels && ldz >= channels &&
              ldgz >= channels);
  if (n_atoms == 0 || t_cap == 0) return FMD_OK;
  FMD_REQUIRE(geps && z3 && geo && line_graph && pair_offsets && gz3 && gsw);
  LineCsr lc{nullptr, nullptr, nullptr, nullptr, line_graph, pair_offsets, n_atoms, t_cap};
  hipLaunchKernelGGL(tb_triplet_bwd_kernel, dim3(kStrideBlocks), dim3(256), 0, stream, lc, geps, ldg, z3, ldz,
                     channels, geo, scale, gz3, ldgz, gsw);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_bond_reduce_f32(const float* ga3, int64_t lda, int32_t channels, const float* gsw,
                           const int64_t* short_offsets, const int32_t* bond_rows, const int64_t* edge_triplet_offsets,
                           const int32_t* second_perm, int64_t n_atoms, int64_t t_cap, float* geps, int64_t ldg,
                           float* gs, int32_t accumulate_gs, hipStream_t stream) {
  FMD_REQUIRE(n_atoms >= 0 && t_cap >= 0 && channels > 0 && channels <= 256 && lda >= 2 * channels &&
              ldg >= channels);
  if (n_atoms == 0 || t_cap == 0) return FMD_OK;
  FMD_REQUIRE(ga3 && gsw && short_offsets && bond_rows && edge_triplet_offsets && second_perm && geps && gs);
  LineCsr lc{short_offsets, bond_rows, edge_triplet_offsets, second_perm, nullptr, nullptr, n_atoms, t_cap};
  hipLaunchKernelGGL(tb_bond_reduce_kernel, dim3(kStrideBlocks), dim3(256), 0, stream, lc, ga3, lda, channels, gsw, geps,
                     ldg, gs, accumulate_gs);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_readout_f32(const float* h, int64_t ldh, int32_t channels, const float* wr, const int32_t* elem,
                       const float* e0, int64_t n, float* energy, hipStream_t stream) {
  FMD_REQUIRE(n >= 0 && channels > 0 && ldh >= channels);
  if (n == 0) return FMD_OK;
  FMD_REQUIRE(h && wr && elem && e0 && energy);
  hipLaunchKernelGGL(tb_readout_kernel, dim3((unsigned)fmd_cdiv(n, 4)), dim3(256), 0, stream, h, ldh, channels, wr,
                     elem, e0, n, energy);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_readout_bwd_f32(const float* gE, float sign, const float* wr, int32_t channels, int64_t n, float* gh,
                           int64_t ldgh, hipStream_t stream) {
  FMD_REQUIRE(n >= 0 && channels > 0 && ldgh >= channels);
  if (n == 0) return FMD_OK;
  FMD_REQUIRE(wr && gh);
  hipLaunchKernelGGL(tb_readout_bwd_kernel, dim3((unsigned)fmd_cdiv(n * channels, 256)), dim3(256), 0, stream, gE,
                     sign, wr, channels, n, gh, ldgh);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_tb_geometry_bwd_f32(const float* geo, const float* def, int32_t nb, const float* gef, int64_t ldgef,
                            const float* gu, int64_t ldgu, const float* gfc, const float* gs, const uint8_t* bond_flags,
                            const int64_t* n_edges, int64_t e_cap, float* gvec, hipStream_t stream) {
  FMD_REQUIRE(e_cap >= 0 && nb > 0);
  if (e_cap == 0) return FMD_OK;
  FMD_REQUIRE(geo && def && n_edges && gvec);
  FMD_REQUIRE(!gef || ldgef >= nb);
  FMD_REQUIRE(!gu || ldgu >= 3);
  hipLaunchKernelGGL(tb_geometry_bwd_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, geo, def, nb,
                     gef, ldgef, gu, ldgu, gfc, gs, bond_flags, n_edges, e_cap, gvec);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
