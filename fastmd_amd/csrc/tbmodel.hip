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

// The channel columns of a lane: c = lane + 64 cc (cc < NC); lanes past C read column C - 1 (a
// real column, so every load stays in the row) and store nothing.
template <int NC>
struct LaneCols {
  int col[NC];
  bool live[NC];
  __device__ __forceinline__ explicit LaneCols(int C) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int c = lane + 64 * cc;
      live[cc] = c < C;
      col[cc] = c < C ? c : C - 1;
    }
  }
};

// the value of lane j (j wave-uniform)
__device__ __forceinline__ float lane_value(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// Rows per batch of the gated sums: a batch's loads (clamped to the run's last row) are all issued
// before its arithmetic, and the rows past the run are masked out of the sums; a run of up to R
// rows costs one memory round trip instead of one per four rows. R = 8 measured faster than 16 at
// one channel per lane (5 000 atoms, 15 edge rows per atom: the partial second batch is cheaper
// than the masked half of a single one, and the waves hold fewer registers).
template <int NC>
constexpr int gated_batch() {
  return 8;
}

template <int NC>
__global__ void __launch_bounds__(256) tb_gated_sum_kernel(const float* z, int64_t ldz, int64_t rows, int C,
                                                            RowWeight rw, const int64_t* off, int64_t n_seg,
                                                            float scale, float* out, int64_t ldo, int accumulate) {
  constexpr int R = gated_batch<NC>();
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (s >= n_seg) return;
  int64_t lo, hi;
  run_of(off, s, rows, lo, hi);
  const LaneCols<NC> lc(C);
  float* o = out + s * ldo;
  float old[NC], acc[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    old[cc] = accumulate ? o[lc.col[cc]] : 0.f;
    acc[cc] = 0.f;
  }
  for (int64_t r0 = lo; r0 < hi; r0 += R) {
    const int m = hi - r0 >= R ? R : (int)(hi - r0);
    // the batch's row weights one per lane (lane j: row j), read back per row from that lane
    const int64_t rl = r0 + (lane < m ? lane : m - 1);
    const float wl = rw.w1(rl) * rw.w2(rl);
    float x[R][NC];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int64_t r = r0 + (j < m ? j : m - 1);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) x[j][cc] = z[r * ldz + lc.col[cc]];
    }
    // rows in order; the masked rows leave the sum as it is
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const float w = lane_value(wl, j);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const float v = x[j][cc] * tb_sigmoid(x[j][cc]) * w;
        acc[cc] = j < m ? acc[cc] + v : acc[cc];
      }
    }
  }
#pragma unroll
  for (int cc = 0; cc < NC; ++cc)
    if (lc.live[cc]) o[lc.col[cc]] = accumulate ? old[cc] + scale * acc[cc] : scale * acc[cc];
}

// VJP: per row of run s, with g = scale * gout[s]: gz[r] = g w(r) silu'(z[r]) and
// gw(r) = sum_c g silu(z[r]) (the weight's gradient; with two indices written as the two
// envelopes' terms (gw w2, gw w1); added to gw with acc_gw); gsum[s] = sum_r gz[r]. Rows past the
// last run: gz = 0, gw = 0 (left as they are with acc_gw).
template <int NC>
__global__ void __launch_bounds__(256) tb_gated_sum_bwd_kernel(const float* gout, int64_t ldg, const float* z,
                                                                int64_t ldz, int64_t rows, int C, RowWeight rw,
                                                                const int64_t* off, int64_t n_seg, float scale,
                                                                float* gz, int64_t ldgz, float* gsum, int64_t ldgs,
                                                                float* gw, int64_t ldgw, int acc_gw,
                                                                int64_t seg_blocks) {
  constexpr int R = gated_batch<NC>();
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
  const LaneCols<NC> lc(C);
  const bool two = rw.i2 != nullptr, old_gw = gw && acc_gw;
  float g[NC], acc[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    g[cc] = lc.live[cc] ? scale * gout[s * ldg + lc.col[cc]] : 0.f;
    acc[cc] = 0.f;
  }
  for (int64_t r0 = lo; r0 < hi; r0 += R) {
    const int m = hi - r0 >= R ? R : (int)(hi - r0);
    // every load of the batch before its arithmetic: the rows, and one per lane (lane j: row j)
    // the row's weights and old weight gradients, read back per row from that lane
    const int64_t rl = r0 + (lane < m ? lane : m - 1);
    const float wal = rw.w1(rl), wbl = rw.w2(rl);
    const float go0 = old_gw ? gw[rl * ldgw] : 0.f, go1 = old_gw && two ? gw[rl * ldgw + 1] : 0.f;
    float xs[R][NC];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int64_t r = r0 + (j < m ? j : m - 1);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) xs[j][cc] = z[r * ldz + lc.col[cc]];
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int64_t r = r0 + j;
      const float a = lane_value(wal, j), b = lane_value(wbl, j), w = a * b;
      float p = 0.f, v[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const float x = xs[j][cc];
        const float sg = tb_sigmoid(x);
        const float si = x * sg;
        v[cc] = g[cc] * w * (sg + si * (1.0f - sg));
        acc[cc] = j < m ? acc[cc] + v[cc] : acc[cc];
        p += g[cc] * si;  // g = 0 on the lanes past C
      }
      if (j < m) {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
          if (lc.live[cc]) gz[r * ldgz + lc.col[cc]] = v[cc];
      }
      if (gw) {
        const float t = wave_sum(p);
        if (j < m && lane == 0) {
          if (two) {
            gw[r * ldgw] = lane_value(go0, j) + t * b;
            gw[r * ldgw + 1] = lane_value(go1, j) + t * a;
          } else {
            gw[r * ldgw] = lane_value(go0, j) + t;
          }
        }
      }
    }
  }
  if (gsum) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
      if (lc.live[cc]) gsum[s * ldgs + lc.col[cc]] = acc[cc];
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
// device, several bonds or triplets per wave and pass (channels across the lanes) whose loads are
// all issued before their arithmetic: one chain of dependent loads per pass, not per item. A
// bond's triplets as first bond are the run [eto[b], eto[b+1]) of the line graph (contiguous), as
// second bond the same run through second_perm.
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

// The index work of a pass runs across the lanes (one load instruction per level of the chain
// bond_rows -> eto -> line graph / second_perm -> envelope for all of the pass's bonds or
// triplets), the channel rows across the wave with the indices read back per lane: a pass costs
// one chain of dependent loads, whatever the number of bonds or triplets in it.
__device__ __forceinline__ int lane_int(int v, int j) { return __builtin_amdgcn_readlane(v, j); }

// Lane q < U: bond slot q of the pass (bond j0 + q NW of bond_rows; past the count the pass's
// first bond again, loaded and not stored) with its run [lo, hi) of triplets as first bond,
// clamped to t_cap.
template <int U>
struct BondSlots {
  int b, lo, hi;
  bool ok;
  __device__ __forceinline__ BondSlots(const LineCsr& lc, int64_t j0, int64_t nw, int64_t nb) {
    const int lane = threadIdx.x & 63;
    const int64_t j = j0 + (lane < U ? lane : 0) * nw;
    ok = j < nb;
    b = lc.bond_rows[ok ? j : j0];
    int64_t l = lc.eto[b], h = lc.eto[(int64_t)b + 1];
    h = h < lc.t_cap ? h : lc.t_cap;
    l = l < h ? l : h;
    lo = (int)l;
    hi = (int)h;
  }
  __device__ __forceinline__ int64_t bond(int q) const { return lane_int(b, q); }
  __device__ __forceinline__ int64_t count(int q) const { return lane_int(hi, q) - lane_int(lo, q); }
  __device__ __forceinline__ bool stored(int q) const { return lane_int(ok ? 1 : 0, q) != 0; }
  // on lane l: triplet t of bond q's run, clamped to its last triplet (row 0 for an empty run,
  // whose loads are then not used as addresses)
  __device__ __forceinline__ int64_t slot_row(int q, int t, bool& empty) const {
    const int l = __shfl(lo, q, 64), h = __shfl(hi, q, 64);
    empty = h <= l;
    return l + t < h ? l + t : (h > l ? h - 1 : 0);
  }
};

// bonds per pass and triplets per bond whose loads go out together (longer runs finish in a loop)
template <int NC>
constexpr int bond_pass() {
  return NC == 1 ? 4 : 2;
}
constexpr int kRunBatch = 4;

// eps[b] += scale * sum over b's triplets (first bond), in order, of silu(z3[k]) s_b s_b2
template <int NC>
__global__ void __launch_bounds__(256) tb_bond_sum_kernel(LineCsr lc, const float* z3, int64_t ldz, int C,
                                                           const float* geo, float scale, float* eps, int64_t lde) {
  constexpr int U = bond_pass<NC>(), TQ = kRunBatch;
  const int lane = threadIdx.x & 63;
  const LaneCols<NC> cols(C);
  const int64_t nb = lc.short_offsets[lc.n], nw = (int64_t)gridDim.x * 4;
  for (int64_t j0 = wave_id(); j0 < nb; j0 += U * nw) {
    const BondSlots<U> bs(lc, j0, nw, nb);
    float old[U][NC], x[U][TQ][NC];
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) old[q][cc] = eps[bs.bond(q) * lde + cols.col[cc]];
    // lane l < U TQ: triplet slot (l / TQ, l % TQ) and its weight s_b s_b2
    const int qs = lane < U * TQ ? lane / TQ : 0;
    bool empty;
    const int64_t ks = bs.slot_row(qs, lane % TQ, empty);
    const int b2raw = lc.line[5 * ks + 4];
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int t = 0; t < TQ; ++t) {
        const int64_t k = lane_int((int)ks, q * TQ + t);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) x[q][t][cc] = z3[k * ldz + cols.col[cc]];
      }
    const int bq = __shfl(bs.b, qs, 64);
    const float w1 = geo[8 * (int64_t)bq + 6];
    const float ws = w1 * geo[8 * (int64_t)(empty ? bq : b2raw) + 6];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      float acc[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) acc[cc] = 0.f;
      const int64_t cnt = bs.count(q);
#pragma unroll
      for (int t = 0; t < TQ; ++t) {
        const float w = lane_value(ws, q * TQ + t);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const float v = x[q][t][cc] * tb_sigmoid(x[q][t][cc]) * w;
          acc[cc] = t < cnt ? acc[cc] + v : acc[cc];
        }
      }
      // the rest of a longer run, four triplets' loads at a time
      const int64_t lo = lane_int(bs.lo, q), hi = lane_int(bs.hi, q);
      const float w1q = lane_value(w1, q * TQ);
      for (int64_t k0 = lo + TQ; k0 < hi; k0 += 4) {
        const int m = hi - k0 >= 4 ? 4 : (int)(hi - k0);
        float y[4][NC], wy[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t k = k0 + (t < m ? t : m - 1);
          wy[t] = w1q * geo[8 * (int64_t)lc.line[5 * k + 4] + 6];
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) y[t][cc] = z3[k * ldz + cols.col[cc]];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            const float v = y[t][cc] * tb_sigmoid(y[t][cc]) * wy[t];
            acc[cc] = t < m ? acc[cc] + v : acc[cc];
          }
      }
      if (bs.stored(q)) {
        const int64_t b = bs.bond(q);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
          if (cols.live[cc]) eps[b * lde + cols.col[cc]] = old[q][cc] + scale * acc[cc];
      }
    }
  }
}

// triplets per pass of the triplet VJP
template <int NC>
constexpr int triplet_pass() {
  return NC == 1 ? 8 : 4;
}

// Per triplet k: with g = scale geps[b1], gz3[k] = g s_b1 s_b2 silu'(z3[k]) and
// gw = sum_c g silu(z3[k]), stored as the envelope terms gsw[k] = (gw s_b2, gw s_b1). Rows past
// the real triplets: gz3 = 0.
template <int NC>
__global__ void __launch_bounds__(256) tb_triplet_bwd_kernel(LineCsr lc, const float* geps, int64_t ldg,
                                                              const float* z3, int64_t ldz, int C, const float* geo,
                                                              float scale, float* gz3, int64_t ldgz, float* gsw) {
  constexpr int U = triplet_pass<NC>();
  const int lane = threadIdx.x & 63;
  const LaneCols<NC> cols(C);
  const int64_t t_all = lc.pair_offsets[lc.n];
  const int64_t t_real = t_all < lc.t_cap ? t_all : lc.t_cap;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t k0 = wave_id(); k0 < lc.t_cap; k0 += U * nw) {
    // lane q < U: triplet slot q (k0 + q NW); a slot past the real triplets loads line-graph row 0
    // and edge row 0 (in bounds, unused)
    const int64_t kl = k0 + (lane < U ? lane : 0) * nw;
    const bool real = kl < t_real;
    const int64_t kr = real ? kl : 0;
    const int r1 = lc.line[5 * kr + 2], r2 = lc.line[5 * kr + 4];
    float x[U][NC], g[U][NC];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int64_t kq = k0 + q * nw < t_real ? k0 + q * nw : 0;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) x[q][cc] = z3[kq * ldz + cols.col[cc]];
    }
    const int b1 = real ? r1 : 0, b2 = real ? r2 : 0;
    const float w1l = geo[8 * (int64_t)b1 + 6], w2l = geo[8 * (int64_t)b2 + 6];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int64_t b = lane_int(b1, q);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) g[q][cc] = scale * geps[b * ldg + cols.col[cc]];
    }
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int64_t kq = k0 + q * nw;
      if (kq >= lc.t_cap) continue;
      float* out = gz3 + kq * ldgz;
      if (kq >= t_real) {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
          if (cols.live[cc]) out[cols.col[cc]] = 0.f;
        continue;
      }
      const float w1 = lane_value(w1l, q), w2 = lane_value(w2l, q), w = w1 * w2;
      float p = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const float sg = tb_sigmoid(x[q][cc]);
        const float si = x[q][cc] * sg;
        if (cols.live[cc]) {
          out[cols.col[cc]] = g[q][cc] * w * (sg + si * (1.0f - sg));
          p += g[q][cc] * si;
        }
      }
      const float gw = wave_sum(p);
      if (lane == 0) {
        gsw[2 * kq] = gw * w2;
        gsw[2 * kq + 1] = gw * w1;
      }
    }
  }
}

// Per bond b: geps[b] += sum over b's triplets as first bond of ga3[k, 0:C], then as second bond
// of ga3[k, C:2C]; gs[b] (+)= the same sums of gsw[k, 0] and gsw[k, 1] (stored, or added with
// acc_gs). A second-bond slot of -1 (no triplet) adds zeros.
template <int NC>
__global__ void __launch_bounds__(256) tb_bond_reduce_kernel(LineCsr lc, const float* ga3, int64_t lda, int C,
                                                              const float* gsw, float* geps, int64_t ldg, float* gs,
                                                              int acc_gs) {
  constexpr int U = bond_pass<NC>(), TQ = kRunBatch;
  const int lane = threadIdx.x & 63;
  const LaneCols<NC> cols(C);
  const int64_t nb = lc.short_offsets[lc.n], nw = (int64_t)gridDim.x * 4;
  for (int64_t j0 = wave_id(); j0 < nb; j0 += U * nw) {
    const BondSlots<U> bs(lc, j0, nw, nb);
    const float gs_l = acc_gs ? gs[bs.b] : 0.f;
    float old[U][NC], x[U][2][TQ][NC];
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) old[q][cc] = geps[bs.bond(q) * ldg + cols.col[cc]];
    // lane l < 2 U TQ: role l / (U TQ), slot ((l % U TQ) / TQ, l % TQ); role 1 through second_perm
    const int sl = lane % (U * TQ), role_l = lane < U * TQ ? 0 : 1;
    bool empty;
    const int64_t pl = bs.slot_row(lane < 2 * U * TQ ? sl / TQ : 0, sl % TQ, empty);
    const int sp = lc.second_perm[pl];
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int t = 0; t < TQ; ++t) {
        const int64_t k = lane_int((int)pl, q * TQ + t);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) x[q][0][t][cc] = ga3[k * lda + cols.col[cc]];
      }
    const int kk = role_l == 0 ? (int)pl : (empty ? -1 : sp);
    const float sw = gsw[2 * (int64_t)(kk >= 0 ? kk : 0) + role_l];
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int t = 0; t < TQ; ++t) {
        const int k = lane_int(kk, U * TQ + q * TQ + t);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) x[q][1][t][cc] = ga3[(int64_t)(k >= 0 ? k : 0) * lda + C + cols.col[cc]];
      }
#pragma unroll
    for (int q = 0; q < U; ++q) {
      float acc[NC], gsum = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) acc[cc] = 0.f;
      const int64_t cnt = bs.count(q), lo = lane_int(bs.lo, q), hi = lane_int(bs.hi, q);
#pragma unroll
      for (int role = 0; role < 2; ++role) {
#pragma unroll
        for (int t = 0; t < TQ; ++t) {
          const int l = role * U * TQ + q * TQ + t;
          const bool use = t < cnt, ok = lane_int(kk, l) >= 0;
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            const float v = ok ? x[q][role][t][cc] : 0.f;
            acc[cc] = use ? acc[cc] + v : acc[cc];
          }
          const float v = ok ? lane_value(sw, l) : 0.f;
          gsum = use ? gsum + v : gsum;
        }
        // the rest of a longer run, four slots' loads at a time
        for (int64_t p0 = lo + TQ; p0 < hi; p0 += 4) {
          const int m = hi - p0 >= 4 ? 4 : (int)(hi - p0);
          int64_t ky[4];
          float y[4][NC], sy[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t p = p0 + (t < m ? t : m - 1);
            ky[t] = role == 0 ? p : (int64_t)lc.second_perm[p];
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t k = ky[t] >= 0 ? ky[t] : 0;
            sy[t] = gsw[2 * k + role];
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) y[t][cc] = ga3[k * lda + role * C + cols.col[cc]];
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const bool use = t < m, ok = ky[t] >= 0;
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
              const float v = ok ? y[t][cc] : 0.f;
              acc[cc] = use ? acc[cc] + v : acc[cc];
            }
            const float v = ok ? sy[t] : 0.f;
            gsum = use ? gsum + v : gsum;
          }
        }
      }
      if (bs.stored(q)) {
        const int64_t b = bs.bond(q);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
          if (cols.live[cc]) geps[b * ldg + cols.col[cc]] = old[q][cc] + acc[cc];
        if (lane == 0) gs[b] = lane_value(gs_l, q) + gsum;
      }
    }
  }
}

RowWeight make_weight(const float* w, int64_t ldw, const int32_t* i1, const int32_t* i2, int64_t ld_idx) {
  return RowWeight{w, ldw, i1, i2, ld_idx};
}

// launch of KERNEL<NC> with NC = ceil(channels / 64) (channels <= 256)
#define TB_LAUNCH_NC(KERNEL, CHANNELS, GRID, ...)                                              \
  do {                                                                                        \
    switch (fmd_cdiv((CHANNELS), 64)) {                                                       \
      case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      case 3: hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
      default: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(256), 0, stream, __VA_ARGS__); break; \
    }                                                                                         \
  } while (0)

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
  TB_LAUNCH_NC(tb_gated_sum_kernel, channels, dim3((unsigned)fmd_cdiv(n_segments, 4)), z, ldz, rows, channels,
               make_weight(w, ldw, index1, index2, ld_index), offsets, n_segments, scale, out, ldo, accumulate);
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
  TB_LAUNCH_NC(tb_gated_sum_bwd_kernel, channels, dim3((unsigned)(seg_blocks + tail_blocks)), gout, ldg, z, ldz, rows,
               channels, make_weight(w, ldw, index1, index2, ld_index), offsets, n_segments, scale, gz, ldgz, gsum,
               ldgs, gw, ldgw, accumulate_gw, seg_blocks);
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
  TB_LAUNCH_NC(tb_bond_sum_kernel, channels, dim3(kStrideBlocks), lc, z3, ldz, channels, geo, scale, eps, lde);
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
  TB_LAUNCH_NC(tb_triplet_bwd_kernel, channels, dim3(kStrideBlocks), lc, geps, ldg, z3, ldz, channels, geo, scale, gz3,
               ldgz, gsw);
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
  TB_LAUNCH_NC(tb_bond_reduce_kernel, channels, dim3(kStrideBlocks), lc, ga3, lda, channels, gsw, geps, ldg, gs,
               accumulate_gs);
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
