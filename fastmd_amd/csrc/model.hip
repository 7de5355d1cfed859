// Model kernels of the MD step: edge geometry + radial basis, the MACE-like interaction
// (fused message + receiver aggregation, symmetric contraction, readout) and their explicit
// VJPs, and the Morse pair potential. fp32, deterministic (no float atomics: receiver sums walk
// the centre CSR, sender sums walk the reverse-edge CSR).
//
// Edge rows: real rows [0, min(n_edges, e_cap)), n_edges read from device memory (a captured
// graph replays them with the current count); rows past it are fixed-capacity padding and are
// skipped (their contributions are exactly zero by the padding contract: far self-loops lie
// beyond the cutoff, where the envelope and its derivative vanish).
// Channel layout: a wavefront owns a node or an edge; lane l holds channels l*CPL .. +CPL
// (C = 64 * CPL). Node features: h0 [N, C], h1 [N, 3, C]. Per edge z [E, 4C] = the four path
// weight blocks (a | b | c | d) before the SiLU.
#include "common.h"
#include "mace_math.h"

#include <initializer_list>

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / FMD_WAVE;
constexpr float kPi = 3.14159265358979323846f;

__device__ __forceinline__ int64_t real_rows(const int64_t* n_edges, int64_t e_cap) {
  const int64_t e = n_edges[0];
  return e < e_cap ? e : e_cap;
}

// 1 / (1 + e^-x) with the hardware reciprocal (1 ulp): the saturated ends give exactly 0 and 1
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// ------------------------------------------------------------------------------------------
// edge geometry: geo[e] = (ux, uy, uz, r, fcut, dfcut, 0, 0); ef[e, n] = b_n(r) fcut(r);
// def[e, n] = d ef / dr. b_n = sqrt(2/rc) sin(n pi r / rc) / r (n = 1..NB), fcut the p = 5
// polynomial envelope 1 - 21 x^5 + 35 x^6 - 15 x^7 (x = r / rc < 1, else 0).
// vec = (pos[j] + image @ cell) - pos[c], image @ cell formed row by row.
// ------------------------------------------------------------------------------------------
struct GeoArgs {
  const float* pos;
  const float* cell;
  const int32_t* system_of;
  const int32_t* edge_index;
  const float* edge_image;
  const int64_t* n_edges;
  int64_t e_cap;
  float rc;
  int nb;
  float* geo;
  float* ef;
  float* def;
};

__device__ __forceinline__ void edge_geometry_row(const GeoArgs& a, int64_t e) {
  const float* pos = a.pos;
  const float* cell = a.cell;
  const int32_t *system_of = a.system_of, *edge_index = a.edge_index;
  const float* edge_image = a.edge_image;
  const int64_t e_cap = a.e_cap;
  const float rc = a.rc;
  const int nb = a.nb;
  float *geo = a.geo, *ef = a.ef, *def = a.def;
  const int64_t rows = real_rows(a.n_edges, e_cap);
  float* g = geo + 8 * e;
  if (e >= rows) {
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = 0.f;
    g[3] = 1.f;
    for (int n = 0; n < nb; ++n) {
      ef[e * nb + n] = 0.f;
      def[e * nb + n] = 0.f;
    }
    return;
  }
  const int32_t c = edge_index[2 * e], j = edge_index[2 * e + 1];
  const float ix = edge_image[3 * e], iy = edge_image[3 * e + 1], iz = edge_image[3 * e + 2];
  if (system_of) cell += 9 * (int64_t)system_of[c];  // a union of systems: the centre's cell
  float v[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    float s = ix * cell[k];
    s = s + iy * cell[3 + k];
    s = s + iz * cell[6 + k];
    v[k] = (pos[3 * j + k] + s) - pos[3 * c + k];
  }
  const float r = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const float inv_r = 1.0f / r;
  const float x = r / rc;
  float fc = 0.f, dfc = 0.f;
  if (x < 1.0f) {
    const float x2 = x * x, x4 = x2 * x2, x5 = x4 * x;
    fc = 1.0f - 21.0f * x5 + 35.0f * x5 * x - 15.0f * x5 * x2;
    const float omx = 1.0f - x;
    dfc = -105.0f * x4 * omx * omx / rc;
  }
  g[0] = v[0] * inv_r;
  g[1] = v[1] * inv_r;
  g[2] = v[2] * inv_r;
  g[3] = r;
  g[4] = fc;
  g[5] = dfc;
  g[6] = 0.f;
  g[7] = 0.f;
  const float pref = sqrtf(2.0f / rc);
  for (int n = 1; n <= nb; ++n) {
    const float k = (float)n * kPi / rc;
    const float sn = sinf(k * r), cs = cosf(k * r);
    const float b = pref * sn * inv_r;
    const float db = pref * (k * cs * inv_r - sn * inv_r * inv_r);
    ef[e * nb + (n - 1)] = b * fc;
    def[e * nb + (n - 1)] = db * fc + b * dfc;
  }
}

__global__ void edge_geometry_kernel(const GeoArgs a) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < a.e_cap) edge_geometry_row(a, e);
}

// g_vec[e] = g_r u + (g_u - (g_u . u) u) / r with g_r = sum_n g_ef[e,n] def[e,n] (over up to two
// g_ef sources) + g_fcut dfcut; g_geo[e] = (g_ux, g_uy, g_uz, g_fcut).
// dE/d(edge vector) of row e from the gradients of its geometry: the radial-basis gradients of
// up to two layers (gef0, gef1, times d ef / dr), the unit-vector and cutoff gradients (ggeo).
__device__ __forceinline__ void edge_vec_grad(const float* geo, const float* def, int nb, const float* gef0,
                                              int64_t ld0, const float* gef1, int64_t ld1, const float* ggeo,
                                              int64_t e, float (&out)[3]) {
  const float* g = geo + 8 * e;
  float gr = 0.f;
  for (int n = 0; n < nb; ++n) {
    float ge = 0.f;
    if (gef0) ge += gef0[e * ld0 + n];
    if (gef1) ge += gef1[e * ld1 + n];
    gr += ge * def[e * nb + n];
  }
  float gu[3] = {0.f, 0.f, 0.f};
  if (ggeo) {
    gu[0] = ggeo[4 * e];
    gu[1] = ggeo[4 * e + 1];
    gu[2] = ggeo[4 * e + 2];
    gr += ggeo[4 * e + 3] * g[5];
  }
  const float inv_r = 1.0f / g[3];
  const float gdotu = gu[0] * g[0] + gu[1] * g[1] + gu[2] * g[2];
#pragma unroll
  for (int k = 0; k < 3; ++k) out[k] = gr * g[k] + (gu[k] - gdotu * g[k]) * inv_r;
}

__global__ void edge_geometry_bwd_kernel(const float* geo, const float* def, int nb, const float* gef0, int64_t ld0,
                                         const float* gef1, int64_t ld1, const float* ggeo, const int64_t* n_edges,
                                         int64_t e_cap, float* gvec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= e_cap) return;
  const int64_t rows = real_rows(n_edges, e_cap);
  if (e >= rows) {
    gvec[3 * e] = gvec[3 * e + 1] = gvec[3 * e + 2] = 0.f;
    return;
  }
  float v[3];
  edge_vec_grad(geo, def, nb, gef0, ld0, gef1, ld1, ggeo, e, v);
#pragma unroll
  for (int k = 0; k < 3; ++k) gvec[3 * e + k] = v[k];
}

// ------------------------------------------------------------------------------------------
// interaction: forward message + receiver sum. One wave per centre node i.
//   w = silu(z_e) * fcut_e; proj = h1_j . u; m0 = wa h0_j + wc proj; m1_x = wb h0_j u_x + wd h1_j,x
//   A0_i = inv_avg * sum_e m0, A1_i = inv_avg * sum_e m1
// Without h1 (a layer whose vector features are zero, where wc and wd meet only zeros) z holds
// just the a | b blocks: [E, 2C]. zq, when given, is the receiver block of z per atom ([N, the
// same width]), added to every row of the centre.
//
// Layout: a half-wave per row (lane l of a half holds channels CPL l .. + CPL, CPL = C / 32), so
// every load of a row's block or of a node row is 16 bytes per lane (the texture path costs the
// same per instruction for 8 and 16 bytes) and one instruction serves two rows. Half h of the
// wave takes rows lo + h, lo + h + 2, ... of the centre. Per 64 rows the wave loads their
// neighbour index and geometry once (one row per lane, coalesced) and each half reads its row's
// with readlane; each group of kPairs row pairs issues all of its loads before any arithmetic
// (one memory round trip per group). The two halves' sums are added at the end (fixed order:
// deterministic).
// ------------------------------------------------------------------------------------------
constexpr int kPairs = 2;

__device__ __forceinline__ int bcast(int v, int s) { return __builtin_amdgcn_readlane(v, s); }
__device__ __forceinline__ float bcast(float v, int s) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), s));
}
// lane s0's v in the lower half-wave, lane s1's in the upper one (s0, s1 uniform)
__device__ __forceinline__ int bcast2(int v, int s0, int s1, bool upper) {
  const int a = bcast(v, s0), b = bcast(v, s1);
  return upper ? b : a;
}
__device__ __forceinline__ float bcast2(float v, int s0, int s1, bool upper) {
  const float a = bcast(v, s0), b = bcast(v, s1);
  return upper ? b : a;
}

// the same exchange for row data that is not on the path to the gathers' addresses: ds_bpermute
// (the LDS crossbar) moves a value per instruction with no VALU work; bperm_addr is the byte
// address of lane s0 in the lower half-wave and of lane s1 in the upper one, shared by the values
__device__ __forceinline__ int bperm_addr(int s0, int s1, bool upper) { return (upper ? s1 : s0) << 2; }
__device__ __forceinline__ float bperm(float v, int addr) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(v)));
}

// CPL consecutive floats (CPL 2: 8-byte, 4 and 8: 16-byte aligned)
template <int CPL>
__device__ __forceinline__ void load_ch(const float* p, float (&v)[CPL]) {
  if constexpr (CPL == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x;
    v[1] = t.y;
  } else {
#pragma unroll
    for (int q = 0; q < CPL; q += 4) {
      const float4 t = *reinterpret_cast<const float4*>(p + q);
      v[q] = t.x;
      v[q + 1] = t.y;
      v[q + 2] = t.z;
      v[q + 3] = t.w;
    }
  }
}

template <int CPL>
__device__ __forceinline__ void store_ch(float* p, const float (&v)[CPL]) {
  if constexpr (CPL == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
#pragma unroll
    for (int q = 0; q < CPL; q += 4) *reinterpret_cast<float4*>(p + q) = make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]);
  }
}

template <int CPL>
__device__ __forceinline__ void store_ch_stream(float* p, const float (&v)[CPL]) {
  if constexpr (CPL == 2) {
    store_stream(p, v[0]);
    store_stream(p + 1, v[1]);
  } else {
#pragma unroll
    for (int q = 0; q < CPL; q += 4)
      store_stream(reinterpret_cast<float4*>(p + q), make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]));
  }
}

// one row's neighbour index and geometry (zeros for ok == false)
struct RowGeo {
  int j;
  float ux, uy, uz, fc;
};

__device__ __forceinline__ RowGeo row_geo(const float* geo, const int32_t* edge_index, int64_t e, bool ok) {
  RowGeo r{0, 0.f, 0.f, 0.f, 0.f};
  if (ok) {
    r.j = edge_index[2 * e + 1];
    const float4 g = *reinterpret_cast<const float4*>(geo + 8 * e);
    r.ux = g.x;
    r.uy = g.y;
    r.uz = g.z;
    r.fc = geo[8 * e + 4];
  }
  return r;
}

// the wave's node (uniform) and its real rows [lo, hi)
__device__ __forceinline__ int64_t wave_rows(const int64_t* off, const int64_t* n_edges, int64_t e_cap, int64_t i,
                                             int64_t& lo) {
  const int64_t rows = real_rows(n_edges, e_cap);
  int64_t hi = off[i + 1];
  lo = off[i];
  hi = hi < rows ? hi : rows;
  lo = lo < hi ? lo : hi;
  return hi;
}

// Several waves per atom (WPA > 1, small systems, where one wave per atom leaves most of the
// chip idle and each wave walks its rows one after the other): wave `sub` of an atom takes the
// row pairs sub, sub + WPA, ... of each 64-row chunk, and the per-atom sums are added over the
// atom's waves in wave order through LDS (fixed order: deterministic; a different association
// than one wave per atom, so the choice is made per system size, not per launch).
// v[k][q] (channels c0 + q of vector k, the same in both halves) becomes the sum over the waves.
template <int WPA, int NV, int CPL>
__device__ __forceinline__ void reduce_waves(float (&v)[NV][CPL], float* s_red, int wib, int sub, int lane) {
  if constexpr (WPA > 1) {
    constexpr int C = 32 * CPL;
    const int c0 = (lane & 31) * CPL;
    float* mine = s_red + wib * NV * C;
    if (lane < 32) {
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int q = 0; q < CPL; ++q) mine[k * C + c0 + q] = v[k][q];
    }
    __syncthreads();
    const float* first = s_red + (wib - sub) * NV * C;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        float t = first[k * C + c0 + q];
#pragma unroll
        for (int w = 1; w < WPA; ++w) t += first[(w * NV + k) * C + c0 + q];
        v[k][q] = t;
      }
  }
}

// Node-factored z (FZ): z_e = [h0_j | h0_i | ef_e] W1 is linear in its three blocks, so with
// P = h0 W1[:C] and Q = h0 W1[C:2C] formed per atom ([N, NZ C] each, node GEMMs) a row is
//   z_e = (P[j] + sum_n ef_e,n W1[2C + n]) + Q[i]
// and no [E, NZ C] array is written or read: the kernels gather P by sender (the centre's Q once
// per wave, or in the sender-side VJP the wave's own P once and Q by receiver) and add the radial
// term from the edge's basis row and W1's radial rows staged in LDS ([RB, 4C], zero past nb).
// The radial rows are applied to a group's rows together (each LDS read serves the group).
// The radial products in one of three loop forms, chosen per kernel by measurement (the same
// products in the same order: the same bits):
//  kRadialFull: unrolled whole (the basis values are registers with constant indices), one radial
//    row per scheduling region (without the barrier the scheduler would issue every LDS read up
//    front and hold all RB * NZ * CPL weights in registers);
//  kRadialShift: a loop over the radial rows, the basis values moved down the row's registers after
//    each step (constant register indices);
//  kRadialPairs: a loop of two radial rows per step, each step's basis value selected among the
//    row's registers (the fewest registers).
constexpr int kRadialPairs = 0, kRadialShift = 1, kRadialFull = 2;

template <int KP, int NZ, int CPL, int RB, int FORM>
__device__ __forceinline__ void add_radial(const float* s_w, int woff, const float (&er)[KP][RB],
                                           float (&zr)[KP][NZ][CPL]) {
  constexpr int C = 32 * CPL;
  if constexpr (FORM == kRadialFull) {
#pragma unroll
    for (int t = 0; t < RB; ++t) {
      float wv[NZ][CPL];
#pragma unroll
      for (int b = 0; b < NZ; ++b) load_ch<CPL>(s_w + t * 4 * C + b * C + woff, wv[b]);
#pragma unroll
      for (int b = 0; b < NZ; ++b)
#pragma unroll
        for (int g = 0; g < KP; ++g)
#pragma unroll
          for (int q = 0; q < CPL; ++q) zr[g][b][q] += er[g][t] * wv[b][q];
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if constexpr (FORM == kRadialShift) {
    float eb[KP][RB];
#pragma unroll
    for (int g = 0; g < KP; ++g)
#pragma unroll
      for (int k = 0; k < RB; ++k) eb[g][k] = er[g][k];
#pragma unroll 1
    for (int t = 0; t < RB; ++t) {
#pragma unroll
      for (int b = 0; b < NZ; ++b) {
        float wv[CPL];
        load_ch<CPL>(s_w + t * 4 * C + b * C + woff, wv);
#pragma unroll
        for (int g = 0; g < KP; ++g)
#pragma unroll
          for (int q = 0; q < CPL; ++q) zr[g][b][q] += eb[g][0] * wv[q];
      }
#pragma unroll
      for (int g = 0; g < KP; ++g)
#pragma unroll
        for (int k = 0; k + 1 < RB; ++k) eb[g][k] = eb[g][k + 1];
    }
  } else {
#pragma unroll 2
    for (int t = 0; t < RB; ++t) {
#pragma unroll
      for (int b = 0; b < NZ; ++b) {
        float wv[CPL];
        load_ch<CPL>(s_w + t * 4 * C + b * C + woff, wv);
#pragma unroll
        for (int g = 0; g < KP; ++g)
#pragma unroll
          for (int q = 0; q < CPL; ++q) zr[g][b][q] += er[g][t] * wv[q];
      }
    }
  }
}

// the basis row of edge e (nb <= RB values, zero past nb)
template <int RB>
__device__ __forceinline__ void load_basis(const float* ef, int nb, int64_t e, float (&v)[RB]) {
  const float* p = ef + e * nb;
  if (nb == RB) {
#pragma unroll
    for (int t = 0; t < RB; t += 4) {
      const float4 x = *reinterpret_cast<const float4*>(p + t);
      v[t] = x.x;
      v[t + 1] = x.y;
      v[t + 2] = x.z;
      v[t + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < RB; ++t) v[t] = t < nb ? p[t] : 0.f;
  }
}

// W1's radial rows [nb, 4C] into LDS as [RB, 4C], zero rows past nb (all threads of the block, which
// has kThreads). Every thread issues all of its loads before its first store (one memory round trip
// per block, not one per element), 16-byte loads when w1ef is 16-byte aligned.
template <int RB, int C>
__device__ __forceinline__ void stage_radial(float* s_w, const float* w1ef, int nb) {
  constexpr int N4 = RB * C, PER = (N4 + kThreads - 1) / kThreads;  // float4s of [RB, 4C]
  const int real4 = w1ef ? nb * C : 0;                               // float4s of the real rows
  const int tid = threadIdx.x;
  float4 v[PER];
  if (((uintptr_t)w1ef & 15) == 0) {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int k = tid + r * kThreads;
      v[r] = k < real4 ? reinterpret_cast<const float4*>(w1ef)[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  } else {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int k = tid + r * kThreads;
      v[r] = k < real4 ? make_float4(w1ef[4 * k], w1ef[4 * k + 1], w1ef[4 * k + 2], w1ef[4 * k + 3])
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int k = tid + r * kThreads;
    if (k < N4) reinterpret_cast<float4*>(s_w)[k] = v[r];
  }
  __syncthreads();
}

// CPL64 = C / 64 (the dispatch parameter); a lane holds CPL = 2 CPL64 channels of a half-wave's row.
// FZ: z is node-factored (P = z, Q = zq, radial rows w1ef and basis ef; RB > 0), else z holds
// the edge rows and zq, when given, the receiver block per atom.
template <int CPL64, bool H1, bool FZ, int RB, int WPA>
__global__ void __launch_bounds__(kThreads) message_kernel(const float* z, const float* zq, const float* geo,
                                                           const int32_t* edge_index, const int64_t* off,
                                                           const int64_t* n_edges, int64_t e_cap, int64_t n,
                                                           const int32_t* order, const float* h0, const float* h1,
                                                           float inv_avg, float* A0, float* A1, const float* ef,
                                                           const float* w1ef, int nb) {
  constexpr int CPL = 2 * CPL64, C = 32 * CPL;
  constexpr int NZ = H1 ? 4 : 2;  // z blocks in a row
  constexpr int RBV = FZ ? RB : 1;
  extern __shared__ float s_w[];  // FZ: [RB, 4C]
  __shared__ float s_red[WPA > 1 ? kWaves * 4 * C : 1];
  if constexpr (FZ) stage_radial<RB, C>(s_w, w1ef, nb);
  const int lane = threadIdx.x & 63;
  const bool upper = lane >= 32;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), sub = wib % WPA;
  const int64_t il = fmd_xcd_block(blockIdx.x, gridDim.x) * (kWaves / WPA) + wib / WPA;
  if (WPA == 1 && il >= n) return;
  const bool active = il < n;  // WPA > 1: an idle wave still takes part in the reduction
  const int64_t i = active ? (order ? order[il] : il) : 0;  // a spatial order keeps gathers in L2
  int64_t lo;
  int64_t hi = wave_rows(off, n_edges, e_cap, i, lo);
  if (!active) hi = lo;
  const int c0 = (lane & 31) * CPL;
  float a0[CPL], a1[3][CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    a0[q] = 0.f;
    a1[0][q] = a1[1][q] = a1[2][q] = 0.f;
  }
  float qz[NZ][CPL];  // the centre's receiver block of z (zq[i]), 0 when z is complete
#pragma unroll
  for (int b = 0; b < NZ; ++b) {
    if (zq) {
      load_ch<CPL>(zq + i * NZ * C + b * C + c0, qz[b]);
    } else {
#pragma unroll
      for (int q = 0; q < CPL; ++q) qz[b][q] = 0.f;
    }
  }
  for (int64_t base = lo; base < hi; base += 64) {
    const int cnt = (int)(hi - base < 64 ? hi - base : 64);
    const RowGeo m = row_geo(geo, edge_index, base + lane, lane < cnt);
    for (int u0 = 2 * kPairs * sub; u0 < cnt; u0 += 2 * kPairs * WPA) {
      float zr[kPairs][NZ][CPL], hj[kPairs][CPL], hv[kPairs][3][CPL];
      float ux[kPairs], uy[kPairs], uz[kPairs], fc[kPairs];
      float er[kPairs][RBV];
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        const int r0 = u0 + 2 * g, s0 = r0 < cnt ? r0 : cnt - 1, s1 = r0 + 1 < cnt ? r0 + 1 : cnt - 1;
        const bool valid = r0 + (upper ? 1 : 0) < cnt;
        const int s = upper ? s1 : s0;
        const int64_t j = bcast2(m.j, s0, s1, upper);
        const int ba = bperm_addr(s0, s1, upper);
        ux[g] = bperm(m.ux, ba);
        uy[g] = bperm(m.uy, ba);
        uz[g] = bperm(m.uz, ba);
        const float f = bperm(m.fc, ba);
        fc[g] = valid ? f : 0.f;  // a row past the end adds exact zeros
        const float* ze = FZ ? z + j * (NZ * C) + c0 : z + (base + s) * (NZ * C) + c0;
#pragma unroll
        for (int b = 0; b < NZ; ++b) load_ch<CPL>(ze + b * C, zr[g][b]);
        if constexpr (FZ) load_basis<RBV>(ef, nb, base + s, er[g]);
        load_ch<CPL>(h0 + j * C + c0, hj[g]);
        if (H1) {
#pragma unroll
          for (int x = 0; x < 3; ++x) load_ch<CPL>(h1 + (j * 3 + x) * C + c0, hv[g][x]);
        }
      }
      if constexpr (FZ) {
        int woff = c0;
        asm volatile("" : "+v"(woff));  // keeps the radial rows in LDS, not in registers
        add_radial<kPairs, NZ, CPL, RBV, kRadialFull>(s_w, woff, er, zr);
      }
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        // no early exit for the rows past the end (fc = 0): a branch here would let the compiler
        // move the group's loads behind it, one round trip per row again
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
          const float za = zr[g][0][q] + qz[0][q], zb = zr[g][1][q] + qz[1][q];
          const float wa = za * sigmoid(za) * fc[g], wb = zb * sigmoid(zb) * fc[g];
          const float hjq = hj[g][q];
          float m0 = wa * hjq;
          const float t = wb * hjq;
          float m1x = t * ux[g], m1y = t * uy[g], m1z = t * uz[g];
          if (H1) {
            constexpr int BC = NZ > 2 ? 2 : 0, BD = NZ > 2 ? 3 : 0;
            const float zc = zr[g][BC][q] + qz[BC][q], zd = zr[g][BD][q] + qz[BD][q];
            const float wc = zc * sigmoid(zc) * fc[g], wd = zd * sigmoid(zd) * fc[g];
            const float hx = hv[g][0][q], hy = hv[g][1][q], hz = hv[g][2][q];
            m0 += wc * (hx * ux[g] + hy * uy[g] + hz * uz[g]);
            m1x += wd * hx;
            m1y += wd * hy;
            m1z += wd * hz;
          }
          a0[q] += m0;
          a1[0][q] += m1x;
          a1[1][q] += m1y;
          a1[2][q] += m1z;
        }
      }
    }
  }
  float red[4][CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    red[0][q] = add_halves(a0[q]);
    red[1][q] = add_halves(a1[0][q]);
    red[2][q] = add_halves(a1[1][q]);
    red[3][q] = add_halves(a1[2][q]);
  }
  reduce_waves<WPA, 4, CPL>(red, s_red, wib, sub, lane);
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    a0[q] = red[0][q] * inv_avg;
    a1[0][q] = red[1][q] * inv_avg;
    a1[1][q] = red[2][q] * inv_avg;
    a1[2][q] = red[3][q] * inv_avg;
  }
  if (!active || sub != 0) return;
  // the lower half writes A0 and the x row of A1, the upper half the y and z rows
  if (!upper) {
    store_ch<CPL>(A0 + i * C + c0, a0);
    store_ch<CPL>(A1 + (i * 3 + 0) * C + c0, a1[0]);
  } else {
    store_ch<CPL>(A1 + (i * 3 + 1) * C + c0, a1[1]);
    store_ch<CPL>(A1 + (i * 3 + 2) * C + c0, a1[2]);
  }
}

// VJP, edge side (one wave per centre node i, its rows e): with gA = inv_avg * (gA0_i, gA1_i),
//   g_wa = gA0 h0_j, g_wb = h0_j (gA1 . u), g_wc = gA0 proj, g_wd = sum_x gA1_x h1_j,x
//   g_z = g_w * fcut * silu'(z)            -> gz [E, NZ C] (NZ = 4 with h1, else 2)
//   g_fcut = sum_ch g_w * silu(z), g_u_x = sum_ch (gA0 wc h1_j,x + gA1_x wb h0_j)  -> ggeo [E, 4]
// With w1ef (the radial-basis rows of the edge GEMM weight, [nb, 4C]) the kernel also forms
// gef[e, n] = sum_k gz[e, k] w1ef[n, k] (the radial block of the gather-cat row gradient) and
// gz itself may be null (not stored): the first layer needs no other part of gz @ W1^T.
// gzsum[i] = sum over the centre's rows of gz (the receiver block's gradient when zq is formed
// per atom). Rows and loads as in message_kernel (a half-wave per row); the channel sums of a
// row (radial gradients and geometry) are reduced over its half-wave.
constexpr int kMaxBasis = 16;

template <int CPL64, bool H1, int RB, bool FZ, int WPA>
__global__ void __launch_bounds__(kThreads) message_bwd_edge_kernel(
    const float* z, const float* zq, const float* geo, const int32_t* edge_index, const int64_t* off,
    const int64_t* n_edges, int64_t e_cap, int64_t n, const int32_t* order, const float* h0, const float* h1,
    const float* gA0, const float* gA1, float inv_avg, float* gz, float* gzsum, float* ggeo, int accumulate_geo,
    const float* w1ef, int nb, float* gef, const float* ef) {
  constexpr int CPL = 2 * CPL64, C = 32 * CPL;
  constexpr int NZ = H1 ? 4 : 2;
  constexpr int kPairs = H1 ? 1 : 2;  // row pairs per load group (registers: three waves per SIMD)
  // w1ef's rows padded to RB (8 or 16) with zero rows (all zero without w1ef): the radial sums
  // run over RB rows without a branch per row; FZ: the same rows form z's radial term
  extern __shared__ float s_w[];  // [RB, 4C]
  __shared__ float s_red[WPA > 1 ? kWaves * NZ * C : 1];
  const int lane = threadIdx.x & 63;
  const bool upper = lane >= 32;
  const int nbv = w1ef ? nb : 0;
  stage_radial<RB, C>(s_w, w1ef, nb);
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), sub = wib % WPA;
  const int64_t il = fmd_xcd_block(blockIdx.x, gridDim.x) * (kWaves / WPA) + wib / WPA;
  if (WPA == 1 && il >= n) return;
  const bool active = il < n;  // WPA > 1: an idle wave still takes part in the reduction
  const int64_t i = active ? (order ? order[il] : il) : 0;  // a spatial order keeps gathers in L2
  int64_t lo;
  int64_t hi = wave_rows(off, n_edges, e_cap, i, lo);
  if (!active) hi = lo;
  const int c0 = (lane & 31) * CPL;
  float g0[CPL], g1[3][CPL];
  load_ch<CPL>(gA0 + i * C + c0, g0);
#pragma unroll
  for (int x = 0; x < 3; ++x) load_ch<CPL>(gA1 + (i * 3 + x) * C + c0, g1[x]);
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    g0[q] *= inv_avg;
    g1[0][q] *= inv_avg;
    g1[1][q] *= inv_avg;
    g1[2][q] *= inv_avg;
  }
  float gs[NZ][CPL];  // sum of gz over this half's rows (in row order)
  float qz[NZ][CPL];  // the centre's receiver block of z (zq[i]), 0 when z is complete
#pragma unroll
  for (int b = 0; b < NZ; ++b) {
    if (zq) {
      load_ch<CPL>(zq + i * NZ * C + b * C + c0, qz[b]);
    } else {
#pragma unroll
      for (int q = 0; q < CPL; ++q) qz[b][q] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < CPL; ++q) gs[b][q] = 0.f;
  }
  const int t_red = half_sum16_index(lane);
  const bool writer = (lane & 1) == 0;
  for (int64_t base = lo; base < hi; base += 64) {
    const int cnt = (int)(hi - base < 64 ? hi - base : 64);
    const RowGeo m = row_geo(geo, edge_index, base + lane, lane < cnt);
    float og[4] = {0.f, 0.f, 0.f, 0.f};  // ggeo of the lane's row before this kernel (accumulating)
    if (accumulate_geo && lane < cnt) {
      const float4 t = *reinterpret_cast<const float4*>(ggeo + 4 * (base + lane));
      og[0] = t.x;
      og[1] = t.y;
      og[2] = t.z;
      og[3] = t.w;
    }
    for (int u0 = 2 * kPairs * sub; u0 < cnt; u0 += 2 * kPairs * WPA) {
      float zr[kPairs][NZ][CPL], hj[kPairs][CPL], hv[kPairs][3][CPL];
      float ux[kPairs], uy[kPairs], uz[kPairs], fc[kPairs];
      float er[kPairs][FZ ? RB : 1];
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        const int r0 = u0 + 2 * g, s0 = r0 < cnt ? r0 : cnt - 1, s1 = r0 + 1 < cnt ? r0 + 1 : cnt - 1;
        const bool valid = r0 + (upper ? 1 : 0) < cnt;
        const int s = upper ? s1 : s0;
        const int64_t j = bcast2(m.j, s0, s1, upper);
        const int ba = bperm_addr(s0, s1, upper);
        ux[g] = bperm(m.ux, ba);
        uy[g] = bperm(m.uy, ba);
        uz[g] = bperm(m.uz, ba);
        const float f = bperm(m.fc, ba);
        fc[g] = valid ? f : 0.f;  // a row past the end adds exact zeros
        const float* ze = FZ ? z + j * (NZ * C) + c0 : z + (base + s) * (NZ * C) + c0;
#pragma unroll
        for (int b = 0; b < NZ; ++b) load_ch<CPL>(ze + b * C, zr[g][b]);
        if constexpr (FZ) load_basis<RB>(ef, nb, base + s, er[g]);
        load_ch<CPL>(h0 + j * C + c0, hj[g]);
        if (H1) {
#pragma unroll
          for (int x = 0; x < 3; ++x) load_ch<CPL>(h1 + (j * 3 + x) * C + c0, hv[g][x]);
        }
      }
      if constexpr (FZ) {
        int woff = c0;
        asm volatile("" : "+v"(woff));
        add_radial<kPairs, NZ, CPL, RB, H1 ? kRadialFull : kRadialPairs>(s_w, woff, er, zr);
      }
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        // rows past the end (fc = 0) are computed and not stored: a branch around them would let
        // the compiler move the group's loads behind it
        const int r0 = u0 + 2 * g, s0 = r0 < cnt ? r0 : cnt - 1, s1 = r0 + 1 < cnt ? r0 + 1 : cnt - 1;
        const bool valid = r0 + (upper ? 1 : 0) < cnt;
        const int64_t e = base + (upper ? s1 : s0);
        float gzl[NZ][CPL];
        float sf = 0.f, su0 = 0.f, su1 = 0.f, su2 = 0.f;
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
          // with t = z s (the SiLU) its derivative is s (1 + z (1 - s)) = s + t - t s
          const float hjq = hj[g][q];
          const float gu = g1[0][q] * ux[g] + g1[1][q] * uy[g] + g1[2][q] * uz[g];
          const float za = zr[g][0][q] + qz[0][q], zb = zr[g][1][q] + qz[1][q];
          const float sa = sigmoid(za), sb = sigmoid(zb);
          const float ta = za * sa, tb = zb * sb;
          const float gwa = g0[q] * hjq, gwb = hjq * gu;
          gzl[0][q] = gwa * fc[g] * __builtin_fmaf(-ta, sa, sa + ta);
          gzl[1][q] = gwb * fc[g] * __builtin_fmaf(-tb, sb, sb + tb);
          sf += gwa * ta + gwb * tb;
          const float wbh = tb * fc[g] * hjq;
          su0 += g1[0][q] * wbh;
          su1 += g1[1][q] * wbh;
          su2 += g1[2][q] * wbh;
          if (H1) {
            constexpr int BC = NZ > 2 ? 2 : 0, BD = NZ > 2 ? 3 : 0;
            const float hx = hv[g][0][q], hy = hv[g][1][q], hz = hv[g][2][q];
            const float zc = zr[g][BC][q] + qz[BC][q], zd = zr[g][BD][q] + qz[BD][q];
            const float sc = sigmoid(zc), sd = sigmoid(zd);
            const float tc = zc * sc, td = zd * sd;
            const float proj = hx * ux[g] + hy * uy[g] + hz * uz[g];
            const float gwc = g0[q] * proj, gwd = g1[0][q] * hx + g1[1][q] * hy + g1[2][q] * hz;
            gzl[BC][q] = gwc * fc[g] * __builtin_fmaf(-tc, sc, sc + tc);
            gzl[BD][q] = gwd * fc[g] * __builtin_fmaf(-td, sd, sd + td);
            sf += gwc * tc + gwd * td;
            const float t = g0[q] * tc * fc[g];
            su0 += t * hx;
            su1 += t * hy;
            su2 += t * hz;
          }
        }
        if (gz && valid) {
          float* gze = gz + e * NZ * C + c0;
#pragma unroll
          for (int b = 0; b < NZ; ++b) store_ch_stream<CPL>(gze + b * C, gzl[b]);
        }
        if (gzsum) {
#pragma unroll
          for (int b = 0; b < NZ; ++b)
#pragma unroll
            for (int q = 0; q < CPL; ++q) gs[b][q] += gzl[b][q];
        }
        // the radial-basis gradients and the four geometry sums, reduced over the half-wave
        // together. The LDS offset is opaque to the compiler, which would otherwise keep all of
        // w1ef in registers across the loop (RB * NZ * CPL of them: fewer waves per SIMD)
        int woff = c0;
        asm volatile("" : "+v"(woff));
        float red[16];
#pragma unroll
        for (int t = 0; t < (RB == 8 ? 8 : 16); ++t) {
          const float* w = s_w + t * 4 * C + woff;
          red[t] = 0.f;
#pragma unroll
          for (int b = 0; b < NZ; ++b) {
            float wv[CPL];
            load_ch<CPL>(w + b * C, wv);
#pragma unroll
            for (int q = 0; q < CPL; ++q) red[t] += gzl[b][q] * wv[q];
          }
        }
        const int ba = bperm_addr(s0, s1, upper);
        const float o0 = bperm(og[0], ba), o1 = bperm(og[1], ba), o2 = bperm(og[2], ba), o3 = bperm(og[3], ba);
        float tg;  // the geometry sum this lane writes (index tgi), if any
        int tgi;
        if constexpr (RB == 8) {
          red[8] = su0;
          red[9] = su1;
          red[10] = su2;
          red[11] = sf;
          red[12] = red[13] = red[14] = red[15] = 0.f;
          const float tot = half_sum16(red);
          if (valid && writer && t_red < nbv) gef[e * nb + t_red] = tot;
          tg = tot;
          tgi = writer && t_red >= 8 && t_red < 12 ? t_red - 8 : -1;
        } else {
          const float tot = half_sum16(red);
          if (valid && writer && t_red < nbv) gef[e * nb + t_red] = tot;
          float g16[16] = {su0, su1, su2, sf, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          tg = half_sum16(g16);
          tgi = writer && t_red < 4 ? t_red : -1;
        }
        if (valid && tgi >= 0) {
          const float old = tgi == 0 ? o0 : tgi == 1 ? o1 : tgi == 2 ? o2 : o3;
          ggeo[4 * e + tgi] = accumulate_geo ? old + tg : tg;
        }
      }
    }
  }
  if (gzsum) {
#pragma unroll
    for (int b = 0; b < NZ; ++b)
#pragma unroll
      for (int q = 0; q < CPL; ++q) gs[b][q] = add_halves(gs[b][q]);
    reduce_waves<WPA, NZ, CPL>(gs, s_red, wib, sub, lane);
    if (!active || sub != 0) return;
    // the lower half writes blocks 0 .. NZ / 2 - 1, the upper half the rest
    float* d = gzsum + i * NZ * C + c0;
#pragma unroll
    for (int b = 0; b < NZ; ++b)
      if ((b < NZ / 2) != upper) store_ch<CPL>(d + b * C, gs[b]);
  }
}

// VJP, sender side (one wave per node j, over the reverse rows e = reverse[e'] of its rows e'
// as a centre; the receiver of e is i = neighbor[e']):
//   g_h0_j += gA0_i wa_e + wb_e (gA1_i . u_e);  g_h1_j,x += gA0_i wc_e u_e,x + gA1_i,x wd_e
// and, with gzsum_src, the sender sums of the edge pre-activation gradient,
//   gzsum_src[j] = sum over the rows e with sender j of g_z[e]   ([N, NZ C], g_z as in
// message_bwd_edge_kernel, recomputed here from z[e], zq[i], gA[i] and the sender's own h0_j,
// h1_j): the sender block of the gather-cat row gradient then is gzsum_src @ W1[:C]^T, one node
// GEMM, instead of the edge GEMM gz @ W1[:C]^T and a segment sum over [E, C] (the same sum by
// linearity) and without g_z ever in memory.
// accumulate: bit 0 adds into gh0, bit 1 into gh1 (else they are overwritten). A half-wave per
// row as in message_kernel: per 64 rows the wave loads reverse[e'], the receiver and the
// geometry of e once (a lane per row); each group of kPairs row pairs issues its z[e], zq[i],
// gA0[i] and gA1[i] loads before any arithmetic.
template <int CPL64, bool H1, bool FZ, int RB, int WPA>
__global__ void __launch_bounds__(kThreads) message_bwd_src_kernel(
    const float* z, const float* zq, const float* geo, const int32_t* edge_index, const int32_t* reverse,
    const int64_t* off, const int64_t* n_edges, int64_t e_cap, int64_t n, const int32_t* order, const float* h0,
    const float* h1, const float* gA0, const float* gA1, float inv_avg, float* gh0, float* gh1, int accumulate,
    float* gzsum_src, const float* ef, const float* w1ef, int nb) {
  constexpr int CPL = 2 * CPL64, C = 32 * CPL;
  constexpr int NZ = H1 ? 4 : 2;
  constexpr int kPairs = H1 ? 1 : 2;  // row pairs per load group (registers: three waves per SIMD)
  constexpr int RBV = FZ ? RB : 1;
  extern __shared__ float s_w[];  // FZ: [RB, 4C]
  __shared__ float s_red[WPA > 1 ? kWaves * (4 + NZ) * C : 1];
  if constexpr (FZ) stage_radial<RB, C>(s_w, w1ef, nb);
  const int lane = threadIdx.x & 63;
  const bool upper = lane >= 32;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), sub = wib % WPA;
  const int64_t jl = fmd_xcd_block(blockIdx.x, gridDim.x) * (kWaves / WPA) + wib / WPA;
  if (WPA == 1 && jl >= n) return;
  const bool active = jl < n;  // WPA > 1: an idle wave still takes part in the reduction
  const int64_t jn = active ? (order ? order[jl] : jl) : 0;  // a spatial order keeps gathers in L2
  int64_t lo;
  int64_t hi = wave_rows(off, n_edges, e_cap, jn, lo);
  if (!active) hi = lo;
  const int c0 = (lane & 31) * CPL;
  float a0[CPL], a1[3][CPL], gsum[NZ][CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) a0[q] = a1[0][q] = a1[1][q] = a1[2][q] = 0.f;
#pragma unroll
  for (int b = 0; b < NZ; ++b)
#pragma unroll
    for (int q = 0; q < CPL; ++q) gsum[b][q] = 0.f;
  // the sender's own features (the h0_j / h1_j of every row here), for the g_z sums
  float hs[CPL], hsv[3][CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) hs[q] = hsv[0][q] = hsv[1][q] = hsv[2][q] = 0.f;
  if (gzsum_src) {
    load_ch<CPL>(h0 + jn * C + c0, hs);
    if (H1) {
#pragma unroll
      for (int x = 0; x < 3; ++x) load_ch<CPL>(h1 + (jn * 3 + x) * C + c0, hsv[x]);
    }
  }
  float pz[FZ ? NZ : 1][CPL];  // FZ: the sender block of z of every row here (P[jn])
  if constexpr (FZ) {
#pragma unroll
    for (int b = 0; b < NZ; ++b) load_ch<CPL>(z + jn * (NZ * C) + b * C + c0, pz[b]);
  }
  for (int64_t base = lo; base < hi; base += 64) {
    const int cnt = (int)(hi - base < 64 ? hi - base : 64);
    int me = -1, mi = 0;
    float mux = 0.f, muy = 0.f, muz = 0.f, mfc = 0.f;
    if (lane < cnt) {
      const int64_t ep = base + lane;
      me = reverse[ep];
      mi = edge_index[2 * ep + 1];
      if (me >= 0) {
        const float4 g = *reinterpret_cast<const float4*>(geo + 8 * (int64_t)me);
        mux = g.x;
        muy = g.y;
        muz = g.z;
        mfc = geo[8 * (int64_t)me + 4];
      }
    }
    for (int u0 = 2 * kPairs * sub; u0 < cnt; u0 += 2 * kPairs * WPA) {
      float zr[kPairs][NZ][CPL], qe[kPairs][NZ][CPL], ga[kPairs][4][CPL];
      float ux[kPairs], uy[kPairs], uz[kPairs], fc[kPairs];
      float eb[kPairs][RBV];
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        const int r0 = u0 + 2 * g, s0 = r0 < cnt ? r0 : cnt - 1, s1 = r0 + 1 < cnt ? r0 + 1 : cnt - 1;
        const bool valid = r0 + (upper ? 1 : 0) < cnt;
        const int er = bcast2(me, s0, s1, upper);
        const int64_t i = bcast2(mi, s0, s1, upper);
        const int64_t e = er < 0 ? 0 : er;  // a missing reverse row reads row 0, weight 0
        const int ba = bperm_addr(s0, s1, upper);
        ux[g] = bperm(mux, ba);
        uy[g] = bperm(muy, ba);
        uz[g] = bperm(muz, ba);
        const float f = bperm(mfc, ba);
        // rows past the end and missing reverse rows add exact zeros (fc = 0)
        fc[g] = valid && er >= 0 ? f : 0.f;
        const float* ze = z + e * (NZ * C) + c0;
        if constexpr (FZ) load_basis<RBV>(ef, nb, e, eb[g]);  // the basis of row e (its own length)
#pragma unroll
        for (int b = 0; b < NZ; ++b) {
          if constexpr (FZ) {
#pragma unroll
            for (int q = 0; q < CPL; ++q) zr[g][b][q] = pz[b][q];
          } else {
            load_ch<CPL>(ze + b * C, zr[g][b]);
          }
          if (zq) {
            load_ch<CPL>(zq + i * (NZ * C) + b * C + c0, qe[g][b]);  // the receiver block of z[e] (row i)
          } else {
#pragma unroll
            for (int q = 0; q < CPL; ++q) qe[g][b][q] = 0.f;
          }
        }
        load_ch<CPL>(gA0 + i * C + c0, ga[g][0]);
#pragma unroll
        for (int x = 0; x < 3; ++x) load_ch<CPL>(gA1 + (i * 3 + x) * C + c0, ga[g][1 + x]);
      }
      if constexpr (FZ) {
        int woff = c0;
        asm volatile("" : "+v"(woff));
        add_radial<kPairs, NZ, CPL, RBV, kRadialShift>(s_w, woff, eb, zr);
      }
#pragma unroll
      for (int g = 0; g < kPairs; ++g) {
        // no branch around the zero rows: it would let the compiler move the loads behind it
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
          const float g0 = ga[g][0][q], gx = ga[g][1][q], gy = ga[g][2][q], gzv = ga[g][3][q];
          const float za = zr[g][0][q] + qe[g][0][q], zb = zr[g][1][q] + qe[g][1][q];
          // with t = z s (the SiLU) its derivative is s (1 + z (1 - s)) = s + t - t s
          const float sa = sigmoid(za), sb = sigmoid(zb);
          const float ta = za * sa, tb = zb * sb;
          const float wa = ta * fc[g], wb = tb * fc[g];
          const float gu = gx * ux[g] + gy * uy[g] + gzv * uz[g];
          a0[q] += g0 * wa + wb * gu;
          if (gzsum_src) {
            const float gwa = g0 * hs[q], gwb = hs[q] * gu;
            gsum[0][q] += gwa * fc[g] * __builtin_fmaf(-ta, sa, sa + ta);
            gsum[1][q] += gwb * fc[g] * __builtin_fmaf(-tb, sb, sb + tb);
          }
          if (H1) {
            constexpr int BC = NZ > 2 ? 2 : 0, BD = NZ > 2 ? 3 : 0;
            const float zc = zr[g][BC][q] + qe[g][BC][q], zd = zr[g][BD][q] + qe[g][BD][q];
            const float sc = sigmoid(zc), sd = sigmoid(zd);
            const float tc = zc * sc, td = zd * sd;
            const float wc = tc * fc[g], wd = td * fc[g];
            const float t = g0 * wc;
            a1[0][q] += t * ux[g] + gx * wd;
            a1[1][q] += t * uy[g] + gy * wd;
            a1[2][q] += t * uz[g] + gzv * wd;
            if (gzsum_src) {
              const float hx = hsv[0][q], hy = hsv[1][q], hz = hsv[2][q];
              const float gwc = g0 * (hx * ux[g] + hy * uy[g] + hz * uz[g]);
              const float gwd = gx * hx + gy * hy + gzv * hz;
              gsum[BC][q] += gwc * fc[g] * __builtin_fmaf(-tc, sc, sc + tc);
              gsum[BD][q] += gwd * fc[g] * __builtin_fmaf(-td, sd, sd + td);
            }
          }
        }
      }
    }
  }
  // the per-node sums: a0, a1 and (with gzsum_src) gsum, over the halves and the atom's waves
  float red[4 + NZ][CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    red[0][q] = add_halves(a0[q]);
    red[1][q] = H1 ? add_halves(a1[0][q]) : 0.f;
    red[2][q] = H1 ? add_halves(a1[1][q]) : 0.f;
    red[3][q] = H1 ? add_halves(a1[2][q]) : 0.f;
#pragma unroll
    for (int b = 0; b < NZ; ++b) red[4 + b][q] = gzsum_src ? add_halves(gsum[b][q]) : 0.f;
  }
  reduce_waves<WPA, 4 + NZ, CPL>(red, s_red, wib, sub, lane);
  if (!active || sub != 0) return;
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    a0[q] = red[0][q] * inv_avg;
    if (H1) {
      a1[0][q] = red[1][q] * inv_avg;
      a1[1][q] = red[2][q] * inv_avg;
      a1[2][q] = red[3][q] * inv_avg;
    }
#pragma unroll
    for (int b = 0; b < NZ; ++b) gsum[b][q] = red[4 + b][q];
  }
  // the lower half writes gh0 and the x row of gh1, the upper half the y and z rows
  if (gh0 && !upper) {
    float* d0 = gh0 + jn * C + c0;
    float v0[CPL];
    if (accumulate & 1) {
      load_ch<CPL>(d0, v0);
#pragma unroll
      for (int q = 0; q < CPL; ++q) v0[q] += a0[q];
    } else {
#pragma unroll
      for (int q = 0; q < CPL; ++q) v0[q] = a0[q];
    }
    store_ch<CPL>(d0, v0);
  }
  if (H1 && gh1) {
#pragma unroll
    for (int x = 0; x < 3; ++x) {
      if ((x == 0) == upper) continue;
      float* d1 = gh1 + (jn * 3 + x) * C + c0;
      float v1[CPL];
      if (accumulate & 2) {
        load_ch<CPL>(d1, v1);
#pragma unroll
        for (int q = 0; q < CPL; ++q) v1[q] += a1[x][q];
      } else {
#pragma unroll
        for (int q = 0; q < CPL; ++q) v1[q] = a1[x][q];
      }
      store_ch<CPL>(d1, v1);
    }
  }
  if (gzsum_src) {
#pragma unroll
    for (int b = 0; b < NZ; ++b)
#pragma unroll
      for (int q = 0; q < CPL; ++q) gsum[b][q] = gsum[b][q] * inv_avg;
    // the lower half writes blocks 0 .. NZ / 2 - 1, the upper half the rest
    float* d = gzsum_src + jn * NZ * C + c0;
#pragma unroll
    for (int b = 0; b < NZ; ++b)
      if ((b < NZ / 2) != upper) store_ch<CPL>(d + b * C, gsum[b]);
  }
}

// ------------------------------------------------------------------------------------------
// symmetric contraction (correlation order 3, L <= 1), per node and channel, element weights
//   n1 = |P1|^2;  B0 = c1 P0 + c2 P0^2 + c3 n1 + c4 P0^3 + c5 P0 n1
//   B1_x = (d1 + d2 P0 + d3 P0^2 + d4 n1) P1_x
// Wc [nel, 5, C], Wd [nel, 4, C]; elem[i] the element index of node i.
// ------------------------------------------------------------------------------------------
__global__ void symcon_kernel(const float* P0, const float* P1, const int32_t* elem, const float* Wc,
                              const float* Wd, int64_t n, int C, float* B0, float* B1) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n * C) return;
  const int64_t i = k / C;
  const int ch = (int)(k - i * C);
  const int el = elem[i];
  const float p0 = P0[k];
  const float px = P1[(i * 3 + 0) * C + ch], py = P1[(i * 3 + 1) * C + ch], pz = P1[(i * 3 + 2) * C + ch];
  const float n1 = px * px + py * py + pz * pz;
  B0[k] = symcon_b0(p0, n1, Wc + (int64_t)el * 5 * C + ch, C);
  if (B1) {
    const float q = symcon_q(p0, n1, Wd + (int64_t)el * 4 * C + ch, C);
    B1[(i * 3 + 0) * C + ch] = q * px;
    B1[(i * 3 + 1) * C + ch] = q * py;
    B1[(i * 3 + 2) * C + ch] = q * pz;
  }
}

__global__ void symcon_bwd_kernel(const float* P0, const float* P1, const int32_t* elem, const float* Wc,
                                  const float* Wd, const float* gB0, const float* gB1, int64_t n, int C, float* gP0,
                                  float* gP1) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n * C) return;
  const int64_t i = k / C;
  const int ch = (int)(k - i * C);
  const int el = elem[i];
  const float p[3] = {P1[(i * 3 + 0) * C + ch], P1[(i * 3 + 1) * C + ch], P1[(i * 3 + 2) * C + ch]};
  float gb1[3] = {0.f, 0.f, 0.f};
  if (gB1)
    for (int x = 0; x < 3; ++x) gb1[x] = gB1[(i * 3 + x) * C + ch];
  float gp0, gp[3];
  symcon_vjp(P0[k], p, Wc + (int64_t)el * 5 * C + ch, Wd + (int64_t)el * 4 * C + ch, C, gB0[k], gB1 != nullptr, gb1,
             gp0, gp);
  gP0[k] = gp0;
#pragma unroll
  for (int x = 0; x < 3; ++x) gP1[(i * 3 + x) * C + ch] = gp[x];
}

// ------------------------------------------------------------------------------------------
// readout and node energy: one wave per node
//   E_i = E0[elem_i] + scale * (h_a,i . wr1 + sum_k silu(y_i,k) wr2b_k) + shift
// VJP: gha_i = scale gE_i wr1, gy_i,k = scale gE_i wr2b_k silu'(y_i,k)
// ------------------------------------------------------------------------------------------
__global__ void energy_kernel(const float* ha, const float* wr1, const float* y, const float* wr2b, int C, int H,
                              const int32_t* elem, const float* e0, float scale, float shift, int64_t n, float* energy) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / 64;
  if (i >= n) return;
  float s = 0.f;
  for (int c = lane; c < C; c += 64) s += ha[i * C + c] * wr1[c];
  for (int k = lane; k < H; k += 64) {
    const float v = y[i * H + k];
    s += v * sigmoid(v) * wr2b[k];
  }
  s = wave_sum(s);
  if (lane == 0) energy[i] = e0[elem[i]] + scale * s + shift;
}

// gy of one readout unit: g wr2b_k silu'(y_k) (shared by the VJP kernel and the fused forward)
__device__ __forceinline__ float readout_gy(float g, float w, float v) {
  const float sg = sigmoid(v);
  return g * w * sg * (1.0f + v * (1.0f - sg));
}

// The forward with the VJP for dE/dE_i = 1 (the explicit force path: no seed to wait for): E_i as
// energy_kernel, and in the same wave gha_i = scale wr1, gy_i = scale wr2b silu'(y_i) (the values
// energy_bwd_kernel writes for a null gE), one launch instead of two.
__global__ void zero_f64_kernel(double* x) { x[0] = 0.0; }

// The float64 total of x[0 .. n) in fmd_sum_f64's fixed order (1 024 strided partials in index
// order, then a pairwise tree over them), formed by the threads of one block.
__device__ void sum_f64_order(const float* x, int64_t n, double* out, double* part) {
  constexpr int kParts = 1024, kU = 8;
  for (int v = threadIdx.x; v < kParts; v += blockDim.x) {
    // the same adds in the same order; eight loads in flight before their adds
    double s = 0.0;
    int64_t k = v;
    for (; k + (kU - 1) * kParts < n; k += kU * kParts) {
      float t[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) t[u] = x[k + u * kParts];
#pragma unroll
      for (int u = 0; u < kU; ++u) s = s + (double)t[u];
    }
    for (; k < n; k += kParts) s = s + (double)x[k];
    part[v] = s;
  }
  __syncthreads();
  for (int width = kParts / 2; width > 0; width >>= 1) {
    for (int v = threadIdx.x; v < width; v += blockDim.x) part[v] = part[v] + part[v + width];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = part[0];
}

// With total (and its completion counter): every block publishes its energies with a
// device-scope fence before it counts itself; the last block to count fences again, forms the
// fixed-order float64 total of all n energies and sets the counter back to zero for the next
// launch (no separate summing launch). A device-scope fence writes back the L2, so this is for
// small launches (a few hundred blocks); large ones sum in a launch of their own.
__global__ void energy_grad_kernel(const float* ha, const float* wr1, const float* y, const float* wr2b, int C, int H,
                                   const int32_t* elem, const float* e0, float scale, float shift, int64_t n,
                                   float* energy, float* gha, float* gy, double* total, unsigned int* counter) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / 64;
  if (i < n) {
    float s = 0.f;
    for (int c = lane; c < C; c += 64) {
      const float w = wr1[c];
      s += ha[i * C + c] * w;
      gha[i * C + c] = scale * w;
    }
    for (int k = lane; k < H; k += 64) {
      const float v = y[i * H + k], w = wr2b[k];
      s += v * sigmoid(v) * w;
      gy[i * H + k] = readout_gy(scale, w, v);
    }
    s = wave_sum(s);
    if (lane == 0) energy[i] = e0[elem[i]] + scale * s + shift;
  }
  if (!total) return;
  __shared__ int last;
  __shared__ double part[1024];
  __syncthreads();  // the block's energies are written; thread 0's device-scope fence publishes them
  if (threadIdx.x == 0) {
    __threadfence();
    last = atomicAdd(counter, 1u) == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  sum_f64_order(energy, n, total, part);
  if (threadIdx.x == 0) atomicExch(counter, 0u);
}

__global__ void energy_bwd_kernel(const float* gE, const float* wr1, const float* y, const float* wr2b, int C, int H,
                                  float scale, int64_t n, float* gha, float* gy) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = n * (C + H);
  if (k >= total) return;
  const int64_t i = k / (C + H);
  const int c = (int)(k - i * (C + H));
  const float g = gE ? scale * gE[i] : scale;  // null gE: dE/dE_i = 1 for every row
  if (c < C) {
    gha[i * C + c] = g * wr1[c];
  } else {
    const int h = c - C;
    gy[i * H + h] = readout_gy(g, wr2b[h], y[i * H + h]);
  }
}

// h0[i] = table[elem[i]]  (element embedding)
__global__ void embed_kernel(const int32_t* elem, const float* table, int64_t n, int C, float* h0) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n * C) return;
  const int64_t i = k / C;
  h0[k] = table[(int64_t)elem[i] * C + (k - i * C)];
}

// Several per-element tables gathered in one launch: out_g[i] = table_g[elem[i]] (widths in
// float4 units); one thread per float4 of the concatenated rows of an atom.
constexpr int kMaxEmbed = 8;
struct EmbedSet {
  const float4* table[kMaxEmbed];
  float4* out[kMaxEmbed];
  int width4[kMaxEmbed];
  int start4[kMaxEmbed + 1];
  int count;
};

__device__ __forceinline__ void embed_row(const int32_t* elem, int64_t n, const EmbedSet& s, int64_t k) {
  const int total = s.start4[s.count];
  if (k >= n * total) return;
  const int64_t i = k / total;
  int c = (int)(k - i * total);
  int g = 0;
#pragma unroll
  for (int q = 1; q < kMaxEmbed; ++q)
    if (q < s.count && c >= s.start4[q]) g = q;
  c -= s.start4[g];
  s.out[g][i * s.width4[g] + c] = s.table[g][(int64_t)elem[i] * s.width4[g] + c];
}

__global__ void embed_rows_kernel(const int32_t* elem, int64_t n, const EmbedSet s) {
  embed_row(elem, n, s, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// The edge geometry (blocks [0, geo_blocks)) and the per-element gathers (the rest) in one launch:
// two independent passes at the start of a force evaluation.
__global__ void geometry_embed_kernel(const GeoArgs a, int64_t geo_blocks, const int32_t* elem, int64_t n,
                                      const EmbedSet s) {
  if ((int64_t)blockIdx.x < geo_blocks) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < a.e_cap) edge_geometry_row(a, e);
  } else {
    embed_row(elem, n, s, ((int64_t)blockIdx.x - geo_blocks) * blockDim.x + threadIdx.x);
  }
}

// ------------------------------------------------------------------------------------------
// Morse pair potential, shifted to zero at the cutoff: per centre node (one thread per node):
//   E_i = 1/2 sum_e V(r_e),  V = D[(1 - exp(-a(r - r0)))^2 - 1] - V_rc (r < rc, else 0)
//   dvdr[e] = V'(r_e) (0 beyond the cutoff)
// ------------------------------------------------------------------------------------------
__global__ void morse_kernel(const float* geo, const int64_t* off, const int64_t* n_edges, int64_t e_cap, int64_t n,
                             float D, float a, float r0, float rc, float vshift, float* energy, float* dvdr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t rows = real_rows(n_edges, e_cap);
  int64_t lo = off[i], hi = off[i + 1];
  hi = hi < rows ? hi : rows;
  lo = lo < hi ? lo : hi;
  float s = 0.f;
  for (int64_t e = lo; e < hi; ++e) {
    const float r = geo[8 * e + 3];
    float v = 0.f, dv = 0.f;
    if (r < rc) {
      const float ex = __expf(-a * (r - r0));
      const float om = 1.0f - ex;
      v = D * (om * om - 1.0f) - vshift;
      dv = 2.0f * D * om * a * ex;
    }
    s += v;
    dvdr[e] = dv;
  }
  energy[i] = 0.5f * s;
}

// g_geo[e] = (0, 0, 0, 0) and g_r folded into g_vec directly: gvec[e] = 0.5 gE[c] V'(r) u
__global__ void morse_bwd_kernel(const float* geo, const float* dvdr, const int32_t* edge_index, const float* gE,
                                 const int64_t* n_edges, int64_t e_cap, float* gvec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= e_cap) return;
  const int64_t rows = real_rows(n_edges, e_cap);
  if (e >= rows) {
    gvec[3 * e] = gvec[3 * e + 1] = gvec[3 * e + 2] = 0.f;
    return;
  }
  const float g = 0.5f * gE[edge_index[2 * e]] * dvdr[e];
  gvec[3 * e] = g * geo[8 * e];
  gvec[3 * e + 1] = g * geo[8 * e + 1];
  gvec[3 * e + 2] = g * geo[8 * e + 2];
}

// ------------------------------------------------------------------------------------------
// Virial of the edge vectors: M_ab = sum_e v_e,a * (dE/dv_e)_b, the derivative of the energy
// under the strain v -> v (I + S) of every edge vector (positions and cell strained together
// move every edge that way). v = u r from the geometry row (u, r). Float64 products and sums
// in a fixed order: a fixed grid of kVirialBlocks blocks strides over the real rows, each block
// writes its 9 partial sums, and one workgroup adds the partials block by block.
// ------------------------------------------------------------------------------------------
constexpr int kVirialBlocks = 256;

__global__ void __launch_bounds__(kThreads) edge_virial_kernel(const float* geo, const float* gvec,
                                                               const int64_t* n_edges, int64_t e_cap, double* part) {
  __shared__ double red[9][kThreads];
  const int64_t rows = real_rows(n_edges, e_cap);
  double m[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) m[k] = 0.0;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < rows; e += (int64_t)kVirialBlocks * kThreads) {
    const float4 g = reinterpret_cast<const float4*>(geo)[2 * e];
    const double v[3] = {(double)g.x * (double)g.w, (double)g.y * (double)g.w, (double)g.z * (double)g.w};
    const double d[3] = {(double)gvec[3 * e], (double)gvec[3 * e + 1], (double)gvec[3 * e + 2]};
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) m[3 * a + b] = m[3 * a + b] + v[a] * d[b];
  }
#pragma unroll
  for (int k = 0; k < 9; ++k) red[k][threadIdx.x] = m[k];
  __syncthreads();
  for (int width = kThreads / 2; width > 0; width >>= 1) {
    if ((int)threadIdx.x < width)
#pragma unroll
      for (int k = 0; k < 9; ++k) red[k][threadIdx.x] = red[k][threadIdx.x] + red[k][threadIdx.x + width];
    __syncthreads();
  }
  if (threadIdx.x < 9) part[9 * blockIdx.x + threadIdx.x] = red[threadIdx.x][0];
}

// stress = (M + M^T) / (2 V), V = |c0 . (c1 x c2)| of the unstrained cell (float64 from the
// float32 rows); one wave
__global__ void virial_stress_kernel(const double* part, const float* cell, float* stress) {
  __shared__ double m[9];
  const int t = threadIdx.x;
  if (t < 9) {
    double s = 0.0;
    for (int b = 0; b < kVirialBlocks; ++b) s = s + part[9 * b + t];
    m[t] = s;
  }
  __syncthreads();
  if (t < 9) {
    double c[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) c[k] = (double)cell[k];
    const double cross0 = c[4] * c[8] - c[5] * c[7];
    const double cross1 = c[5] * c[6] - c[3] * c[8];
    const double cross2 = c[3] * c[7] - c[4] * c[6];
    const double vol = fabs(c[0] * cross0 + c[1] * cross1 + c[2] * cross2);
    const int a = t / 3, b = t % 3;
    stress[t] = (float)(0.5 * (m[3 * a + b] + m[3 * b + a]) / vol);
  }
}

template <int CPL, int WPA>
int launch_message(bool h1, bool fz, int rb, hipStream_t s, const float* z, const float* zq,
                   const float* geo, const int32_t* ei, const int64_t* off, const int64_t* ne, int64_t e_cap, int64_t n,
                   const int32_t* order, const float* h0, const float* h1p, float inv_avg, float* A0, float* A1,
                   const float* ef, const float* w1ef, int nb) {
  const size_t lds = fz ? (size_t)rb * 4 * 64 * CPL * sizeof(float) : 0;  // [RB, 4C]
  const dim3 grid((unsigned)fmd_cdiv(n * WPA, kWaves));
#define FMD_MSG(H, F, R)                                                                                       \
  hipLaunchKernelGGL((message_kernel<CPL, H, F, R, WPA>), grid, dim3(kThreads), lds, s, z, zq, geo, ei, off, ne, \
                     e_cap, n, order, h0, h1p, inv_avg, A0, A1, ef, w1ef, nb)
  if (!fz) {
    if (h1)
      FMD_MSG(true, false, 0);
    else
      FMD_MSG(false, false, 0);
  } else if (rb == 8) {
    if (h1)
      FMD_MSG(true, true, 8);
    else
      FMD_MSG(false, true, 8);
  } else {
    if (h1)
      FMD_MSG(true, true, 16);
    else
      FMD_MSG(false, true, 16);
  }
#undef FMD_MSG
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // namespace

// the message kernels load a lane's channels as vectors: the per-node and per-row arrays start on
// 8-byte (C = 64) or 16-byte boundaries, geo and ggeo on 16 bytes
static bool aligned_to(uintptr_t a, std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (p && ((uintptr_t)p % a) != 0) return false;
  return true;
}

// a lane's CPL = C / 32 channels: 8-byte loads for C = 64, 16-byte loads above
static uintptr_t channel_alignment(int channels) { return channels <= 64 ? 8 : 16; }

#define FMD_CPL_DISPATCH(C, FN, ...)                 \
  switch ((C) / 64) {                                \
    case 1: return FN<1>(__VA_ARGS__);               \
    case 2: return FN<2>(__VA_ARGS__);               \
    case 4: return FN<4>(__VA_ARGS__);               \
    default: return FMD_EUNSUPPORTED;                \
  }

namespace {
template <int CPL, int WPA>
int launch_bwd_edge(bool h1, bool fz, hipStream_t s, const float* z, const float* zq, const float* geo,
                    const int32_t* ei, const int64_t* off, const int64_t* ne, int64_t e_cap, int64_t n,
                    const int32_t* order, const float* h0, const float* h1p, const float* gA0, const float* gA1,
                    float inv_avg, float* gz, float* gzsum, float* ggeo, int acc, const float* w1ef, int nb, float* gef,
                    const float* ef) {
  const bool wide = w1ef && nb > 8;  // radial rows padded to 16 instead of 8
  const size_t lds = (size_t)(wide ? 16 : 8) * 4 * 64 * CPL * sizeof(float);  // RB x 4C floats
  const dim3 grid((unsigned)fmd_cdiv(n * WPA, kWaves));
#define FMD_BWD_EDGE(H, RB, F)                                                                                   \
  hipLaunchKernelGGL((message_bwd_edge_kernel<CPL, H, RB, F, WPA>), grid, dim3(kThreads), lds, s, z, zq, geo, ei, \
                     off, ne, e_cap, n, order, h0, h1p, gA0, gA1, inv_avg, gz, gzsum, ggeo, acc, w1ef, nb, gef, ef)
#define FMD_BWD_EDGE_F(H, RB) \
  if (fz)                     \
    FMD_BWD_EDGE(H, RB, true); \
  else                        \
    FMD_BWD_EDGE(H, RB, false)
  if (h1 && wide) {
    FMD_BWD_EDGE_F(true, 16);
  } else if (h1) {
    FMD_BWD_EDGE_F(true, 8);
  } else if (wide) {
    FMD_BWD_EDGE_F(false, 16);
  } else {
    FMD_BWD_EDGE_F(false, 8);
  }
#undef FMD_BWD_EDGE_F
#undef FMD_BWD_EDGE
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

template <int CPL, int WPA>
int launch_bwd_src(bool h1, bool fz, int rb, hipStream_t s, const float* z, const float* zq,
                   const float* geo, const int32_t* ei, const int32_t* rev, const int64_t* off, const int64_t* ne,
                   int64_t e_cap, int64_t n, const int32_t* order, const float* h0, const float* h1p, const float* gA0,
                   const float* gA1, float inv_avg, float* gh0, float* gh1, int acc, float* gzsum_src, const float* ef,
                   const float* w1ef, int nb) {
  const size_t lds = fz ? (size_t)rb * 4 * 64 * CPL * sizeof(float) : 0;
  const dim3 grid((unsigned)fmd_cdiv(n * WPA, kWaves));
#define FMD_BWD_SRC(H, F, R)                                                                                       \
  hipLaunchKernelGGL((message_bwd_src_kernel<CPL, H, F, R, WPA>), grid, dim3(kThreads), lds, s, z, zq, geo, ei, rev, \
                     off, ne, e_cap, n, order, h0, h1p, gA0, gA1, inv_avg, gh0, gh1, acc, gzsum_src, ef, w1ef, nb)
  if (!fz) {
    if (h1)
      FMD_BWD_SRC(true, false, 0);
    else
      FMD_BWD_SRC(false, false, 0);
  } else if (rb == 8) {
    if (h1)
      FMD_BWD_SRC(true, true, 8);
    else
      FMD_BWD_SRC(false, true, 8);
  } else {
    if (h1)
      FMD_BWD_SRC(true, true, 16);
    else
      FMD_BWD_SRC(false, true, 16);
  }
#undef FMD_BWD_SRC
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}
}  // namespace

extern "C" {

int fmd_edge_geometry_f32(const float* positions, const float* cell, const int32_t* system_of,
                          const int32_t* edge_index, const float* edge_image, const int64_t* n_edges, int64_t e_cap,
                          float rc, int32_t nb, float* geo, float* ef, float* def, hipStream_t stream) {
  FMD_REQUIRE(positions && cell && edge_index && edge_image && n_edges && geo && ef && def);
  FMD_REQUIRE(e_cap >= 0 && nb > 0 && rc > 0.f);
  if (e_cap == 0) return FMD_OK;
  const GeoArgs a{positions, cell, system_of, edge_index, edge_image, n_edges, e_cap, rc, nb, geo, ef, def};
  hipLaunchKernelGGL(edge_geometry_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, a);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_edge_geometry_bwd_f32(const float* geo, const float* def, int32_t nb, const float* gef0, int64_t ld0,
                              const float* gef1, int64_t ld1, const float* ggeo, const int64_t* n_edges,
                              int64_t e_cap, float* gvec, hipStream_t stream) {
  FMD_REQUIRE(geo && def && n_edges && gvec && e_cap >= 0 && nb > 0);
  if (e_cap == 0) return FMD_OK;
  hipLaunchKernelGGL(edge_geometry_bwd_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, geo, def,
                     nb, gef0, ld0, gef1, ld1, ggeo, n_edges, e_cap, gvec);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

// one or four waves per atom (the launchers' WPA)
#define FMD_WPA_DISPATCH(WPA_ARG, FN, CPLV, ...)                 \
  ((WPA_ARG) == 4 ? FN<CPLV, 4>(__VA_ARGS__) : FN<CPLV, 1>(__VA_ARGS__))

int fmd_mace_message_f32(const float* z, const float* zq, const float* geo, const int32_t* edge_index,
                         const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap, int64_t n_atoms,
                         const int32_t* order, int32_t channels, const float* h0, const float* h1, float inv_avg,
                         float* A0, float* A1, int32_t z_per_node, const float* ef, const float* w1ef, int32_t nb,
                         int32_t waves_per_atom, hipStream_t stream) {
  FMD_REQUIRE(z && geo && edge_index && edge_offsets && n_edges && h0 && A0 && A1 && n_atoms >= 0);
  FMD_REQUIRE(!z_per_node || (zq && ef && w1ef && nb > 0 && nb <= kMaxBasis));
  FMD_REQUIRE(waves_per_atom == 1 || waves_per_atom == 4);
  FMD_REQUIRE(aligned_to(channel_alignment(channels), {z, zq, h0, h1, A0, A1}) && aligned_to(16, {geo, ef}));
  if (n_atoms == 0) return FMD_OK;
  const int rb = nb > 8 ? 16 : 8;
  const bool fz = z_per_node != 0, hv = h1 != nullptr;
  switch (channels / 64) {
    case 1: return FMD_WPA_DISPATCH(waves_per_atom, launch_message, 1, hv, fz, rb, stream, z, zq, geo, edge_index,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, inv_avg, A0, A1, ef, w1ef, nb);
    case 2: return FMD_WPA_DISPATCH(waves_per_atom, launch_message, 2, hv, fz, rb, stream, z, zq, geo, edge_index,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, inv_avg, A0, A1, ef, w1ef, nb);
    case 4: return FMD_WPA_DISPATCH(waves_per_atom, launch_message, 4, hv, fz, rb, stream, z, zq, geo, edge_index,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, inv_avg, A0, A1, ef, w1ef, nb);
    default: return FMD_EUNSUPPORTED;
  }
}

int fmd_mace_message_bwd_f32(const float* z, const float* zq, const float* geo, const int32_t* edge_index,
                             const int32_t* reverse,
                             const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap, int64_t n_atoms,
                             const int32_t* order, int32_t channels, const float* h0, const float* h1,
                             const float* gA0, const float* gA1,
                             float inv_avg, float* gz, float* gzsum, float* gzsum_src, float* ggeo,
                             int32_t accumulate_geo, float* gh0, float* gh1, int32_t accumulate_h, const float* w1ef,
                             int32_t nb, float* gef, int32_t z_per_node, const float* ef, int32_t waves_per_atom,
                             hipStream_t stream) {
  FMD_REQUIRE(z && geo && edge_index && edge_offsets && n_edges && h0 && gA0 && gA1 && ggeo && n_atoms >= 0);
  FMD_REQUIRE(gz || w1ef || gzsum);
  FMD_REQUIRE(!w1ef || (gef && nb > 0 && nb <= kMaxBasis));
  FMD_REQUIRE(!z_per_node || (zq && ef && w1ef && !gz));
  FMD_REQUIRE(!(gh0 || gzsum_src) || reverse);
  FMD_REQUIRE(waves_per_atom == 1 || waves_per_atom == 4);
  FMD_REQUIRE(aligned_to(channel_alignment(channels), {z, zq, h0, h1, gA0, gA1, gz, gzsum, gzsum_src, gh0, gh1}) &&
              aligned_to(16, {geo, ggeo, ef}));
  if (n_atoms == 0) return FMD_OK;
  const bool fz = z_per_node != 0, hv = h1 != nullptr;
  const int rb = nb > 8 ? 16 : 8;
  // accumulate_h bit 2: the sender-side kernel alone (the edge side ran in a call before)
  const bool sender_only = (accumulate_h & 4) != 0;
  accumulate_h &= 3;
  const int w = waves_per_atom;
  int rc = FMD_OK;
  if (!sender_only) switch (channels / 64) {
    case 1: rc = FMD_WPA_DISPATCH(w, launch_bwd_edge, 1, hv, fz, stream, z, zq, geo, edge_index, edge_offsets,
                                  n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gz, gzsum, ggeo,
                                  accumulate_geo, w1ef, nb, gef, ef); break;
    case 2: rc = FMD_WPA_DISPATCH(w, launch_bwd_edge, 2, hv, fz, stream, z, zq, geo, edge_index, edge_offsets,
                                  n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gz, gzsum, ggeo,
                                  accumulate_geo, w1ef, nb, gef, ef); break;
    case 4: rc = FMD_WPA_DISPATCH(w, launch_bwd_edge, 4, hv, fz, stream, z, zq, geo, edge_index, edge_offsets,
                                  n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gz, gzsum, ggeo,
                                  accumulate_geo, w1ef, nb, gef, ef); break;
    default: return FMD_EUNSUPPORTED;
  }
  if (rc != FMD_OK || !(gh0 || gzsum_src)) return rc;
  switch (channels / 64) {
    case 1: return FMD_WPA_DISPATCH(w, launch_bwd_src, 1, hv, fz, rb, stream, z, zq, geo, edge_index, reverse,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gh0, gh1,
                                    accumulate_h, gzsum_src, ef, w1ef, nb);
    case 2: return FMD_WPA_DISPATCH(w, launch_bwd_src, 2, hv, fz, rb, stream, z, zq, geo, edge_index, reverse,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gh0, gh1,
                                    accumulate_h, gzsum_src, ef, w1ef, nb);
    case 4: return FMD_WPA_DISPATCH(w, launch_bwd_src, 4, hv, fz, rb, stream, z, zq, geo, edge_index, reverse,
                                    edge_offsets, n_edges, e_cap, n_atoms, order, h0, h1, gA0, gA1, inv_avg, gh0, gh1,
                                    accumulate_h, gzsum_src, ef, w1ef, nb);
    default: return FMD_EUNSUPPORTED;
  }
}

int fmd_mace_symcon_f32(const float* P0, const float* P1, const int32_t* elem, const float* Wc, const float* Wd,
                        int64_t n_atoms, int32_t channels, float* B0, float* B1, hipStream_t stream) {
  FMD_REQUIRE(P0 && P1 && elem && Wc && B0 && (!B1 || Wd) && n_atoms >= 0 && channels > 0);
  if (n_atoms == 0) return FMD_OK;
  const int64_t total = n_atoms * channels;
  hipLaunchKernelGGL(symcon_kernel, dim3((unsigned)fmd_cdiv(total, 256)), dim3(256), 0, stream, P0, P1, elem, Wc, Wd,
                     n_atoms, channels, B0, B1);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_symcon_bwd_f32(const float* P0, const float* P1, const int32_t* elem, const float* Wc, const float* Wd,
                            const float* gB0, const float* gB1, int64_t n_atoms, int32_t channels, float* gP0,
                            float* gP1, hipStream_t stream) {
  FMD_REQUIRE(P0 && P1 && elem && Wc && gB0 && gP0 && gP1 && (!gB1 || Wd) && n_atoms >= 0 && channels > 0);
  if (n_atoms == 0) return FMD_OK;
  const int64_t total = n_atoms * channels;
  hipLaunchKernelGGL(symcon_bwd_kernel, dim3((unsigned)fmd_cdiv(total, 256)), dim3(256), 0, stream, P0, P1, elem, Wc,
                     Wd, gB0, gB1, n_atoms, channels, gP0, gP1);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_energy_f32(const float* ha, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                        int32_t hidden, const int32_t* elem, const float* e0, float scale, float shift,
                        int64_t n_atoms, float* energy, hipStream_t stream) {
  FMD_REQUIRE(ha && wr1 && y && wr2b && elem && e0 && energy && n_atoms >= 0);
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(energy_kernel, dim3((unsigned)fmd_cdiv(n_atoms, kWaves)), dim3(kThreads), 0, stream, ha, wr1, y,
                     wr2b, channels, hidden, elem, e0, scale, shift, n_atoms, energy);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_energy_grad_f32(const float* ha, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                             int32_t hidden, const int32_t* elem, const float* e0, float scale, float shift,
                             int64_t n_atoms, float* energy, float* gha, float* gy, double* total,
                             uint32_t* counter, hipStream_t stream) {
  FMD_REQUIRE(ha && wr1 && y && wr2b && elem && e0 && energy && gha && gy && n_atoms >= 0 && (!total || counter));
  if (n_atoms == 0) {
    if (total) {  // the empty sum (a kernel, not a memset node: callers capture this launch)
      hipLaunchKernelGGL(zero_f64_kernel, dim3(1), dim3(1), 0, stream, total);
      FMD_CHECK_LAUNCH();
    }
    return FMD_OK;
  }
  hipLaunchKernelGGL(energy_grad_kernel, dim3((unsigned)fmd_cdiv(n_atoms, kWaves)), dim3(kThreads), 0, stream, ha,
                     wr1, y, wr2b, channels, hidden, elem, e0, scale, shift, n_atoms, energy, gha, gy, total,
                     reinterpret_cast<unsigned int*>(counter));
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_energy_bwd_f32(const float* gE, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                            int32_t hidden, float scale, int64_t n_atoms, float* gha, float* gy, hipStream_t stream) {
  FMD_REQUIRE(wr1 && y && wr2b && gha && gy && n_atoms >= 0);
  if (n_atoms == 0) return FMD_OK;
  const int64_t total = n_atoms * (channels + hidden);
  hipLaunchKernelGGL(energy_bwd_kernel, dim3((unsigned)fmd_cdiv(total, 256)), dim3(256), 0, stream, gE, wr1, y, wr2b,
                     channels, hidden, scale, n_atoms, gha, gy);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_embed_f32(const int32_t* elem, const float* table, int64_t n_atoms, int32_t channels, float* h0,
                  hipStream_t stream) {
  FMD_REQUIRE(elem && table && h0 && n_atoms >= 0 && channels > 0);
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)fmd_cdiv(n_atoms * channels, 256)), dim3(256), 0, stream, elem,
                     table, n_atoms, channels, h0);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"

namespace {
int embed_set(int32_t count, const float* const* tables, const int32_t* widths, float* const* outs, EmbedSet& set) {
  FMD_REQUIRE(count >= 1 && count <= kMaxEmbed && tables && widths && outs);
  set = EmbedSet{};
  set.count = count;
  set.start4[0] = 0;
  for (int g = 0; g < count; ++g) {
    FMD_REQUIRE(tables[g] && outs[g] && widths[g] > 0 && widths[g] % 4 == 0);
    FMD_REQUIRE(aligned_to(16, {tables[g], outs[g]}));
    set.table[g] = reinterpret_cast<const float4*>(tables[g]);
    set.out[g] = reinterpret_cast<float4*>(outs[g]);
    set.width4[g] = widths[g] / 4;
    set.start4[g + 1] = set.start4[g] + widths[g] / 4;
  }
  return FMD_OK;
}
}  // namespace

extern "C" {

int fmd_embed_rows_f32(const int32_t* elem, int64_t n_atoms, int32_t count, const float* const* tables,
                       const int32_t* widths, float* const* outs, hipStream_t stream) {
  FMD_REQUIRE(elem && n_atoms >= 0);
  EmbedSet set;
  const int rc = embed_set(count, tables, widths, outs, set);
  if (rc != FMD_OK) return rc;
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)fmd_cdiv(n_atoms * set.start4[count], 256)), dim3(256), 0,
                     stream, elem, n_atoms, set);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_edge_geometry_embed_f32(const float* positions, const float* cell, const int32_t* system_of,
                                const int32_t* edge_index, const float* edge_image, const int64_t* n_edges,
                                int64_t e_cap, float rc, int32_t nb, float* geo, float* ef, float* def,
                                const int32_t* elem, int64_t n_atoms, int32_t count, const float* const* tables,
                                const int32_t* widths, float* const* outs, hipStream_t stream) {
  FMD_REQUIRE(positions && cell && edge_index && edge_image && n_edges && geo && ef && def);
  FMD_REQUIRE(e_cap >= 0 && nb > 0 && rc > 0.f && elem && n_atoms >= 0);
  EmbedSet set;
  const int st = embed_set(count, tables, widths, outs, set);
  if (st != FMD_OK) return st;
  const int64_t geo_blocks = fmd_cdiv(e_cap, 256), emb_blocks = fmd_cdiv(n_atoms * set.start4[count], 256);
  if (geo_blocks + emb_blocks == 0) return FMD_OK;
  FMD_REQUIRE(geo_blocks + emb_blocks < (int64_t(1) << 31));
  const GeoArgs a{positions, cell, system_of, edge_index, edge_image, n_edges, e_cap, rc, nb, geo, ef, def};
  hipLaunchKernelGGL(geometry_embed_kernel, dim3((unsigned)(geo_blocks + emb_blocks)), dim3(256), 0, stream, a,
                     geo_blocks, elem, n_atoms, set);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_morse_f32(const float* geo, const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap,
                  int64_t n_atoms, float D, float a, float r0, float rc, float vshift, float* energy, float* dvdr,
                  hipStream_t stream) {
  FMD_REQUIRE(geo && edge_offsets && n_edges && energy && dvdr && n_atoms >= 0);
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(morse_kernel, dim3((unsigned)fmd_cdiv(n_atoms, 256)), dim3(256), 0, stream, geo, edge_offsets,
                     n_edges, e_cap, n_atoms, D, a, r0, rc, vshift, energy, dvdr);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_morse_bwd_f32(const float* geo, const float* dvdr, const int32_t* edge_index, const float* gE,
                      const int64_t* n_edges, int64_t e_cap, float* gvec, hipStream_t stream) {
  FMD_REQUIRE(geo && dvdr && edge_index && gE && n_edges && gvec && e_cap >= 0);
  if (e_cap == 0) return FMD_OK;
  hipLaunchKernelGGL(morse_bwd_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, geo, dvdr,
                     edge_index, gE, n_edges, e_cap, gvec);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int64_t fmd_edge_virial_work_size(void) { return 9 * (int64_t)kVirialBlocks; }

int fmd_edge_stress_f32(const float* geo, const float* gvec, const int64_t* n_edges, int64_t e_cap, const float* cell,
                        double* work, float* stress, hipStream_t stream) {
  FMD_REQUIRE(geo && gvec && n_edges && cell && work && stress && e_cap >= 0);
  FMD_REQUIRE(aligned_to(16, {geo}));
  hipLaunchKernelGGL(edge_virial_kernel, dim3(kVirialBlocks), dim3(kThreads), 0, stream, geo, gvec, n_edges, e_cap,
                     work);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(virial_stress_kernel, dim3(1), dim3(FMD_WAVE), 0, stream, work, cell, stress);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
