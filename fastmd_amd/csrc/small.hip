// Node side of the MACE-like interaction for small systems (up to a few thousand atoms).
//
// There every node GEMM is a few hundred output tiles of K <= 1 024 and a 64 x 64 tile walks its K
// slices one memory round trip after another (10 us per launch at 135 atoms for ~1 us of matrix
// work). Here an output tile is 16 x 16, one workgroup of four waves, and each wave takes its own
// contiguous share of K with every operand load issued straight from global memory into the
// registers the MFMA reads (no LDS staging, no barrier per slice); the four partial tiles are
// added in wave order at the end (a fixed order: deterministic, but not the K order of the 64 x 64
// kernel, so the bits differ from fmd_gemm_group_f32's). Two kernels also fuse the symmetric
// contraction into the GEMM that feeds it: a workgroup computes the scalar row and the three
// vector rows of 16 atoms over 16 channels (one wave each, all of K), then the contraction (or its
// VJP) of those 16 x 16 (atom, channel) pairs from the four tiles in LDS, one launch instead of two.
//
// MFMA v_mfma_f32_16x16x4_f32 (one 16 x 16 block, fp32 operands, 4 k per instruction):
//   A operand: lane l holds A[l % 16][k(l / 16)];  B operand: lane l holds B[k(l / 16)][l % 16]
//   D: lane l, register v holds D[(l / 16) * 4 + v][l % 16]
// A 32-k slice is 8 instructions; at step s lane group g = l / 16 supplies k = 8 g + s (any
// bijection shared by A and B gives the same product), so over a slice a lane reads 8 consecutive
// k of its A row and of its B row: two float4 loads per operand.
#include "common.h"
#include "mace_math.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256, kWaves = kThreads / FMD_WAVE;
constexpr int kSlice = 32;
constexpr int kMaxGroup = 4;

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// 8 consecutive values p[0 .. 8), zero from index lim on (lim may be <= 0)
__device__ __forceinline__ void load8(const float* p, int lim, float (&v)[8]) {
  if (lim >= 8) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    const float4 y = *reinterpret_cast<const float4*>(p + 4);
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
    v[4] = y.x;
    v[5] = y.y;
    v[6] = y.z;
    v[7] = y.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = i < lim ? p[i] : 0.f;
  }
}

// One lane's rows of a K-split product: A row [a | a2] (k < ksplit from a, beyond from a2 at
// k - ksplit; ksplit a multiple of the slice; a2 = a when ksplit = k) and B row b (K-contiguous),
// K = k.
struct LaneRows {
  const float* a;
  const float* a2;
  const float* b;
  int64_t ksplit, k;
};

// slice s of the lane's rows: its 8 k (8 g .. 8 g + 8 of the slice) of A and of B
__device__ __forceinline__ void load_slice(const LaneRows& r, int64_t s, int g, float (&av)[8], float (&bv)[8]) {
  const int64_t k0 = s * kSlice + 8 * g;
  const bool first = s * kSlice < r.ksplit;
  const float* ap = first ? r.a + k0 : r.a2 + (k0 - r.ksplit);
  const int64_t end = first ? r.ksplit : r.k;
  load8(ap, (int)(end - k0 < 8 ? end - k0 : 8), av);
  load8(r.b + k0, (int)(r.k - k0 < 8 ? r.k - k0 : 8), bv);
}

// acc += the product over slices [s0, s1): slice s + 1's loads are in flight during slice s's
// eight MFMAs
__device__ __forceinline__ void ks_accumulate(const LaneRows& r, int64_t s0, int64_t s1, f32x4& acc) {
  const int g = (threadIdx.x & 63) >> 4;
  if (s0 >= s1) return;
  float av[8], bv[8];
  load_slice(r, s0, g, av, bv);
  for (int64_t s = s0; s < s1; ++s) {
    const bool more = s + 1 < s1;
    float an[8], bn[8];
    if (more) load_slice(r, s + 1, g, an, bn);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[i], acc, 0, 0, 0);
    if (more) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        av[i] = an[i];
        bv[i] = bn[i];
      }
    }
  }
}

// the 16 x 16 tile of a wave into LDS: blk[i][j] (pitch 17: conflict-free both ways)
__device__ __forceinline__ void tile_to_lds(const f32x4& acc, float (*blk)[17]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int v = 0; v < 4; ++v) blk[(lane >> 4) * 4 + v][lane & 15] = acc[v];
}

struct KsDesc {
  const float* a;
  const float* a2;
  const float* b;
  const float* bias;
  float* c;
  int64_t lda, lda2, ksplit, ldb, ldc, m, n, k, tiles_n, tile0;
  int accumulate;
};
struct KsGroup {
  KsDesc d[kMaxGroup];
  int count;
  int act;
};

// C (+)= [a | a2] b^T (+ bias), then the activation, for up to four problems: workgroup w takes
// problem g with tile0[g] <= w < tile0[g + 1], its 16 x 16 tile (w - tile0[g]) in row-major
// order; wave q multiplies the slices [S q / 4, S (q + 1) / 4) of the S = ceil(K / 32).
__global__ void __launch_bounds__(kThreads) gemm_ks_group_kernel(const KsGroup grp) {
  __shared__ float part[kWaves][16][17];
  const int64_t w = blockIdx.x;
  int g = 0;
#pragma unroll
  for (int q = 1; q < kMaxGroup; ++q)
    if (q < grp.count && w >= grp.d[q].tile0) g = q;
  const KsDesc& d = grp.d[g];
  const int64_t t = w - d.tile0, tm = t / d.tiles_n, tn = t - tm * d.tiles_n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = tm * 16, col0 = tn * 16;
  // rows past M and columns past N read the last row / column: computed, never stored
  const int64_t r = row0 + (lane & 15) < d.m ? row0 + (lane & 15) : d.m - 1;
  const int64_t cj = col0 + (lane & 15) < d.n ? col0 + (lane & 15) : d.n - 1;
  const float* ar = d.a + r * d.lda;
  const LaneRows rows{ar, d.a2 ? d.a2 + r * d.lda2 : ar, d.b + cj * d.ldb, d.ksplit, d.k};
  const int64_t S = fmd_cdiv(d.k, kSlice);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  ks_accumulate(rows, S * wave / kWaves, S * (wave + 1) / kWaves, acc);
  tile_to_lds(acc, part[wave]);
  __syncthreads();
  const int i = threadIdx.x >> 4, j = threadIdx.x & 15;
  const int64_t row = row0 + i, col = col0 + j;
  if (row >= d.m || col >= d.n) return;
  float x = part[0][i][j] + part[1][i][j] + part[2][i][j] + part[3][i][j];
  if (d.bias) x += d.bias[col];
  float* dst = d.c + row * d.ldc + col;
  if (d.accumulate) x = *dst + x;
  if (grp.act == 1) x = silu(x);
  *dst = x;
}

// P0 = A0 Wm0, P1 = A1 Wm1 and the contraction B0, B1 of the same 16 atoms x 16 channels: wave 0
// the scalar rows, wave 1 + x the vector rows x (A1 row 3 atom + x), all of K = C each; the
// contraction of (atom, channel) by thread 16 atom + channel of the tile. P0 and P1 are written
// too (the VJP reads them). Weights [C_out, C_in] (K-contiguous).
__global__ void __launch_bounds__(kThreads) mix_symcon_kernel(const float* A0, const float* A1, const float* wm0t,
                                                              const float* wm1t, const int32_t* elem, const float* Wc,
                                                              const float* Wd, int64_t n, int C, float* P0, float* P1,
                                                              float* B0, float* B1) {
  __shared__ float blk[kWaves][16][17];
  const int tiles_c = C / 16;
  const int64_t at = blockIdx.x / tiles_c;
  const int ct = (int)(blockIdx.x - at * tiles_c);
  const int64_t a0 = at * 16;
  const int c0 = ct * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ar = a0 + (lane & 15) < n ? a0 + (lane & 15) : n - 1;  // past n: computed, never stored
  const float* arow = wave == 0 ? A0 + ar * C : A1 + (ar * 3 + (wave - 1)) * C;
  const float* brow = (wave == 0 ? wm0t : wm1t) + (int64_t)(c0 + (lane & 15)) * C;
  const LaneRows rows{arow, arow, brow, C, C};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  ks_accumulate(rows, 0, C / kSlice, acc);
  tile_to_lds(acc, blk[wave]);
  __syncthreads();
  const int i = threadIdx.x >> 4, j = threadIdx.x & 15;
  const int64_t a = a0 + i;
  if (a >= n) return;
  const int ch = c0 + j;
  const int64_t k = a * C + ch;
  const float p0 = blk[0][i][j], px = blk[1][i][j], py = blk[2][i][j], pz = blk[3][i][j];
  P0[k] = p0;
  P1[(a * 3 + 0) * C + ch] = px;
  P1[(a * 3 + 1) * C + ch] = py;
  P1[(a * 3 + 2) * C + ch] = pz;
  const int el = elem[a];
  const float n1 = px * px + py * py + pz * pz;
  B0[k] = symcon_b0(p0, n1, Wc + (int64_t)el * 5 * C + ch, C);
  if (B1) {
    const float q = symcon_q(p0, n1, Wd + (int64_t)el * 4 * C + ch, C);
    B1[(a * 3 + 0) * C + ch] = q * px;
    B1[(a * 3 + 1) * C + ch] = q * py;
    B1[(a * 3 + 2) * C + ch] = q * pz;
  }
}

// The VJP's first half: gB0 = g0 wb0^T (g0 [N, k0]: k0 = C, or the readout width with the merged
// last layer's weight), gB1 = g1 wb1^T (g1 [N, 3, C], may be null: no vector output gradient),
// then the contraction's VJP -> gP0, gP1 of the same 16 atoms x 16 channels (gB0 and gB1 stay in
// LDS). Weights [C, K] (K-contiguous).
__global__ void __launch_bounds__(kThreads) mix_symcon_bwd_kernel(const float* g0, int64_t k0, const float* wb0,
                                                                  const float* g1, const float* wb1, const float* P0,
                                                                  const float* P1, const int32_t* elem,
                                                                  const float* Wc, const float* Wd, int64_t n, int C,
                                                                  float* gP0, float* gP1) {
  __shared__ float blk[kWaves][16][17];
  const int tiles_c = C / 16;
  const int64_t at = blockIdx.x / tiles_c;
  const int ct = (int)(blockIdx.x - at * tiles_c);
  const int64_t a0 = at * 16;
  const int c0 = ct * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ar = a0 + (lane & 15) < n ? a0 + (lane & 15) : n - 1;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (wave == 0) {
    const float* gr = g0 + ar * k0;
    const LaneRows rows{gr, gr, wb0 + (int64_t)(c0 + (lane & 15)) * k0, k0, k0};
    ks_accumulate(rows, 0, fmd_cdiv(k0, kSlice), acc);
  } else if (g1) {
    const float* gr = g1 + (ar * 3 + (wave - 1)) * C;
    const LaneRows rows{gr, gr, wb1 + (int64_t)(c0 + (lane & 15)) * C, C, C};
    ks_accumulate(rows, 0, C / kSlice, acc);
  }
  tile_to_lds(acc, blk[wave]);
  __syncthreads();
  const int i = threadIdx.x >> 4, j = threadIdx.x & 15;
  const int64_t a = a0 + i;
  if (a >= n) return;
  const int ch = c0 + j;
  const int64_t k = a * C + ch;
  const float p[3] = {P1[(a * 3 + 0) * C + ch], P1[(a * 3 + 1) * C + ch], P1[(a * 3 + 2) * C + ch]};
  const float gb1[3] = {blk[1][i][j], blk[2][i][j], blk[3][i][j]};
  const int el = elem[a];
  float gp0, gp[3];
  symcon_vjp(P0[k], p, Wc + (int64_t)el * 5 * C + ch, Wd + (int64_t)el * 4 * C + ch, C, blk[0][i][j], g1 != nullptr,
             gb1, gp0, gp);
  gP0[k] = gp0;
#pragma unroll
  for (int x = 0; x < 3; ++x) gP1[(a * 3 + x) * C + ch] = gp[x];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

int fmd_gemm_group_ks_f32(int32_t count, const float* const* a, const int64_t* lda, const float* const* a2,
                          const int64_t* lda2, const int64_t* ksplit, const float* const* b, const int64_t* ldb,
                          const float* const* bias, float* const* c, const int64_t* ldc, const int64_t* m,
                          const int64_t* n, const int64_t* k, const int32_t* accumulate, int32_t epilogue_kind,
                          hipStream_t stream) {
  FMD_REQUIRE(count >= 1 && count <= kMaxGroup && a && lda && b && ldb && c && ldc && m && n && k);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  KsGroup grp{};
  grp.act = epilogue_kind;
  int64_t tiles = 0;
  for (int g = 0; g < count; ++g) {
    FMD_REQUIRE(m[g] >= 0 && n[g] >= 0 && k[g] >= 0);
    if (m[g] == 0 || n[g] == 0) continue;  // (an empty output may have a null pointer)
    FMD_REQUIRE(c[g] && ldc[g] >= n[g]);
    const bool split = a2 && a2[g];
    const int64_t ks = split ? ksplit[g] : k[g];
    FMD_REQUIRE(k[g] == 0 || (a[g] && b[g] && ldb[g] >= k[g] && lda[g] >= ks));
    FMD_REQUIRE(!split || (lda2 && ks > 0 && ks < k[g] && lda2[g] >= k[g] - ks));
    // float4 operand loads: 16-byte aligned rows; a slice never straddles a and a2
    if (k[g] > 0 && (!aligned16(a[g]) || lda[g] % 4 || !aligned16(b[g]) || ldb[g] % 4)) return FMD_EUNSUPPORTED;
    if (split && (ks % kSlice || !aligned16(a2[g]) || lda2[g] % 4)) return FMD_EUNSUPPORTED;
    KsDesc& d = grp.d[grp.count++];
    d = KsDesc{a[g], split ? a2[g] : nullptr, b[g], bias ? bias[g] : nullptr, c[g], lda[g], split ? lda2[g] : 0, ks,
               ldb[g], ldc[g], m[g], n[g], k[g], fmd_cdiv(n[g], 16), tiles, accumulate ? accumulate[g] : 0};
    tiles += fmd_cdiv(m[g], 16) * d.tiles_n;
  }
  if (grp.count == 0) return FMD_OK;
  FMD_REQUIRE(tiles < (int64_t(1) << 31));
  hipLaunchKernelGGL(gemm_ks_group_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, stream, grp);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_mix_symcon_f32(const float* A0, const float* A1, const float* wm0t, const float* wm1t,
                            const int32_t* elem, const float* Wc, const float* Wd, int64_t n_atoms, int32_t channels,
                            float* P0, float* P1, float* B0, float* B1, hipStream_t stream) {
  FMD_REQUIRE(A0 && A1 && wm0t && wm1t && elem && Wc && P0 && P1 && B0 && (!B1 || Wd) && n_atoms >= 0);
  FMD_REQUIRE(channels > 0 && channels % kSlice == 0);
  FMD_REQUIRE(aligned16(A0) && aligned16(A1) && aligned16(wm0t) && aligned16(wm1t));
  if (n_atoms == 0) return FMD_OK;
  const int64_t blocks = fmd_cdiv(n_atoms, 16) * (channels / 16);
  FMD_REQUIRE(blocks < (int64_t(1) << 31));
  hipLaunchKernelGGL(mix_symcon_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, A0, A1, wm0t, wm1t, elem, Wc,
                     Wd, n_atoms, (int)channels, P0, P1, B0, B1);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_mix_symcon_bwd_f32(const float* g0, int64_t k0, const float* wb0, const float* g1, const float* wb1,
                                const float* P0, const float* P1, const int32_t* elem, const float* Wc,
                                const float* Wd, int64_t n_atoms, int32_t channels, float* gP0, float* gP1,
                                hipStream_t stream) {
  FMD_REQUIRE(g0 && wb0 && P0 && P1 && elem && Wc && gP0 && gP1 && (!g1 || (wb1 && Wd)) && n_atoms >= 0);
  FMD_REQUIRE(channels > 0 && channels % kSlice == 0 && k0 > 0);
  FMD_REQUIRE(aligned16(g0) && k0 % 4 == 0 && aligned16(wb0) && (!g1 || (aligned16(g1) && aligned16(wb1))));
  if (n_atoms == 0) return FMD_OK;
  const int64_t blocks = fmd_cdiv(n_atoms, 16) * (channels / 16);
  FMD_REQUIRE(blocks < (int64_t(1) << 31));
  hipLaunchKernelGGL(mix_symcon_bwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, g0, k0, wb0, g1, wb1,
                     P0, P1, elem, Wc, Wd, n_atoms, (int)channels, gP0, gP1);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
