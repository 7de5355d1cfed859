// (d) Wide edge GEMM on CDNA4 matrix cores.
//
// C[M,N] = A[M,K] * op(B) (+ bias) (+ C), fp32 output, MFMA accumulation in fp32:
//   fp32: v_mfma_f32_32x32x2_f32   (A/B operands fp32; 157 TFLOP/s dense peak on MI355X)
//   fp32 as three bf16 planes: each operand x = x0 + x1 + x2 (bf16, round to nearest: the three
//         planes hold x's 24 significand bits) and C = sum of the six products xi*yj with
//         i + j <= 2 on v_mfma_f32_32x32x16_bf16 (fp32 accumulation). The dropped products are
//         below 2^-24 relative, so the result is as accurate as an fp32 GEMM (measured: max error
//         vs fp64 7e-7 of max|C| at K = 264, against 9e-7 for the fp32 MFMA kernel), at
//         2.5 PFLOP/s / 6 = 417 TFLOP/s of fp32 work instead of 157 (CDNA4 has no TF32).
//   bf16: v_mfma_f32_32x32x16_bf16 (A/B operands bf16; 2.5 PFLOP/s dense peak)
// Workgroup: 256 threads = 4 waves in a 2x2 arrangement; block tile 128x128 (each wave a 64x64
// sub-tile: 2x2 MFMA 32x32 blocks, 64 accumulator registers per lane) or 64x64 for small
// problems. The K dimension is staged through LDS in BK-wide slices; the next slice's global
// loads are issued before the MFMAs of the current one. Any M, N, K (tails are zero-filled in
// LDS), so K = 2F+8 (136, 264, 520) needs no padding by the caller.
// MFMA operand layouts (32x32, one block):
//   A operand: lane l holds A[l%32][k0 + (l/32)*KPL .. +KPL)   (KPL = 1 fp32 / 8 bf16)
//   B operand: lane l holds B[k0 + (l/32)*KPL .. +KPL)[l%32]
//   D: lane l, register v holds D[(v/4)*8 + (l/32)*4 + v%4][l%32]
#include "common.h"

// thin.hip: the K <= 16 and N <= 16 shapes of fmd_gemm_f32; FMD_EUNSUPPORTED for the others
__attribute__((visibility("hidden"))) int launch_gemm_thin(const float* a, int64_t lda, const float* b, int64_t ldb, int32_t b_layout, const float* bias,
                     float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t act,
                     hipStream_t stream);

namespace {

constexpr int BM = 128, BN = 128, kThreads = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// A 16-byte load through the global address space. A pointer whose origin the compiler cannot see
// (behind an empty asm, a select with another object) is loaded as generic (flat) memory, and a
// flat load counts against the LDS counter too: every wait for an LDS read would then also wait
// for it.
__device__ __forceinline__ bf16x8 load_global(const __bf16* p) {
  return *(const __attribute__((address_space(1))) bf16x8*)(p);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

template <int WM, int WN>
__device__ __forceinline__ void epilogue(const f32x16 (&acc)[WM][WN], int64_t row0, int64_t col0, int64_t m,
                                         int64_t n, const float* bias, float* c, int64_t ldc, int accumulate, int act) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int bi = 0; bi < WM; ++bi)
#pragma unroll
    for (int bj = 0; bj < WN; ++bj) {
      const int64_t col = col0 + bj * 32 + (lane & 31);
      if (col >= n) continue;
      const float b = bias ? bias[col] : 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = row0 + bi * 32 + (v / 4) * 8 + (lane / 32) * 4 + (v % 4);
        if (row >= m) continue;
        float x = acc[bi][bj][v] + b;
        float* dst = c + row * ldc + col;
        if (accumulate) x = *dst + x;
        if (act == 1) x = silu(x);
        *dst = x;
      }
    }
}

// ---------------------------------------------------------------------------------------- fp32
// Block tile BM x BN (64 or 128 each), K staged in BK = 32 slices through a double-buffered LDS
// (one barrier per slice: the next slice is stored into the other buffer while this one feeds
// the MFMAs). 4 waves in 2 x 2; wave tile (BM/2) x (BN/2) = WM x WN MFMA blocks of 32 x 32.
// LDS holds both operands k-major (As[k][i], Bs[k][j]) so a lane's MFMA operand is one
// ds_read_b32 at a conflict-free address (consecutive lanes, consecutive i / j).
constexpr int BK32 = 32;

// One BM x BN tile at (row_blk, col_blk). A may be split along K: columns [0, ksplit) from a,
// [ksplit, k) from a2 (ksplit a multiple of BK32), i.e. [a | a2] @ op(b) in one accumulation.
template <int BM, int BN, int BLAYOUT>
__device__ __forceinline__ void gemm_f32_tile(const float* __restrict__ a, int64_t lda, const float* __restrict__ a2,
                                              int64_t lda2, int64_t ksplit, const float* __restrict__ b, int64_t ldb,
                                              const float* __restrict__ bias, float* c, int64_t ldc, int64_t m,
                                              int64_t n, int64_t k, int accumulate, int act, int64_t row_blk,
                                              int64_t col_blk) {
  constexpr int WM = BM / 64, WN = BN / 64;           // MFMA blocks per wave
  constexpr int LDA = BM + 4, LDB = BN + 4;           // padded LDS rows
  constexpr int A_VEC = BM * BK32 / 4 / kThreads;     // float4 loads per thread (A)
  constexpr int B_VEC = BN * BK32 / 4 / kThreads;     // float4 loads per thread (B)
  __shared__ float As[2][BK32][LDA];
  __shared__ float Bs[2][BK32][LDB];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  float4 ra[A_VEC], rb[B_VEC];
  auto load4 = [&](const float* p, bool in_rows, int64_t kk, int64_t kmax) -> float4 {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!in_rows) return v;
    if (kk + 3 < kmax && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) return *reinterpret_cast<const float4*>(p);
    v.x = kk < kmax ? p[0] : 0.f;
    v.y = kk + 1 < kmax ? p[1] : 0.f;
    v.z = kk + 2 < kmax ? p[2] : 0.f;
    v.w = kk + 3 < kmax ? p[3] : 0.f;
    return v;
  };
  // A tile: BM rows x 32 k; id -> (row id / 8, k (id % 8) * 4)
  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < A_VEC; ++q) {
      const int id = t + q * kThreads;
      const int r = id >> 3, kc = (id & 7) * 4;
      const int64_t gr = row_blk + r, gk = k0 + kc;
      const float* src = k0 < ksplit ? a + gr * lda + gk : a2 + gr * lda2 + (gk - ksplit);
      ra[q] = load4(src, gr < m, gk, k);
    }
  };
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < B_VEC; ++q) {
      const int id = t + q * kThreads;
      if (BLAYOUT == 0) {  // B [N, K]: row j, 4 consecutive k
        const int r = id >> 3, kc = (id & 7) * 4;
        const int64_t gj = col_blk + r, gk = k0 + kc;
        rb[q] = load4(b + gj * ldb + gk, gj < n, gk, k);
      } else {  // B [K, N]: row k, 4 consecutive j
        constexpr int JV = BN / 4;
        const int kr = id / JV, jc = (id % JV) * 4;
        const int64_t gk = k0 + kr, gj = col_blk + jc;
        rb[q] = load4(b + gk * ldb + gj, gk < k, gj, n);
      }
    }
  };
  auto store_tiles = [&](int st) {
#pragma unroll
    for (int q = 0; q < A_VEC; ++q) {
      const int id = t + q * kThreads;
      const int r = id >> 3, kc = (id & 7) * 4;
      As[st][kc + 0][r] = ra[q].x;
      As[st][kc + 1][r] = ra[q].y;
      As[st][kc + 2][r] = ra[q].z;
      As[st][kc + 3][r] = ra[q].w;
    }
#pragma unroll
    for (int q = 0; q < B_VEC; ++q) {
      const int id = t + q * kThreads;
      if (BLAYOUT == 0) {
        const int r = id >> 3, kc = (id & 7) * 4;
        Bs[st][kc + 0][r] = rb[q].x;
        Bs[st][kc + 1][r] = rb[q].y;
        Bs[st][kc + 2][r] = rb[q].z;
        Bs[st][kc + 3][r] = rb[q].w;
      } else {
        constexpr int JV = BN / 4;
        const int kr = id / JV, jc = (id % JV) * 4;
        *reinterpret_cast<float4*>(&Bs[st][kr][jc]) = rb[q];
      }
    }
  };

  f32x16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, BK32);
  load_a(0);
  load_b(0);
  store_tiles(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int st = (int)(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      load_a((kt + 1) * BK32);
      load_b((kt + 1) * BK32);
    }
#pragma unroll
    for (int kk = 0; kk < BK32; kk += 2) {
      const int kr = kk + (lane >> 5);
      float av[WM], bv[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) av[i] = As[st][kr][wm * (BM / 2) + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < WN; ++j) bv[j] = Bs[st][kr][wn * (BN / 2) + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles(st ^ 1);
    __syncthreads();
  }
  epilogue<WM, WN>(acc, row_blk + wm * (BM / 2), col_blk + wn * (BN / 2), m, n, bias, c, ldc, accumulate, act);
}

template <int BM, int BN, int BLAYOUT>
__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(const float* __restrict__ a, int64_t lda,
                                                            const float* __restrict__ b, int64_t ldb,
                                                            const float* __restrict__ bias, float* c, int64_t ldc,
                                                            int64_t m, int64_t n, int64_t k, int accumulate, int act) {
  gemm_f32_tile<BM, BN, BLAYOUT>(a, lda, a, lda, k, b, ldb, bias, c, ldc, m, n, k, accumulate, act,
                                 (int64_t)blockIdx.x * BM, (int64_t)blockIdx.y * BN);
}

// Several independent GEMMs of one b layout in one launch (the node side of an interaction
// layer: fewer, fuller launches). Workgroup w takes problem g with tile0[g] <= w < tile0[g + 1],
// tile (w - tile0[g]) in row-major order of its 64 x 64 tiles. Each problem's result is the one
// fmd_gemm_f32's 64 x 64 kernel gives (same K order), with [a | a2] when a2 is set.
constexpr int kMaxGroup = 4;
struct GemmDesc {
  const float* a;
  const float* a2;
  const float* b;
  const float* bias;
  float* c;
  int64_t lda, lda2, ksplit, ldb, ldc, m, n, k, tiles_n, tile0;
  int accumulate;
};
struct GemmGroup {
  GemmDesc d[kMaxGroup];
  int count;
  int act;
};

// Deterministic split-K for tall-K node GEMMs (few output tiles, long K): workgroup (tile, s)
// multiplies K slice s ([s ks, (s + 1) ks), inside one of the parts a | a2) into the workspace
// partial ws[s] ([M, N]); splitk_sum_kernel adds the partials in the order s = 0, 1, ...
template <int BLAYOUT>
__global__ void __launch_bounds__(kThreads) gemm_f32_splitk_kernel(const float* __restrict__ a, int64_t lda,
                                                                   const float* __restrict__ a2, int64_t lda2,
                                                                   int64_t ksplit, const float* __restrict__ b,
                                                                   int64_t ldb, float* ws, int64_t m, int64_t n,
                                                                   int64_t ks, int64_t tiles_n, int64_t tiles) {
  const int64_t w = blockIdx.x, s = w / tiles, t = w - s * tiles;
  const int64_t tm = t / tiles_n, tn = t - tm * tiles_n;
  const int64_t k0 = s * ks;
  const bool second = k0 >= ksplit;
  const float* ap = second ? a2 + (k0 - ksplit) : a + k0;
  const int64_t la = second ? lda2 : lda;
  const float* bp = BLAYOUT == 0 ? b + k0 : b + k0 * ldb;
  gemm_f32_tile<64, 64, BLAYOUT>(ap, la, ap, la, ks, bp, ldb, nullptr, ws + s * m * n, n, m, n, ks, 0, 0, tm * 64,
                                 tn * 64);
}

__global__ void splitk_sum_kernel(const float* __restrict__ ws, int splits, int64_t m, int64_t n,
                                  const float* __restrict__ bias, float* c, int64_t ldc, int accumulate) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= m * n) return;
  const int64_t r = id / n, col = id - r * n;
  float x = ws[id];
  for (int sp = 1; sp < splits; ++sp) x += ws[sp * m * n + id];
  if (bias) x += bias[col];
  float* d = c + r * ldc + col;
  *d = accumulate ? *d + x : x;
}

// The same sums for S slices, four columns per thread (N, ldc multiples of 4, 16-byte aligned
// workspace and C, M N < 2^32): the S loads all in flight before the adds, which run in slice
// order as above (the same bits).
template <int S>
__global__ void __launch_bounds__(256) splitk_sum4_kernel(const float* __restrict__ ws, uint32_t m, uint32_t n,
                                                          const float* __restrict__ bias, float* c, int64_t ldc,
                                                          int accumulate) {
  const uint32_t id = 4u * (blockIdx.x * 256u + threadIdx.x);
  const uint32_t mn = m * n;
  if (id >= mn) return;
  const uint32_t r = id / n, col = id - r * n;
  float4 v[S];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) v[sp] = *reinterpret_cast<const float4*>(ws + (size_t)sp * mn + id);
  float4 x = v[0];
#pragma unroll
  for (int sp = 1; sp < S; ++sp) {
    x.x += v[sp].x;
    x.y += v[sp].y;
    x.z += v[sp].z;
    x.w += v[sp].w;
  }
  if (bias) {
    const float4 b = *reinterpret_cast<const float4*>(bias + col);
    x.x += b.x;
    x.y += b.y;
    x.z += b.z;
    x.w += b.w;
  }
  float4* d = reinterpret_cast<float4*>(c + (int64_t)r * ldc + col);
  if (accumulate) {
    const float4 o = *d;
    x.x = o.x + x.x;
    x.y = o.y + x.y;
    x.z = o.z + x.z;
    x.w = o.w + x.w;
  }
  *d = x;
}

void launch_splitk_sum(const float* ws, int splits, int64_t m, int64_t n, const float* bias, float* c, int64_t ldc,
                       int accumulate, hipStream_t stream) {
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = n % 4 == 0 && ldc % 4 == 0 && m * n < (int64_t(1) << 32) && aligned(ws) && aligned(c) &&
                   (!bias || aligned(bias)) && (splits == 2 || splits == 4 || splits == 8);
  if (!vec) {
    hipLaunchKernelGGL(splitk_sum_kernel, dim3((unsigned)fmd_cdiv(m * n, 256)), dim3(256), 0, stream, ws, splits, m,
                       n, bias, c, ldc, accumulate);
    return;
  }
  const dim3 grid((unsigned)fmd_cdiv(m * n, 4 * 256));
  const uint32_t mu = (uint32_t)m, nu = (uint32_t)n;
  if (splits == 2)
    hipLaunchKernelGGL(splitk_sum4_kernel<2>, grid, dim3(256), 0, stream, ws, mu, nu, bias, c, ldc, accumulate);
  else if (splits == 4)
    hipLaunchKernelGGL(splitk_sum4_kernel<4>, grid, dim3(256), 0, stream, ws, mu, nu, bias, c, ldc, accumulate);
  else
    hipLaunchKernelGGL(splitk_sum4_kernel<8>, grid, dim3(256), 0, stream, ws, mu, nu, bias, c, ldc, accumulate);
}

template <int BLAYOUT>
__global__ void __launch_bounds__(kThreads) gemm_f32_group_kernel(const GemmGroup grp) {
  const int64_t w = blockIdx.x;
  int g = 0;
#pragma unroll
  for (int q = 1; q < kMaxGroup; ++q)
    if (q < grp.count && w >= grp.d[q].tile0) g = q;
  const GemmDesc& d = grp.d[g];
  const int64_t t = w - d.tile0;
  const int64_t tm = t / d.tiles_n, tn = t - tm * d.tiles_n;
  gemm_f32_tile<64, 64, BLAYOUT>(d.a, d.lda, d.a2 ? d.a2 : d.a, d.a2 ? d.lda2 : d.lda, d.a2 ? d.ksplit : d.k, d.b,
                                 d.ldb, d.bias, d.c, d.ldc, d.m, d.n, d.k, d.accumulate, grp.act, tm * 64, tn * 64);
}

// ------------------------------------------------------------------------- fp32, both K-major
// The edge GEMMs of the MD step (z = a W1 with W1 stored transposed, and its VJP gz W1^T) have
// both operands K-contiguous ("NT": A [M,K], B [N,K]). This kernel is built for that case (each
// choice below was timed against the alternatives at the 10 000-atom shapes):
//  * LDS rows hold one operand row each in natural k order (pitch 36 floats: 16-byte aligned
//    float4 stores, conflict-free b128 reads). The 32 k of a slice are fed to the 16 MFMAs as
//    k = 16 h + 4 q + p at step (q, p) (h = lane / 32), so the values a lane needs are contiguous:
//    4 ds_read_b128 per operand block instead of 16 ds_read_b32 (the MFMA sums its two k slots,
//    so any bijection (q, p, h) -> k shared by A and B gives the same product).
//  * one LDS buffer (36 KB) and one register stage: the next slice's float4 loads are in flight
//    during the current slice's 64 MFMAs per wave, and three workgroups fit on a CU (12 waves).
//    Interior slices use unconditional loads (rows past M/N are clamped to the last row: computed,
//    never stored); a partial last slice is masked on a workgroup-uniform branch, and only its
//    first ceil(kv / 4) step groups are issued (K = 2F + 8 leaves kv = 8: 2 of 4).
//  * tiles are assigned XCD-aware: workgroups are dispatched round-robin over the 8 XCDs, and
//    the linear id is remapped so that each XCD walks a contiguous run of tiles (N fastest), so
//    the N tiles sharing one A tile run on the same XCD and read it from its L2.
//  * interior wave tiles without bias/accumulate/activation store straight from the
//    accumulators with incremental row pointers; the general epilogue handles the rest.
constexpr int NT_PITCH = 36;
__device__ __forceinline__ int64_t xcd_tile(int64_t w, int64_t g) { return fmd_xcd_block(w, g); }

constexpr int NT_V = 128 * BK32 / 4 / kThreads;  // float4 per thread per operand and slice (4)

__global__ void __launch_bounds__(kThreads) gemm_f32_nt_kernel(const float* __restrict__ a, int64_t lda,
                                                               const float* __restrict__ b, int64_t ldb,
                                                               const float* __restrict__ bias, float* c, int64_t ldc,
                                                               int64_t m, int64_t n, int64_t k, int accumulate,
                                                               int act, int vec_ok, int64_t n_tiles) {
  constexpr int TM = 128, TN = 128;
  __shared__ float As[TM][NT_PITCH];
  __shared__ float Bs[TN][NT_PITCH];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t row_blk = (tile / n_tiles) * TM, col_blk = (tile % n_tiles) * TN;

  // thread -> (row, 4 consecutive k) of a 128 x 32 slice: 8 lanes cover one row's 128 bytes
  const int kc = (t & 7) * 4;
  int64_t arow[NT_V], brow[NT_V];
#pragma unroll
  for (int q = 0; q < NT_V; ++q) {
    const int r = (t + q * kThreads) >> 3;
    arow[q] = min(row_blk + r, m - 1) * lda + kc;
    brow[q] = min(col_blk + r, n - 1) * ldb + kc;
  }
  float4 ra[NT_V], rb[NT_V];
  auto load = [&](int64_t k0) {
    if (vec_ok && k0 + BK32 <= k) {
#pragma unroll
      for (int q = 0; q < NT_V; ++q) {
        ra[q] = *reinterpret_cast<const float4*>(a + arow[q] + k0);
        rb[q] = *reinterpret_cast<const float4*>(b + brow[q] + k0);
      }
    } else {
      const int64_t g = k0 + kc;
#pragma unroll
      for (int q = 0; q < NT_V; ++q) {
        const float* pa = a + arow[q] + k0;
        const float* pb = b + brow[q] + k0;
        ra[q] = make_float4(g < k ? pa[0] : 0.f, g + 1 < k ? pa[1] : 0.f, g + 2 < k ? pa[2] : 0.f,
                            g + 3 < k ? pa[3] : 0.f);
        rb[q] = make_float4(g < k ? pb[0] : 0.f, g + 1 < k ? pb[1] : 0.f, g + 2 < k ? pb[2] : 0.f,
                            g + 3 < k ? pb[3] : 0.f);
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int q = 0; q < NT_V; ++q) {
      const int r = (t + q * kThreads) >> 3;
      *reinterpret_cast<float4*>(&As[r][kc]) = ra[q];
      *reinterpret_cast<float4*>(&Bs[r][kc]) = rb[q];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto compute = [&](int nq) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q >= nq) break;
      float4 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        av[i] = *reinterpret_cast<const float4*>(&As[wm * 64 + i * 32 + (lane & 31)][h * 16 + q * 4]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = *reinterpret_cast<const float4*>(&Bs[wn * 64 + j * 32 + (lane & 31)][h * 16 + q * 4]);
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][p], bv[j][p], acc[i][j], 0, 0, 0);
    }
  };

  const int64_t nk = fmd_cdiv(k, BK32);
  const int kv_last = (int)(k - (nk - 1) * BK32);  // real k in the last slice (1..32)
  // the last slice's real k sit at slots 0..kv-1, all with h = 0 when kv <= 16
  const int nq_last = kv_last <= 16 ? (kv_last + 3) / 4 : 4;
  load(0);
  for (int64_t kt = 0; kt < nk; ++kt) {
    if (kt) __syncthreads();  // every wave is done reading the previous slice
    store();
    __syncthreads();
    if (kt + 1 < nk) load((kt + 1) * BK32);
    compute(kt + 1 < nk ? 4 : nq_last);
  }
  const int64_t row0 = row_blk + wm * 64, col0 = col_blk + wn * 64;
  if (!bias && !accumulate && act == 0 && row0 + 64 <= m && col0 + 64 <= n) {
    float* base = c + (row0 + h * 4) * ldc + col0 + (lane & 31);
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float* rp = base + (int64_t)(bi * 32 + (v / 4) * 8 + (v % 4)) * ldc;
        rp[0] = acc[bi][0][v];
        rp[32] = acc[bi][1][v];
      }
    return;
  }
  epilogue<2, 2>(acc, row0, col0, m, n, bias, c, ldc, accumulate, act);
}

// ---------------------------------------------------------------------------------------- bf16
constexpr int BK16 = 32;
constexpr int LDK16 = BK16 + 8;  // bf16 elements per LDS row (+pad, keeps 16-byte alignment)

template <int BLAYOUT>
__global__ void __launch_bounds__(kThreads) gemm_bf16_kernel(const uint16_t* __restrict__ a, int64_t lda,
                                                             const uint16_t* __restrict__ b, int64_t ldb,
                                                             const float* __restrict__ bias, float* c, int64_t ldc,
                                                             int64_t m, int64_t n, int64_t k, int accumulate,
                                                             int act) {
  // As[i][k], Bs[j][k]: k contiguous so a lane reads its 8 k values as one 16-byte load
  __shared__ uint16_t As[BM][LDK16];
  __shared__ uint16_t Bs[BN][LDK16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t row_blk = (int64_t)blockIdx.x * BM, col_blk = (int64_t)blockIdx.y * BN;

  // A: 128 rows x 32 k = 512 chunks of 8 bf16; 2 per thread
  uint4 ra[2], rb[2];
  auto load_rowmajor = [&](const uint16_t* base, int64_t ld, int64_t rows_total, int64_t r0, int64_t k0, uint4* out) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int id = t + q * kThreads;
      const int r = id >> 2, kc = (id & 3) * 8;
      const int64_t gr = r0 + r, gk = k0 + kc;
      uint16_t e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (gr < rows_total) {
        const uint16_t* p = base + gr * ld + gk;
        if (gk + 7 < k && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
          out[q] = *reinterpret_cast<const uint4*>(p);
          continue;
        }
#pragma unroll
        for (int x = 0; x < 8; ++x) e[x] = (gk + x < k) ? p[x] : (uint16_t)0;
      }
      out[q] = make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16), e[4] | ((uint32_t)e[5] << 16),
                          e[6] | ((uint32_t)e[7] << 16));
    }
  };
  // B [K, N] (layout 1): 32 k rows x 128 j; each thread gathers 8 k of one j column
  auto load_b_kn = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int id = t + q * kThreads;
      const int j = id >> 2, kc = (id & 3) * 8;
      const int64_t gj = col_blk + j;
      uint16_t e[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int64_t gk = k0 + kc + x;
        e[x] = (gj < n && gk < k) ? b[gk * ldb + gj] : (uint16_t)0;
      }
      rb[q] = make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16), e[4] | ((uint32_t)e[5] << 16),
                         e[6] | ((uint32_t)e[7] << 16));
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int id = t + q * kThreads;
      const int r = id >> 2, kc = (id & 3) * 8;
      *reinterpret_cast<uint4*>(&As[r][kc]) = ra[q];
      *reinterpret_cast<uint4*>(&Bs[r][kc]) = rb[q];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, BK16);
  auto issue = [&](int64_t k0) {
    load_rowmajor(a, lda, m, row_blk, k0, ra);
    if (BLAYOUT == 0)
      load_rowmajor(b, ldb, n, col_blk, k0, rb);
    else
      load_b_kn(k0);
  };
  issue(0);
  for (int64_t kt = 0; kt < nk; ++kt) {
    __syncthreads();
    store_tiles();
    __syncthreads();
    if (kt + 1 < nk) issue((kt + 1) * BK16);
#pragma unroll
    for (int kk = 0; kk < BK16; kk += 16) {
      const int kc = kk + (lane >> 5) * 8;
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint4 raw = *reinterpret_cast<const uint4*>(&As[wm * 64 + i * 32 + (lane & 31)][kc]);
        av[i] = __builtin_bit_cast(bf16x8, raw);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint4 raw = *reinterpret_cast<const uint4*>(&Bs[wn * 64 + j * 32 + (lane & 31)][kc]);
        bv[j] = __builtin_bit_cast(bf16x8, raw);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }
  epilogue<2, 2>(acc, row_blk + wm * 64, col_blk + wn * 64, m, n, bias, c, ldc, accumulate, act);
}

// ------------------------------------------------------------- fp32 as three bf16 planes, NT
// C[M,N] = A[M,K] B[N,K]^T (+ bias) (+ C), both operands K-contiguous fp32. A is the column
// concatenation of up to three parts, part p reading row idx_p[r * istride_p] of src_p (or row
// r): the gather-cat of edge rows fused into the GEMM's operand load, so the [M, K] row matrix
// never exists in HBM. Block tile 128 x 128, 4 waves of 64 x 64 (2 x 2 blocks of 32 x 32),
// K in slices of 16: every thread loads two float4 of A and two of B (a row's 16 k take four
// threads), splits them into the three bf16 planes and stores 8-byte pieces into LDS; the 8-k
// chunk pair of LDS row r is swapped when bit 3 of r is set, so the sixteen 16-byte operand reads
// of a quarter wave hit distinct bank groups. Two LDS buffers (48 KB: three workgroups per CU,
// the register budget held to three waves per SIMD): slice kt + 1 is split and stored, and slice kt + 2 loaded into registers, while
// the MFMAs of slice kt run. Part widths are multiples of 4 and all but the last multiples of 16
// (a slice never straddles two parts); k past a part's width or past K loads as zero. An optional
// gathered row is added to each output row before the epilogue (C[r] += Q[idx[r]]: the receiver
// block of an edge GEMM formed once per atom).
struct X3Part {
  const float* src;
  const int32_t* idx;
  int64_t ld, istride;
  int32_t width;
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split3(float4 v, bf16x4& p0, bf16x4& p1, bf16x4& p2) {
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

constexpr int X3_PL = 128 * 16, X3_OP = 3 * X3_PL, X3_BUF = 2 * X3_OP;

#define X3_LOAD(K0, S)                                                                              \
  do {                                                                                              \
    const int64_t k0_ = (K0);                                                                       \
    const bool q2_ = k0_ >= ks2, q1_ = !q2_ && k0_ >= ks1;                                          \
    const float* base_ = q2_ ? src2 : q1_ ? src1 : src0;                                            \
    const int64_t kin_ = q2_ ? k0_ - ks2 : q1_ ? k0_ - ks1 : k0_;                                   \
    const int w_ = q2_ ? w2 : q1_ ? w1 : w0;                                                        \
    _Pragma("unroll") for (int q = 0; q < AQ; ++q) {                                                \
      const int64_t o_ = q2_ ? ao2[q] : q1_ ? ao1[q] : ao0[q];                                      \
      ra##S[q] = (kin_ + kc < w_) ? *reinterpret_cast<const float4*>(base_ + o_ + kin_)                \
                               : make_float4(0.f, 0.f, 0.f, 0.f);                                   \
    }                                                                                               \
    _Pragma("unroll") for (int q = 0; q < BQ; ++q)                                                   \
      rb##S[q] = (k0_ + kc < k) ? *reinterpret_cast<const float4*>(b + bo[q] + k0_)                    \
                             : make_float4(0.f, 0.f, 0.f, 0.f);                                     \
  } while (0)

#define X3_STORE(BUFI, S)                                                                           \
  do {                                                                                              \
    __bf16* sb_ = lds + (BUFI) * X3_BUF;                                                            \
    _Pragma("unroll") for (int q = 0; q < AQ; ++q) {                                                \
      bf16x4 x0_, x1_, x2_;                                                                         \
      split3(ra##S[q], x0_, x1_, x2_);                                                                 \
      *reinterpret_cast<bf16x4*>(sb_ + 0 * X3_PL + soff[q]) = x0_;                                  \
      *reinterpret_cast<bf16x4*>(sb_ + 1 * X3_PL + soff[q]) = x1_;                                  \
      *reinterpret_cast<bf16x4*>(sb_ + 2 * X3_PL + soff[q]) = x2_;                                  \
    }                                                                                               \
    _Pragma("unroll") for (int q = 0; q < BQ; ++q) {                                                 \
      bf16x4 x0_, x1_, x2_;                                                                         \
      split3(rb##S[q], x0_, x1_, x2_);                                                                 \
      *reinterpret_cast<bf16x4*>(sb_ + X3_OP + 0 * X3_PL + soff[q]) = x0_;                          \
      *reinterpret_cast<bf16x4*>(sb_ + X3_OP + 1 * X3_PL + soff[q]) = x1_;                          \
      *reinterpret_cast<bf16x4*>(sb_ + X3_OP + 2 * X3_PL + soff[q]) = x2_;                          \
    }                                                                                               \
  } while (0)

// six products per block, the small ones first: (0,2) (1,1) (2,0) (0,1) (1,0) (0,0)
#define X3_COMPUTE(BUFI, MBV)                                                                       \
  do {                                                                                              \
    const __bf16* as_ = lds + (BUFI) * X3_BUF;                                                      \
    const __bf16* bs_ = as_ + X3_OP;                                                                \
    bf16x8 av_[3][2], bv_[3][2];                                                                    \
    _Pragma("unroll") for (int p = 0; p < 3; ++p) {                                                 \
      _Pragma("unroll") for (int i = 0; i < (MBV); ++i)                                             \
        av_[p][i] = *reinterpret_cast<const bf16x8*>(as_ + p * X3_PL + (wm * 32 * (MBV) + i * 32) * 16 + rd); \
      _Pragma("unroll") for (int j = 0; j < 2; ++j)                                                 \
        bv_[p][j] = *reinterpret_cast<const bf16x8*>(bs_ + p * X3_PL + (wn * 64 + j * 32) * 16 + rd); \
    }                                                                                               \
    /* product-major: consecutive MFMAs go to the four accumulators in turn (four independent   \
       chains in flight); each accumulator still takes its six products in the same order */     \
    _Pragma("unroll") for (int pr = 0; pr < 6; ++pr) {                                              \
      const int pa_ = pr == 0 ? 0 : pr == 1 ? 1 : pr == 2 ? 2 : pr == 3 ? 0 : pr == 4 ? 1 : 0;      \
      const int pb_ = pr == 0 ? 2 : pr == 1 ? 1 : pr == 2 ? 0 : pr == 3 ? 1 : pr == 4 ? 0 : 0;      \
      _Pragma("unroll") for (int i = 0; i < (MBV); ++i) _Pragma("unroll") for (int j = 0; j < 2; ++j) \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av_[pa_][i], bv_[pb_][j], acc[i][j], 0, 0, 0); \
    }                                                                                               \
  } while (0)

// The end of a split-plane tile: C (+)= acc (+ radd[radd.idx[r]]) (+ bias), then the activation;
// interior wave tiles without bias / accumulate / activation store straight from the accumulators.
template <int MB>
__device__ __forceinline__ void x3_finish(f32x16 (&acc)[MB][2], const X3Part& radd, const float* __restrict__ bias,
                                          float* c, int64_t ldc, int64_t m, int64_t n, int accumulate, int act,
                                          int64_t row0, int64_t col0, int h, int rr) {
  if (radd.src) {
    // C[r, :] += radd[radd.idx[r], :] (a gathered row added to the product)
#pragma unroll
    for (int bi = 0; bi < MB; ++bi)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = min(row0 + bi * 32 + (v / 4) * 8 + h * 4 + (v % 4), m - 1);
        const float* qr = radd.src + (radd.idx ? (int64_t)radd.idx[row * radd.istride] : row) * radd.ld;
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
          const int64_t col = min(col0 + bj * 32 + rr, n - 1);
          acc[bi][bj][v] += qr[col];
        }
      }
  }
  if (!bias && act == 0 && row0 + 32 * MB <= m && col0 + 64 <= n) {
    float* base = c + (row0 + h * 4) * ldc + col0 + rr;
    if (accumulate) {
      // every old value loaded before any store: one memory round trip, not one per row (the
      // stores could alias the loads, so the compiler keeps a load-add-store chain in order)
#pragma unroll
      for (int bi = 0; bi < MB; ++bi) {
        float old[16][2];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float* rp = base + (int64_t)(bi * 32 + (v / 4) * 8 + (v % 4)) * ldc;
          old[v][0] = rp[0];
          old[v][1] = rp[32];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float* rp = base + (int64_t)(bi * 32 + (v / 4) * 8 + (v % 4)) * ldc;
          rp[0] = old[v][0] + acc[bi][0][v];
          rp[32] = old[v][1] + acc[bi][1][v];
        }
      }
      return;
    }
#pragma unroll
    for (int bi = 0; bi < MB; ++bi)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float* rp = base + (int64_t)(bi * 32 + (v / 4) * 8 + (v % 4)) * ldc;
        store_stream(rp, acc[bi][0][v]);
        store_stream(rp + 32, acc[bi][1][v]);
      }
    return;
  }
  epilogue<MB, 2>(acc, row0, col0, m, n, bias, c, ldc, accumulate, act);
}

// One 128 x BN tile of C at (row_blk, col_blk): A as up to three gathered column parts (K order
// P0 | P1 | P2), B [N, K] K-contiguous, both split into their planes as they are staged. BN = 128:
// waves 2 x 2, each 64 x 64 (MB = 2 blocks of 32 rows); BN = 64 (N <= 64, where a 128-wide tile
// would leave half its MFMAs idle): waves 4 x 1, each 32 x 64 (MB = 1). AQ / BQ: the loader's
// passes over A's 128 and B's BN rows. Every product keeps its K order: the same C either way.
template <int BN>
__device__ __forceinline__ void x3_tile(const X3Part& P0, const X3Part& P1, const X3Part& P2, int np,
                                        const float* __restrict__ b, int64_t ldb, const X3Part& radd,
                                        const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n,
                                        int64_t k, int accumulate, int act, int64_t row_blk, int64_t col_blk) {
  constexpr int MB = BN / 64, AQ = 2, BQ = BN / 64;
  __shared__ __attribute__((aligned(16))) __bf16 lds[2 * X3_BUF];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = BN == 128 ? wave >> 1 : wave, wn = BN == 128 ? wave & 1 : 0, h = lane >> 5, rr = lane & 31;
  const int64_t ks1 = P0.width, ks2 = ks1 + (np > 1 ? P1.width : 0);
  const float *src0 = P0.src, *src1 = P1.src, *src2 = P2.src;
  const int w0 = P0.width, w1 = P1.width, w2 = P2.width;
  // loader: thread t, pass q -> row (t + 256 q) / 4 of the tile, k (t % 4) * 4 of the slice
  const int kc = (t & 3) * 4;
  int64_t ao0[2], ao1[2], ao2[2], bo[2];
  int soff[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = (t + q * kThreads) >> 2;
    const int64_t gr = min(row_blk + r, m - 1);
    ao0[q] = (P0.idx ? (int64_t)P0.idx[gr * P0.istride] : gr) * P0.ld + kc;
    ao1[q] = np > 1 ? (P1.idx ? (int64_t)P1.idx[gr * P1.istride] : gr) * P1.ld + kc : 0;
    ao2[q] = np > 2 ? (P2.idx ? (int64_t)P2.idx[gr * P2.istride] : gr) * P2.ld + kc : 0;
    bo[q] = min(col_blk + r, n - 1) * ldb + kc;
    soff[q] = r * 16 + (((kc >> 3) ^ ((r >> 3) & 1)) * 8) + (kc & 7);
  }
  const int rd = rr * 16 + ((h ^ ((rr >> 3) & 1)) * 8);  // this lane's 8 k of its MFMA row
  float4 ra0[AQ], rb0[BQ];
  f32x16 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, 16);
  X3_LOAD(0, 0);
  X3_STORE(0, 0);
  if (nk > 1) X3_LOAD(16, 0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) {
      X3_STORE(cur ^ 1, 0);                       // slice kt + 1 (loaded one iteration ago)
      if (kt + 2 < nk) X3_LOAD((kt + 2) * 16, 0);  // slice kt + 2 stays in flight over these MFMAs
    }
    X3_COMPUTE(cur, MB);
    __syncthreads();  // buffer cur is free, buffer cur ^ 1 is complete
  }
  const int64_t row0 = row_blk + wm * 32 * MB, col0 = col_blk + wn * 64;
  x3_finish<MB>(acc, radd, bias, c, ldc, m, n, accumulate, act, row0, col0, h, rr);
}

template <int BN>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) gemm_x3_kernel(X3Part P0, X3Part P1, X3Part P2, int np,
                                                           const float* __restrict__ b, int64_t ldb, X3Part radd,
                                                           const float* __restrict__ bias, float* c, int64_t ldc,
                                                           int64_t m, int64_t n, int64_t k, int accumulate, int act,
                                                           int64_t n_tiles) {
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  x3_tile<BN>(P0, P1, P2, np, b, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, (tile / n_tiles) * 128,
              (tile % n_tiles) * BN);
}

// ------------------------------------------------- fp32 as three bf16 planes, pre-split operands
// The same product as gemm_x3_kernel (same planes, same six MFMA products in the same order, same
// K order: bitwise the same C) with the operands split into their bf16 planes beforehand
// (split3_kernel): B always (a weight, split once), A either as planes (the planes of per-atom
// features and per-edge radial rows, split once per evaluation instead of once per column tile:
// gemm_x3p_dma_kernel) or fp32 split here (gemm_x3p_kernel). Plane arrays are slice-interleaved,
// [rows][S][3][16] bf16 (S = width / 16 rounded up, zero past the width): the three planes of a
// row's 16-k slice are 96 contiguous bytes, so a slice of a gathered row is one contiguous read.
// An operand slice in LDS is 768 16-byte slots: slot s holds plane s / 256 of row (s / 2) % 128,
// stored half s % 2 (logical k-half (s % 2) ^ ((row / 8) % 2), the swizzle X3_COMPUTE reads).
// Plane loads copy 16-byte chunks without arithmetic, slot s by thread s % 256 (consecutive
// lanes on consecutive slots: conflict-free LDS stores).
struct X3PPart {
  const void* src;
  const int32_t* idx;
  int64_t ld, istride;  // ld: row stride in elements (48 S for planes)
  int32_t width;
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// XP_LOAD(K0, S): slice K0 into register stage S (ra##S for A, pb##S for B's planes);
// XP_STORE(BUFI, S): stage S into LDS buffer BUFI
#define XP_LOAD(K0, S)                                                                              \
  do {                                                                                              \
    const int64_t k0_ = (K0);                                                                       \
    const bool q2_ = k0_ >= ks2, q1_ = !q2_ && k0_ >= ks1;                                          \
    const float* base_ = q2_ ? fa2 : q1_ ? fa1 : fa0;                                               \
    const int64_t kin_ = q2_ ? k0_ - ks2 : q1_ ? k0_ - ks1 : k0_;                                   \
    const int w_ = q2_ ? w2 : q1_ ? w1 : w0;                                                        \
    _Pragma("unroll") for (int q = 0; q < MB; ++q) {                                                \
      const int64_t o_ = q2_ ? ao2[q] : q1_ ? ao1[q] : ao0[q];                                      \
      ra##S[q] = (kin_ + kc < w_) ? *reinterpret_cast<const float4*>(base_ + o_ + kin_)             \
                                  : make_float4(0.f, 0.f, 0.f, 0.f);                                \
    }                                                                                               \
    _Pragma("unroll") for (int j = 0; j < 3; ++j)                                                   \
      pb##S[j] = *reinterpret_cast<const u32x4*>(bp + bo[j] + k0_ * 3);                            \
  } while (0)

#define XP_STORE(BUFI, S)                                                                           \
  do {                                                                                              \
    __bf16* sb_ = lds + (BUFI) * X3_BUF;                                                            \
    _Pragma("unroll") for (int q = 0; q < MB; ++q) {                                                \
      bf16x4 x0_, x1_, x2_;                                                                         \
      split3(ra##S[q], x0_, x1_, x2_);                                                              \
      *reinterpret_cast<bf16x4*>(sb_ + 0 * X3_PL + soff[q]) = x0_;                                  \
      *reinterpret_cast<bf16x4*>(sb_ + 1 * X3_PL + soff[q]) = x1_;                                  \
      *reinterpret_cast<bf16x4*>(sb_ + 2 * X3_PL + soff[q]) = x2_;                                  \
    }                                                                                               \
    _Pragma("unroll") for (int j = 0; j < 3; ++j)                                                   \
      *reinterpret_cast<u32x4*>(sb_ + X3_OP + (t + j * kThreads) * 8) = pb##S[j];                  \
  } while (0)

// One (64 MB) x 128 tile with fp32 A (MB as in x3_tile) and B's planes. Two register stages
// (loads issued two slices ahead) measured no faster than one at two waves per SIMD instead of
// three, so the tile keeps one stage: slice kt + 1 is stored into LDS and slice kt + 2 loaded into
// the stage while the MFMAs of slice kt run.
template <int MB>
__device__ __forceinline__ void x3p_tile(const X3PPart& P0, const X3PPart& P1, const X3PPart& P2, int np,
                                         const __bf16* __restrict__ bp, int64_t ldb, const X3Part& radd,
                                         const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n,
                                         int64_t k, int accumulate, int act, int64_t row_blk, int64_t col_blk) {
  __shared__ __attribute__((aligned(16))) __bf16 lds[2 * X3_BUF];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, rr = lane & 31;
  const int64_t ks1 = P0.width, ks2 = ks1 + (np > 1 ? P1.width : 0);
  const int w0 = P0.width, w1 = P1.width, w2 = P2.width;
  const float *fa0 = static_cast<const float*>(P0.src), *fa1 = static_cast<const float*>(P1.src),
              *fa2 = static_cast<const float*>(P2.src);
  // B planes: slot t + 256 j (plane j)
  int64_t bo[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int r = (t >> 1) & 127, hf = (t & 1) ^ ((r >> 3) & 1);
    bo[j] = min(col_blk + r, n - 1) * ldb + j * 16 + hf * 8;
  }
  // fp32 A: row (t + 256 q) / 4, k (t % 4) * 4
  const int kc = (t & 3) * 4;
  int64_t ao0[2], ao1[2], ao2[2];
  int soff[2];
#pragma unroll
  for (int q = 0; q < MB; ++q) {
    const int r = (t + q * kThreads) >> 2;
    const int64_t gr = min(row_blk + r, m - 1);
    ao0[q] = (P0.idx ? (int64_t)P0.idx[gr * P0.istride] : gr) * P0.ld + kc;
    ao1[q] = np > 1 ? (P1.idx ? (int64_t)P1.idx[gr * P1.istride] : gr) * P1.ld + kc : 0;
    ao2[q] = np > 2 ? (P2.idx ? (int64_t)P2.idx[gr * P2.istride] : gr) * P2.ld + kc : 0;
    soff[q] = r * 16 + (((kc >> 3) ^ ((r >> 3) & 1)) * 8) + (kc & 7);
  }
  const int rd = rr * 16 + ((h ^ ((rr >> 3) & 1)) * 8);  // this lane's 8 k of its MFMA row
  u32x4 pb0[3];
  float4 ra0[MB];
  f32x16 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, 16);
  XP_LOAD(0, 0);
  XP_STORE(0, 0);
  if (nk > 1) XP_LOAD(16, 0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) {
      XP_STORE(cur ^ 1, 0);                       // slice kt + 1 (loaded one iteration ago)
      if (kt + 2 < nk) XP_LOAD((kt + 2) * 16, 0);  // slice kt + 2 stays in flight over these MFMAs
    }
    X3_COMPUTE(cur, MB);
    __syncthreads();  // buffer cur is free, buffer cur ^ 1 is complete
  }
  const int64_t row0 = row_blk + wm * 32 * MB, col0 = col_blk + wn * 64;
  x3_finish<MB>(acc, radd, bias, c, ldc, m, n, accumulate, act, row0, col0, h, rr);
}

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) gemm_x3p_kernel(
    X3PPart P0, X3PPart P1, X3PPart P2, int np, const __bf16* __restrict__ bp, int64_t ldb, X3Part radd,
    const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int accumulate, int act,
    int64_t n_tiles) {
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  x3p_tile<2>(P0, P1, P2, np, bp, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, (tile / n_tiles) * 128,
                    (tile % n_tiles) * 128);
}

// The product with both operands as planes, copied straight into LDS by the memory system
// (global_load_lds_dwordx4: no register stage, no VALU, no LDS bank conflicts), three LDS stages
// (72 KB, two workgroups per CU): the loads of slice kt + 2 are in flight while slice kt feeds the
// MFMAs. Wave w's load instruction j fills the slots (3 w + j) * 64 + lane of an operand's region
// (the slot layout above). The three stages are separate arrays and every slice issues its loads
// unconditionally (the tail re-loads the last slice into a free stage), so the compiler's wait
// tracking for LDS-bound loads stays exact; the waits between stages are explicit vmcnt counts
// (six loads per wave per slice, returned in order). Same planes, same products, same K order:
// bitwise the C of gemm_x3_kernel. Measured at the 10 000-atom edge GEMM: 6 % faster than staging
// the planes through registers (waves spend half as long waiting), with three stages at two
// workgroups per CU.
constexpr int XD_STAGE = 2 * X3_OP;                      // bf16 elements per stage (A then B region)
constexpr int kVmcnt6 = 6 | (7 << 4) | (15 << 8);         // s_waitcnt vmcnt(6): the older slice landed
constexpr int kVmcnt0 = 0 | (7 << 4) | (15 << 8);         // s_waitcnt vmcnt(0)

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void lds_dma16(const __bf16* g, __bf16* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)l, 16, 0, 0);
}

#define XD_ISSUE(K0, STAGE)                                                                         \
  do {                                                                                              \
    const int64_t k0_ = (K0);                                                                       \
    const bool q2_ = k0_ >= ks2, q1_ = !q2_ && k0_ >= ks1;                                          \
    const __bf16* base_ = q2_ ? ap2 : q1_ ? ap1 : ap0;                                              \
    const int64_t kin_ = q2_ ? k0_ - ks2 : q1_ ? k0_ - ks1 : k0_;                                   \
    __bf16* sa_ = (STAGE) + dst0;                                                                   \
    _Pragma("unroll") for (int j = 0; j < 3; ++j)                                                   \
      lds_dma16(base_ + (q2_ ? ao2[j] : q1_ ? ao1[j] : ao0[j]) + kin_ * 3, sa_ + j * 512);          \
    _Pragma("unroll") for (int j = 0; j < 3; ++j)                                                   \
      lds_dma16(bp + bo[j] + k0_ * 3, sa_ + X3_OP + j * 512);                                       \
  } while (0)

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) gemm_x3p_dma_kernel(
    X3PPart P0, X3PPart P1, X3PPart P2, int np, const __bf16* __restrict__ bp, int64_t ldb, X3Part radd,
    const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int accumulate, int act,
    int64_t n_tiles) {
  __shared__ __attribute__((aligned(16))) __bf16 st0[XD_STAGE];
  __shared__ __attribute__((aligned(16))) __bf16 st1[XD_STAGE];
  __shared__ __attribute__((aligned(16))) __bf16 st2[XD_STAGE];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, rr = lane & 31;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t row_blk = (tile / n_tiles) * 128, col_blk = (tile % n_tiles) * 128;
  const int64_t ks1 = P0.width, ks2 = ks1 + (np > 1 ? P1.width : 0);
  const __bf16 *ap0 = static_cast<const __bf16*>(P0.src), *ap1 = static_cast<const __bf16*>(P1.src),
               *ap2 = static_cast<const __bf16*>(P2.src);
  int64_t ao0[3], ao1[3], ao2[3], bo[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int sl = (wave * 3 + j) * 64 + lane, pl = sl >> 8, r = (sl >> 1) & 127;
    const int sub = pl * 16 + (((sl & 1) ^ ((r >> 3) & 1)) * 8);
    const int64_t gr = min(row_blk + r, m - 1);
    ao0[j] = (P0.idx ? (int64_t)P0.idx[gr * P0.istride] : gr) * P0.ld + sub;
    ao1[j] = np > 1 ? (P1.idx ? (int64_t)P1.idx[gr * P1.istride] : gr) * P1.ld + sub : 0;
    ao2[j] = np > 2 ? (P2.idx ? (int64_t)P2.idx[gr * P2.istride] : gr) * P2.ld + sub : 0;
    bo[j] = min(col_blk + r, n - 1) * ldb + sub;
  }
  const int dst0 = wave * 3 * 512;  // element offset of this wave's first slot in a region
  const int rd = rr * 16 + ((h ^ ((rr >> 3) & 1)) * 8);
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, 16), last = (nk - 1) * 16;
  XD_ISSUE(0, st0);
  XD_ISSUE(min((int64_t)16, last), st1);
#define XD_BLOCK(NEXT, ISSUE_STAGE, STAGE)                                                          \
  do {                                                                                              \
    __builtin_amdgcn_s_waitcnt(kVmcnt6);                                                            \
    __builtin_amdgcn_s_barrier();                                                                   \
    XD_ISSUE(min((NEXT) * 16, last), ISSUE_STAGE);                                                  \
    const __bf16* lds = STAGE;                                                                      \
    X3_COMPUTE(0, 2);                                                                               \
  } while (0)
  // stage 0 holds slice kt, stage 1 slice kt + 1; each block issues slice kt + 2 into the stage
  // freed by the block before
  int64_t kt = 0;
  for (; kt + 3 <= nk; kt += 3) {
    XD_BLOCK(kt + 2, st2, st0);
    XD_BLOCK(kt + 3, st0, st1);
    XD_BLOCK(kt + 4, st1, st2);
  }
  if (kt < nk) XD_BLOCK(kt + 2, st2, st0);
  if (kt + 1 < nk) XD_BLOCK(kt + 3, st0, st1);
#undef XD_BLOCK
  __builtin_amdgcn_s_waitcnt(kVmcnt0);  // no load into LDS outlives the workgroup
  constexpr int MB = 2;
  const int64_t row0 = row_blk + wm * 64, col0 = col_blk + wn * 64;
  x3_finish<MB>(acc, radd, bias, c, ldc, m, n, accumulate, act, row0, col0, h, rr);
}

#undef XD_ISSUE

// ---------------------------------------------------- bf16 operands, copied straight into LDS
// C = A B^T (+ bias) (+ C) with bf16 A [M, K] and B [N, K], both K-contiguous (rows 16-byte
// aligned, K % 8 == 0): the HBM-bound form of the edge GEMM (bf16 in, fp32 out). Every 16-byte
// chunk of an operand slice goes from global memory straight into LDS (global_load_lds_dwordx4:
// no register stage, no VALU). Four LDS stages of 32 k (64 KB, two workgroups per CU) keep the
// loads of slices kt + 1 .. kt + 3 in flight over slice kt's MFMAs; one v_mfma_f32_32x32x16_bf16
// per 32 x 32 block and 16 k, K in order (the products and their order of the register-staged
// gemm_bf16_kernel: the same C). An operand stage is 512 slots of 16 bytes: wave w's load j fills
// slots (2 w + j) * 64 + lane, slot s holds row s / 4 of the tile and its k chunk
// (s % 4) ^ ((row / 4) % 4), so the sixteen 16-byte operand reads of a quarter wave (16
// consecutive rows, one chunk) fall on distinct banks. Chunks past K, and every chunk of a slice
// past the last one (the loads are issued unconditionally so the vmcnt waits stay exact), are read
// from a zero chunk. Rows past M / N are clamped to the last row (computed, never stored).
// 128 x 128 tiles in XCD-aware order (the column tiles of one row block share an XCD's L2),
// streaming stores for interior tiles.
constexpr int BD_K = 32, BD_OP = 128 * BD_K, BD_STAGE = 2 * BD_OP;  // bf16 elements
constexpr int kVmcnt8 = 8 | (7 << 4) | (15 << 8);                  // s_waitcnt vmcnt(8)
__device__ __attribute__((aligned(16))) uint32_t g_bf16_zero_chunk[4];

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) gemm_bf16_dma_kernel(
    const __bf16* __restrict__ a, int64_t lda, const __bf16* __restrict__ b, int64_t ldb,
    const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int accumulate, int act,
    int64_t n_tiles) {
  __shared__ __attribute__((aligned(16))) __bf16 st0[BD_STAGE];
  __shared__ __attribute__((aligned(16))) __bf16 st1[BD_STAGE];
  __shared__ __attribute__((aligned(16))) __bf16 st2[BD_STAGE];
  __shared__ __attribute__((aligned(16))) __bf16 st3[BD_STAGE];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, rr = lane & 31;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t row_blk = (tile / n_tiles) * 128, col_blk = (tile % n_tiles) * 128;
  const __bf16* zero = reinterpret_cast<const __bf16*>(g_bf16_zero_chunk);
  // this lane's two slots per operand: row offsets and the chunk's k
  int64_t ao[2], bo[2];
  int kc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int s = (wave * 2 + j) * 64 + lane, r = s >> 2;
    kc[j] = ((s & 3) ^ ((r >> 2) & 3)) * 8;
    ao[j] = min(row_blk + r, m - 1) * lda + kc[j];
    bo[j] = min(col_blk + r, n - 1) * ldb + kc[j];
  }
  const int dst0 = wave * 2 * 512;  // element offset of this wave's first slot in an operand region
  // this lane's operand reads: row (32-row block base + rr), logical chunk 2 kk + h
  int rdo[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) rdo[kk] = rr * BD_K + (((2 * kk + h) ^ ((rr >> 2) & 3)) * 8);
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk = fmd_cdiv(k, BD_K);
#define BD_ISSUE(SLICE, STAGE)                                                                      \
  do {                                                                                              \
    const int64_t s_ = (SLICE), k0_ = s_ * BD_K;                                                    \
    const bool live_ = s_ < nk;                                                                     \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                                 \
      const bool ok_ = live_ && k0_ + kc[j] < k;                                                    \
      const __bf16* src_ = ok_ ? a + ao[j] + k0_ : zero;                                            \
      asm volatile("" : "+v"(src_)); /* one load instruction with a per-lane address */             \
      lds_dma16(src_, (STAGE) + dst0 + j * 512);                                                    \
    }                                                                                               \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                                 \
      const bool ok_ = live_ && k0_ + kc[j] < k;                                                    \
      const __bf16* src_ = ok_ ? b + bo[j] + k0_ : zero;                                            \
      asm volatile("" : "+v"(src_));                                                                \
      lds_dma16(src_, (STAGE) + BD_OP + dst0 + j * 512);                                            \
    }                                                                                               \
  } while (0)
#define BD_BLOCK(NEXT, ISSUE_STAGE, STAGE)                                                          \
  do {                                                                                              \
    __builtin_amdgcn_s_waitcnt(kVmcnt8); /* this wave's loads of the slice landed */                \
    __builtin_amdgcn_s_barrier();        /* everyone's, and the stage to refill is read */          \
    BD_ISSUE(NEXT, ISSUE_STAGE);                                                                    \
    const __bf16* as_ = (STAGE) + (wm * 64) * BD_K;                                                 \
    const __bf16* bs_ = (STAGE) + BD_OP + (wn * 64) * BD_K;                                         \
    _Pragma("unroll") for (int kk = 0; kk < 2; ++kk) {                                              \
      bf16x8 av_[2], bv_[2];                                                                        \
      _Pragma("unroll") for (int i = 0; i < 2; ++i)                                                 \
        av_[i] = *reinterpret_cast<const bf16x8*>(as_ + i * 32 * BD_K + rdo[kk]);                   \
      _Pragma("unroll") for (int j = 0; j < 2; ++j)                                                 \
        bv_[j] = *reinterpret_cast<const bf16x8*>(bs_ + j * 32 * BD_K + rdo[kk]);                   \
      _Pragma("unroll") for (int i = 0; i < 2; ++i) _Pragma("unroll") for (int j = 0; j < 2; ++j)  \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av_[i], bv_[j], acc[i][j], 0, 0, 0);    \
    }                                                                                               \
  } while (0)
  BD_ISSUE(0, st0);
  BD_ISSUE(1, st1);
  BD_ISSUE(2, st2);
  // stage q holds slice kt with kt % 4 == q; each block refills the stage the block before read
  int64_t kt = 0;
  for (; kt + 4 <= nk; kt += 4) {
    BD_BLOCK(kt + 3, st3, st0);
    BD_BLOCK(kt + 4, st0, st1);
    BD_BLOCK(kt + 5, st1, st2);
    BD_BLOCK(kt + 6, st2, st3);
  }
  if (kt < nk) BD_BLOCK(kt + 3, st3, st0);
  if (kt + 1 < nk) BD_BLOCK(kt + 4, st0, st1);
  if (kt + 2 < nk) BD_BLOCK(kt + 5, st1, st2);
#undef BD_BLOCK
#undef BD_ISSUE
  __builtin_amdgcn_s_waitcnt(kVmcnt0);  // no load into LDS outlives the workgroup
  const X3Part none{};
  x3_finish<2>(acc, none, bias, c, ldc, m, n, accumulate, act, row_blk + wm * 64, col_blk + wn * 64, h, rr);
}

// bf16 GEMM for tall A (tens of thousands of edge rows and more, K <= 544) with a column slab of
// B resident in LDS. Each workgroup has 8 waves, at most two per SIMD, so that the whole K extent
// of a wave's A rows and its 32 x 32 NCB accumulators fit in registers. It copies NSL slabs of
// 32 NCB of B's rows (columns of C) once, zero-padded to Kp = 16 ceil(K / 16), with a row stride
// of Kp + 8 elements (odd multiples of 4 dwords: conflict-free 16-byte reads). It then walks row
// blocks of 256 rows, a wave per 32 rows. A wave loads its rows' whole K extent straight into
// registers (one 16-byte load per lane and k-step, issued together), then, slab by slab, runs the
// k-steps in order over the NCB column blocks and stores them. Each A row is read once per
// workgroup column range (N / (32 NCB NSL) times) and B once per workgroup;
// the 128 x 128 tiles read both operands per tile. Workgroup w runs on XCD w % 8, and the slabs of
// one row walker are placed on the same XCD, so the walker's rows come from HBM once per XCD L2.
// Per element it runs the same MFMA sequence over the same k-steps as the 128 x 128 kernels
// (k-steps of 16 in order, zero chunk past K): bitwise their result.
constexpr int BR_WAVES = 8, BR_ROWS = 32 * BR_WAVES;

// KR = 2 (one slab only, K up to 2 NKS k-steps): a wave holds NKS k-steps of its rows at a time;
// as each k-step's MFMAs are issued its register is refilled with k-step NKS + ks, and a second
// round runs those (K still in order, the same result as one round over all k-steps).
template <int NCB, int NKS, int NSL, int KR = 1>
__global__ void __launch_bounds__(64 * BR_WAVES) __attribute__((amdgpu_waves_per_eu(1, 2))) gemm_bf16_bres_kernel(
    const __bf16* __restrict__ a, int64_t lda, const __bf16* __restrict__ b, int64_t ldb,
    const float* __restrict__ bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int accumulate, int act,
    int n_slabs, int walkers) {
  static_assert(KR == 1 || (KR == 2 && NSL == 1), "a second round of k-steps overwrites the first: one slab");
  constexpr int NB = 32 * NCB, SKMAX = 16 * NKS * KR + 8;
  __shared__ __attribute__((aligned(16))) __bf16 sb[NSL * NB * SKMAX];
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5, rr = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int w = blockIdx.x, xcd = w & 7, u = w >> 3;
  const int slab = u % n_slabs, walker = xcd + 8 * (u / n_slabs);
  const int nks = (int)fmd_cdiv(k, 16), sk = 16 * nks + 8;
  const int64_t col_blk = (int64_t)slab * NSL * NB;
  // the slab of B: 16-byte chunks, rows past N clamped (their columns are never stored)
  const int cpr = sk / 8;  // chunks per LDS row (the last one is padding, left unwritten)
  for (int q = t; q < NSL * NB * cpr; q += 64 * BR_WAVES) {
    const int r = q / cpr, kq = (q - r * cpr) * 8;
    if (kq >= 16 * nks) continue;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (kq < k) v = *reinterpret_cast<const uint4*>(b + min(col_blk + r, n - 1) * ldb + kq);
    *reinterpret_cast<uint4*>(sb + r * sk + kq) = v;
  }
  __syncthreads();
  const __bf16* zero = reinterpret_cast<const __bf16*>(g_bf16_zero_chunk);
  const int64_t n_rb = fmd_cdiv(m, BR_ROWS);
  const X3Part none{};
  for (int64_t rb = walker; rb < n_rb; rb += walkers) {
    const int64_t row0 = rb * BR_ROWS + wave * 32;
    if (row0 >= m) break;  // uniform per wave; the wave's later row blocks start further on
    const __bf16* ap = a + min(row0 + rr, m - 1) * lda + 8 * h;
    // every load unconditional (the zero chunk past K) and in one straight run: the wait before a
    // k-step's MFMAs then covers that k-step's load only
    bf16x8 av[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const __bf16* src = 16 * ks + 8 * h < k ? ap + 16 * ks : zero;
      asm volatile("" : "+v"(src));  // one load with a per-lane address, no branch
      av[ks] = load_global(src);
    }
    // the slabs one after the other on the same A registers (one accumulator set live); unrolled,
    // so that the first slab's MFMAs wait for their own k-step's load only (a loop header makes the
    // compiler wait for every A load)
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      const int64_t col0 = col_blk + (int64_t)sl * NB;
      if (col0 >= n) break;
      f32x16 acc[NCB / 2][1][2];
#pragma unroll
      for (int p = 0; p < NCB / 2; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[p][0][j][v] = 0.f;
      const __bf16* bs = sb + (sl * NB + rr) * sk + 8 * h;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        if (ks < nks) {
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bs + cb * 32 * sk + 16 * ks);
            acc[cb / 2][0][cb % 2] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[ks], bv, acc[cb / 2][0][cb % 2], 0, 0, 0);
          }
        }
        if constexpr (KR == 2) {
          // k-step NKS + ks into the register k-step ks has just been used from
          const __bf16* src = 16 * (NKS + ks) + 8 * h < k ? ap + 16 * (NKS + ks) : zero;
          asm volatile("" : "+v"(src));
          av[ks] = load_global(src);
        }
      }
      if constexpr (KR == 2) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          if (NKS + ks < nks) {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
              const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bs + cb * 32 * sk + 16 * (NKS + ks));
              acc[cb / 2][0][cb % 2] =
                  __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[ks], bv, acc[cb / 2][0][cb % 2], 0, 0, 0);
            }
          }
        }
      }
#pragma unroll
      for (int p = 0; p < NCB / 2; ++p)
        x3_finish<1>(acc[p], none, bias, c, ldc, m, n, accumulate, act, row0, col0 + 64 * p, h, rr);
    }
  }
}

// Several independent GEMMs with pre-split weights in one launch (the node side of an interaction
// layer at thousands of atoms): problem g owns the tiles [tile0[g], tile0[g + 1]) of the XCD-aware
// order, (64 MB) x 128 each; A = [a | a2] fp32 (a's width a multiple of 16), split as it is
// staged; B the planes of a [N, K] weight. Each problem's C is bitwise the one gemm_x3_kernel
// gives for it (same planes, same K order).
struct X3PGroupDesc {
  X3PPart p0, p1;
  int np;
  const __bf16* b;
  const float* bias;
  float* c;
  int64_t ldb, ldc, m, n, k, n_tiles, tile0;
  int accumulate;
  X3Part radd;  // a gathered row added to every row of C (src null: none)
};
struct X3PGroup {
  X3PGroupDesc d[kMaxGroup];
  int count;
  int act;
};

template <int MB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) gemm_x3p_group_kernel(const X3PGroup grp) {
  const int64_t w = xcd_tile(blockIdx.x, gridDim.x);
  int g = 0;
#pragma unroll
  for (int q = 1; q < kMaxGroup; ++q)
    if (q < grp.count && w >= grp.d[q].tile0) g = q;
  const X3PGroupDesc& d = grp.d[g];
  const int64_t t = w - d.tile0;
  x3p_tile<MB>(d.p0, d.p1, d.p1, d.np, d.b, d.ldb, d.radd, d.bias, d.c, d.ldc, d.m, d.n, d.k, d.accumulate,
               grp.act, (t / d.n_tiles) * (64 * MB), (t % d.n_tiles) * 128);
}

#undef XP_LOAD
#undef XP_STORE

// planes[r][s][p][0, 16) = the bf16 planes of src[r][16 s, 16 s + 16) (split3), zero past the
// width (the slice-interleaved operand format of gemm_x3p_kernel); one thread per 8 elements
__global__ void split3_kernel(const float* __restrict__ src, int64_t ld, int64_t rows, int width, __bf16* planes,
                              int64_t slices) {
  const int64_t chunks = slices * 2;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * chunks) return;
  const int64_t r = id / chunks;
  const int c = (int)(id - r * chunks), k0 = c * 8;
  const float* s = src + r * ld + k0;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = k0 + e < width ? s[e] : 0.f;
  bf16x4 p[3][2];
  split3(make_float4(x[0], x[1], x[2], x[3]), p[0][0], p[1][0], p[2][0]);
  split3(make_float4(x[4], x[5], x[6], x[7]), p[0][1], p[1][1], p[2][1]);
  __bf16* d = planes + r * slices * 48 + (c >> 1) * 48 + (c & 1) * 8;
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    *reinterpret_cast<bf16x4*>(d + q * 16) = p[q][0];
    *reinterpret_cast<bf16x4*>(d + q * 16 + 4) = p[q][1];
  }
}

#undef X3_LOAD
#undef X3_STORE
#undef X3_COMPUTE

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// the resident-B bf16 kernel: taken from this many rows (below, the 128 x 128 tiles fill the chip
// with fewer re-reads to save); one workgroup per CU of MI355X's 256
constexpr int64_t kBresMinRows = 32768;
constexpr int kBresWorkgroups = 256;

bool k_fits_int(int32_t n_parts, const int32_t* widths) {
  if (n_parts < 1 || n_parts > 3) return false;
  int64_t k = 0;
  for (int p = 0; p < n_parts; ++p) {
    if (widths[p] <= 0) return false;
    k += widths[p];
  }
  return k < (int64_t(1) << 30);
}

// Launch of gemm_x3_kernel; FMD_EUNSUPPORTED when the parts do not meet its layout conditions.
int launch_gemm_x3(int32_t n_parts, const float* const* srcs, const int32_t* const* indices,
                   const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                   const float* b, int64_t ldb, const float* row_add, const int32_t* row_add_index,
                   int64_t row_add_index_stride, int64_t ld_row_add, const float* bias, float* c, int64_t ldc,
                   int64_t n, int32_t accumulate, int32_t act, hipStream_t stream) {
  if (n_parts < 1 || n_parts > 3) return FMD_EUNSUPPORTED;
  X3Part P[3] = {};
  int64_t k = 0;
  for (int p = 0; p < n_parts; ++p) {
    if (!srcs[p] || widths[p] <= 0 || widths[p] % 4 || (p + 1 < n_parts && widths[p] % 16)) return FMD_EUNSUPPORTED;
    if (!aligned16(srcs[p]) || lds[p] % 4) return FMD_EUNSUPPORTED;
    P[p] = X3Part{srcs[p], indices ? indices[p] : nullptr, lds[p], index_strides ? index_strides[p] : 1, widths[p]};
    if (P[p].istride < 1) return FMD_EINVAL;
    k += widths[p];
  }
  if (!b || !aligned16(b) || ldb % 4 || ldb < k) return FMD_EUNSUPPORTED;
  X3Part radd{row_add, row_add_index, ld_row_add, row_add_index_stride, 0};
  if (row_add && (ld_row_add < n || row_add_index_stride < 1)) return FMD_EINVAL;
  // 128 x 64 tiles for N <= 64 (the three-body model's edge rows): no idle half tile
  const int64_t bn = n <= 64 ? 64 : 128;
  const int64_t n_tiles = fmd_cdiv(n, bn), tiles = fmd_cdiv(m, 128) * n_tiles;
  if (tiles >= (int64_t(1) << 31)) return FMD_EINVAL;
  if (bn == 64)
    hipLaunchKernelGGL(gemm_x3_kernel<64>, dim3((unsigned)tiles), dim3(kThreads), 0, stream, P[0], P[1], P[2], n_parts,
                       b, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, n_tiles);
  else
    hipLaunchKernelGGL(gemm_x3_kernel<128>, dim3((unsigned)tiles), dim3(kThreads), 0, stream, P[0], P[1], P[2], n_parts,
                       b, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, n_tiles);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

// Grouped split-plane launches use 64-row tiles below this many tiles of 128 x 128 (eight per CU;
// the MACE-like merged node group at 10 000 / 16 875 / 40 000 atoms, 946 to 3 755 such tiles, ran
// 16 / 9 / 20 us per step faster on 64-row tiles than with the switch at three per CU).
constexpr int64_t kGroupX3HalfTilesBelow = 8 * 256;

// Tile choice: 128 x 128 when that still gives two workgroups per CU (256 CUs), else 64 x 64
// (small node-side GEMMs and the 135-atom edge GEMM: 4x more workgroups, 4x less serial K work
// per wave).
template <int BM, int BN>
void launch_gemm_f32(const float* a, int64_t lda, const float* b, int64_t ldb, int32_t b_layout,
                            const float* bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                            int32_t accumulate, int32_t act, hipStream_t stream) {
  dim3 grid((unsigned)fmd_cdiv(m, BM), (unsigned)fmd_cdiv(n, BN));
  if (b_layout == 0)
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, 0>), grid, dim3(kThreads), 0, stream, a, lda, b, ldb, bias, c, ldc, m,
                       n, k, accumulate, act);
  else
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, 1>), grid, dim3(kThreads), 0, stream, a, lda, b, ldb, bias, c, ldc, m,
                       n, k, accumulate, act);
}

// Launch of gemm_x3p_kernel (B as slice-interleaved planes, row stride ldb = 48 ceil(K / 16)); A
// parts as planes (a_planes, row stride 48 ceil(width / 16)) or fp32 (the conditions of
// launch_gemm_x3); FMD_EUNSUPPORTED otherwise.
int launch_gemm_x3p(int32_t a_planes, int32_t n_parts, const void* const* srcs, const int32_t* const* indices,
                    const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                    const uint16_t* bp, int64_t ldb, int64_t k_b, const float* row_add, const int32_t* row_add_index,
                    int64_t row_add_index_stride, int64_t ld_row_add, const float* bias, float* c, int64_t ldc,
                    int64_t n, int32_t accumulate, int32_t act, hipStream_t stream) {
  if (n_parts < 1 || n_parts > 3) return FMD_EUNSUPPORTED;
  X3PPart P[3] = {};
  int64_t k = 0;
  for (int p = 0; p < n_parts; ++p) {
    if (!srcs[p] || widths[p] <= 0 || !aligned16(srcs[p])) return FMD_EUNSUPPORTED;
    if (p + 1 < n_parts && widths[p] % 16) return FMD_EUNSUPPORTED;
    if (a_planes ? (widths[p] % 8 || lds[p] != 48 * fmd_cdiv(widths[p], 16)) : (widths[p] % 4 || lds[p] % 4))
      return FMD_EUNSUPPORTED;
    P[p] = X3PPart{srcs[p], indices ? indices[p] : nullptr, lds[p], index_strides ? index_strides[p] : 1, widths[p]};
    if (P[p].istride < 1) return FMD_EINVAL;
    k += widths[p];
  }
  if (k != k_b) return FMD_EINVAL;
  if (!bp || !aligned16(bp) || ldb != 48 * fmd_cdiv(k, 16)) return FMD_EUNSUPPORTED;
  X3Part radd{row_add, row_add_index, ld_row_add, row_add_index_stride, 0};
  if (row_add && (ld_row_add < n || row_add_index_stride < 1)) return FMD_EINVAL;
  const int64_t n_tiles = fmd_cdiv(n, 128), tiles = fmd_cdiv(m, 128) * n_tiles;
  if (tiles >= (int64_t(1) << 31)) return FMD_EINVAL;
  const __bf16* b = reinterpret_cast<const __bf16*>(bp);
  if (a_planes)
    hipLaunchKernelGGL(gemm_x3p_dma_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, stream, P[0], P[1], P[2],
                       n_parts, b, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, n_tiles);
  else
    hipLaunchKernelGGL(gemm_x3p_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, stream, P[0], P[1], P[2],
                       n_parts, b, ldb, radd, bias, c, ldc, m, n, k, accumulate, act, n_tiles);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // namespace

extern "C" {

int fmd_split3_f32(const float* src, int64_t ld, int64_t rows, int32_t width, uint16_t* planes, hipStream_t stream) {
  FMD_REQUIRE(rows >= 0 && width > 0 && ld >= width);
  if (rows == 0) return FMD_OK;
  FMD_REQUIRE(src && planes && aligned16(planes));
  const int64_t slices = fmd_cdiv(width, 16), threads = rows * slices * 2;
  hipLaunchKernelGGL(split3_kernel, dim3((unsigned)fmd_cdiv(threads, 256)), dim3(256), 0, stream, src, ld, rows, width,
                     reinterpret_cast<__bf16*>(planes), slices);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_x3_planes_f32(int32_t a_planes, int32_t n_parts, const void* const* srcs, const int32_t* const* indices,
                           const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                           const uint16_t* b_planes, int64_t ldb, int64_t k, const float* row_add,
                           const int32_t* row_add_index, int64_t row_add_index_stride, int64_t ld_row_add,
                           const float* bias, float* c, int64_t ldc, int64_t n, int32_t accumulate,
                           int32_t epilogue_kind, hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && c && ldc >= n && srcs && lds && widths);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(k_fits_int(n_parts, widths));
  return launch_gemm_x3p(a_planes, n_parts, srcs, indices, index_strides, lds, widths, m, b_planes, ldb, k, row_add,
                         row_add_index, row_add_index_stride, ld_row_add, bias, c, ldc, n, accumulate, epilogue_kind,
                         stream);
}

int fmd_gemm_f32(const float* a, int64_t lda, const float* b, int64_t ldb, int32_t b_layout, const float* bias,
                 float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t epilogue_kind,
                 hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && k >= 0 && c && ldc >= n);
  FMD_REQUIRE(b_layout == 0 || b_layout == 1);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(k == 0 || (a && b && lda >= k && ldb >= (b_layout == 0 ? k : n)));
  FMD_REQUIRE(fmd_cdiv(m, 64) < (int64_t(1) << 31) && fmd_cdiv(n, 64) < 65536);
  {
    // K <= 16 or N <= 16: fp32 FMA chains on the vector ALUs (thin.hip)
    const int st = launch_gemm_thin(a, lda, b, ldb, b_layout, bias, c, ldc, m, n, k, accumulate, epilogue_kind, stream);
    if (st != FMD_EUNSUPPORTED) return st;
  }
  const int64_t big_tiles = fmd_cdiv(m, 128) * fmd_cdiv(n, 128);
  if (big_tiles >= 256 && b_layout == 0 && k > 0 && k % 4 == 0) {
    // fp32-accurate on the bf16 matrix cores when the operands allow 16-byte loads (from 256
    // tiles of 128 x 128: below that the 64 x 64 fp32 kernel's four times more workgroups win)
    const int64_t lda64 = lda;
    const int32_t width = (int32_t)k;
    const int st = launch_gemm_x3(1, &a, nullptr, nullptr, &lda64, &width, m, b, ldb, nullptr, nullptr, 1, 0, bias, c,
                                  ldc, n, accumulate, epilogue_kind, stream);
    if (st != FMD_EUNSUPPORTED) return st;
  }
  if (big_tiles >= 512 && b_layout == 0) {
    FMD_REQUIRE(big_tiles < (int64_t(1) << 31));
    const int vec_ok = (lda % 4 == 0) && (ldb % 4 == 0) && ((reinterpret_cast<uintptr_t>(a) & 15) == 0) &&
                       ((reinterpret_cast<uintptr_t>(b) & 15) == 0);
    hipLaunchKernelGGL(gemm_f32_nt_kernel, dim3((unsigned)big_tiles), dim3(kThreads), 0, stream, a, lda, b, ldb, bias,
                       c, ldc, m, n, k, accumulate, epilogue_kind, vec_ok, fmd_cdiv(n, 128));
  } else if (big_tiles >= 512)
    launch_gemm_f32<128, 128>(a, lda, b, ldb, b_layout, bias, c, ldc, m, n, k, accumulate, epilogue_kind, stream);
  else
    launch_gemm_f32<64, 64>(a, lda, b, ldb, b_layout, bias, c, ldc, m, n, k, accumulate, epilogue_kind, stream);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_group_f32(int32_t count, const float* const* a, const int64_t* lda, const float* const* a2,
                       const int64_t* lda2, const int64_t* ksplit, const float* const* b, const int64_t* ldb,
                       int32_t b_layout, const float* const* bias, float* const* c, const int64_t* ldc,
                       const int64_t* m, const int64_t* n, const int64_t* k, const int32_t* accumulate,
                       int32_t epilogue_kind, hipStream_t stream) {
  FMD_REQUIRE(count >= 1 && count <= kMaxGroup && a && lda && b && ldb && c && ldc && m && n && k);
  FMD_REQUIRE(b_layout == 0 || b_layout == 1);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  GemmGroup grp{};
  grp.act = epilogue_kind;
  int64_t tiles = 0;
  for (int g = 0; g < count; ++g) {
    GemmDesc& d = grp.d[grp.count];
    FMD_REQUIRE(m[g] >= 0 && n[g] >= 0 && k[g] >= 0);
    if (m[g] == 0 || n[g] == 0) continue;  // (an empty output may have a null pointer)
    FMD_REQUIRE(c[g] && ldc[g] >= n[g]);
    const bool split = a2 && a2[g];
    const int64_t ks = split ? ksplit[g] : k[g];
    FMD_REQUIRE(k[g] == 0 || (a[g] && b[g] && ldb[g] >= (b_layout == 0 ? k[g] : n[g])));
    FMD_REQUIRE(k[g] == 0 || lda[g] >= ks);
    FMD_REQUIRE(!split || (lda2 && ks > 0 && ks < k[g] && ks % BK32 == 0 && lda2[g] >= k[g] - ks));
    d.a = a[g];
    d.a2 = split ? a2[g] : nullptr;
    d.lda = lda[g];
    d.lda2 = split ? lda2[g] : 0;
    d.ksplit = ks;
    d.b = b[g];
    d.ldb = ldb[g];
    d.bias = bias ? bias[g] : nullptr;
    d.c = c[g];
    d.ldc = ldc[g];
    d.m = m[g];
    d.n = n[g];
    d.k = k[g];
    d.accumulate = accumulate ? accumulate[g] : 0;
    d.tiles_n = fmd_cdiv(n[g], 64);
    d.tile0 = tiles;
    tiles += fmd_cdiv(m[g], 64) * d.tiles_n;
    ++grp.count;
  }
  if (grp.count == 0) return FMD_OK;
  FMD_REQUIRE(tiles < (int64_t(1) << 31));
  if (b_layout == 0)
    hipLaunchKernelGGL(gemm_f32_group_kernel<0>, dim3((unsigned)tiles), dim3(kThreads), 0, stream, grp);
  else
    hipLaunchKernelGGL(gemm_f32_group_kernel<1>, dim3((unsigned)tiles), dim3(kThreads), 0, stream, grp);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_group_x3_planes_f32(int32_t count, const float* const* a, const int64_t* lda, const float* const* a2,
                                 const int64_t* lda2, const int64_t* ksplit, const uint16_t* const* b_planes,
                                 const int64_t* ldb, const float* const* bias, float* const* c, const int64_t* ldc,
                                 const int64_t* m, const int64_t* n, const int64_t* k, const int32_t* accumulate,
                                 int32_t epilogue_kind, hipStream_t stream) {
  return fmd_gemm_group_x3_planes_rows_f32(count, a, lda, a2, lda2, ksplit, b_planes, ldb, bias, c, ldc, m, n, k,
                                           accumulate, nullptr, nullptr, nullptr, epilogue_kind, stream);
}

int fmd_gemm_group_x3_planes_rows_f32(int32_t count, const float* const* a, const int64_t* lda,
                                      const float* const* a2, const int64_t* lda2, const int64_t* ksplit,
                                      const uint16_t* const* b_planes, const int64_t* ldb, const float* const* bias,
                                      float* const* c, const int64_t* ldc, const int64_t* m, const int64_t* n,
                                      const int64_t* k, const int32_t* accumulate, const float* const* row_add,
                                      const int32_t* const* row_index, const int64_t* row_ld, int32_t epilogue_kind,
                                      hipStream_t stream) {
  FMD_REQUIRE(count >= 1 && count <= kMaxGroup && a && lda && b_planes && ldb && c && ldc && m && n && k);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  X3PGroup grp{};
  grp.act = epilogue_kind;
  int64_t big = 0;
  for (int g = 0; g < count; ++g) {
    FMD_REQUIRE(m[g] >= 0 && n[g] >= 0 && k[g] >= 0);
    if (m[g] == 0 || n[g] == 0) continue;
    FMD_REQUIRE(c[g] && ldc[g] >= n[g]);
    const bool split = a2 && a2[g];
    const int64_t ks = split ? ksplit[g] : k[g];
    FMD_REQUIRE(k[g] > 0 && k[g] < (int64_t(1) << 30) && a[g] && b_planes[g] && lda[g] >= ks);
    FMD_REQUIRE(!split || (lda2 && ks > 0 && ks < k[g] && lda2[g] >= k[g] - ks));
    if (!aligned16(a[g]) || lda[g] % 4 || ks % 4 || !aligned16(b_planes[g]) || ldb[g] != 48 * fmd_cdiv(k[g], 16))
      return FMD_EUNSUPPORTED;
    if (split && (ks % 16 || !aligned16(a2[g]) || lda2[g] % 4 || (k[g] - ks) % 4)) return FMD_EUNSUPPORTED;
    X3PGroupDesc& d = grp.d[grp.count++];
    d.p0 = X3PPart{a[g], nullptr, lda[g], 1, (int32_t)ks};
    d.p1 = split ? X3PPart{a2[g], nullptr, lda2[g], 1, (int32_t)(k[g] - ks)} : X3PPart{};
    d.np = split ? 2 : 1;
    d.b = reinterpret_cast<const __bf16*>(b_planes[g]);
    d.bias = bias ? bias[g] : nullptr;
    d.c = c[g];
    d.ldb = ldb[g];
    d.ldc = ldc[g];
    d.m = m[g];
    d.n = n[g];
    d.k = k[g];
    d.n_tiles = fmd_cdiv(n[g], 128);
    d.accumulate = accumulate ? accumulate[g] : 0;
    d.radd = X3Part{};
    if (row_add && row_add[g]) {
      FMD_REQUIRE(row_index && row_index[g] && row_ld && row_ld[g] >= n[g]);
      d.radd = X3Part{row_add[g], row_index[g], row_ld[g], 1, 0};
    }
    big += fmd_cdiv(m[g], 128) * d.n_tiles;
  }
  if (grp.count == 0) return FMD_OK;
  const int mb = big < kGroupX3HalfTilesBelow ? 1 : 2;
  int64_t t0 = 0;
  for (int g = 0; g < grp.count; ++g) {
    grp.d[g].tile0 = t0;
    t0 += fmd_cdiv(grp.d[g].m, 64 * mb) * grp.d[g].n_tiles;
  }
  FMD_REQUIRE(t0 < (int64_t(1) << 31));
  if (mb == 1)
    hipLaunchKernelGGL(gemm_x3p_group_kernel<1>, dim3((unsigned)t0), dim3(kThreads), 0, stream, grp);
  else
    hipLaunchKernelGGL(gemm_x3p_group_kernel<2>, dim3((unsigned)t0), dim3(kThreads), 0, stream, grp);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_splitk_f32(const float* a, int64_t lda, const float* a2, int64_t lda2, int64_t ksplit, const float* b,
                        int64_t ldb, int32_t b_layout, const float* bias, float* c, int64_t ldc, int64_t m, int64_t n,
                        int64_t k, int32_t accumulate, int32_t splits, float* workspace, hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && k > 0 && splits >= 1 && (b_layout == 0 || b_layout == 1));
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(a && b && c && workspace && ldc >= n && k % splits == 0);
  const int64_t ks = k / splits;
  const int64_t ksp = a2 ? ksplit : k;
  FMD_REQUIRE(ks % 32 == 0 && ksp % ks == 0 && lda >= ksp && (!a2 || lda2 >= k - ksp));
  FMD_REQUIRE(ldb >= (b_layout == 0 ? k : n));
  const int64_t tiles_n = fmd_cdiv(n, 64), tiles = fmd_cdiv(m, 64) * tiles_n;
  FMD_REQUIRE(tiles * splits < (int64_t(1) << 31));
  const float* a2p = a2 ? a2 : a;
  const int64_t lda2p = a2 ? lda2 : lda;
  if (b_layout == 0)
    hipLaunchKernelGGL(gemm_f32_splitk_kernel<0>, dim3((unsigned)(tiles * splits)), dim3(kThreads), 0, stream, a, lda,
                       a2p, lda2p, ksp, b, ldb, workspace, m, n, ks, tiles_n, tiles);
  else
    hipLaunchKernelGGL(gemm_f32_splitk_kernel<1>, dim3((unsigned)(tiles * splits)), dim3(kThreads), 0, stream, a, lda,
                       a2p, lda2p, ksp, b, ldb, workspace, m, n, ks, tiles_n, tiles);
  FMD_CHECK_LAUNCH();
  launch_splitk_sum(workspace, splits, m, n, bias, c, ldc, accumulate, stream);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_splitk_x3_planes_f32(const float* a, int64_t lda, const float* a2, int64_t lda2, int64_t ksplit,
                                  const uint16_t* b_planes, int64_t ldb, const float* bias, float* c, int64_t ldc,
                                  int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t splits,
                                  float* workspace, hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && k > 0 && splits >= 1 && splits <= kMaxGroup);
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(a && b_planes && c && workspace && ldc >= n && k % splits == 0 && ldb == 48 * fmd_cdiv(k, 16));
  const int64_t ks = k / splits, ksp = a2 ? ksplit : k;
  FMD_REQUIRE(ks % 16 == 0 && ksp % ks == 0 && lda >= ksp && (!a2 || (ksp < k && lda2 >= k - ksp)));
  FMD_REQUIRE(aligned16(a) && lda % 4 == 0 && aligned16(b_planes) && (!a2 || (aligned16(a2) && lda2 % 4 == 0)));
  FMD_REQUIRE(fmd_cdiv(m, 64) * fmd_cdiv(n, 128) * splits < (int64_t(1) << 31));
  // split s: columns [s ks, (s + 1) ks) of [a | a2] against the same slices of B's planes (16-k
  // slices of 48 bf16 per B row), into workspace slice s
  X3PGroup grp{};
  grp.act = 0;
  int64_t big = 0;
  for (int sp = 0; sp < splits; ++sp) {
    X3PGroupDesc& d = grp.d[grp.count++];
    const int64_t k0 = sp * ks;
    d.p0 = k0 < ksp ? X3PPart{a + k0, nullptr, lda, 1, (int32_t)ks} : X3PPart{a2 + (k0 - ksp), nullptr, lda2, 1, (int32_t)ks};
    d.p1 = X3PPart{};
    d.np = 1;
    d.b = reinterpret_cast<const __bf16*>(b_planes) + (k0 / 16) * 48;
    d.bias = nullptr;
    d.c = workspace + sp * m * n;
    d.ldb = ldb;
    d.ldc = n;
    d.m = m;
    d.n = n;
    d.k = ks;
    d.n_tiles = fmd_cdiv(n, 128);
    d.accumulate = 0;
    d.radd = X3Part{};
    big += fmd_cdiv(m, 128) * d.n_tiles;
  }
  const int mb = big < kGroupX3HalfTilesBelow ? 1 : 2;
  int64_t t0 = 0;
  for (int g = 0; g < grp.count; ++g) {
    grp.d[g].tile0 = t0;
    t0 += fmd_cdiv(m, 64 * mb) * grp.d[g].n_tiles;
  }
  if (mb == 1)
    hipLaunchKernelGGL(gemm_x3p_group_kernel<1>, dim3((unsigned)t0), dim3(kThreads), 0, stream, grp);
  else
    hipLaunchKernelGGL(gemm_x3p_group_kernel<2>, dim3((unsigned)t0), dim3(kThreads), 0, stream, grp);
  FMD_CHECK_LAUNCH();
  launch_splitk_sum(workspace, splits, m, n, bias, c, ldc, accumulate, stream);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_gemm_gather_f32(int32_t n_parts, const float* const* srcs, const int32_t* const* indices,
                        const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                        const float* b, int64_t ldb, const float* row_add, const int32_t* row_add_index,
                        int64_t row_add_index_stride, int64_t ld_row_add, const float* bias, float* c, int64_t ldc,
                        int64_t n, int32_t accumulate, int32_t epilogue_kind, hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && c && ldc >= n && srcs && lds && widths);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(k_fits_int(n_parts, widths));
  return launch_gemm_x3(n_parts, srcs, indices, index_strides, lds, widths, m, b, ldb, row_add, row_add_index,
                        row_add_index_stride, ld_row_add, bias, c, ldc, n, accumulate, epilogue_kind, stream);
}

int fmd_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int32_t b_layout, const float* bias,
                  float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t epilogue_kind,
                  hipStream_t stream) {
  FMD_REQUIRE(m >= 0 && n >= 0 && k >= 0 && c && ldc >= n);
  FMD_REQUIRE(b_layout == 0 || b_layout == 1);
  FMD_REQUIRE(epilogue_kind == 0 || epilogue_kind == 1);
  if (m == 0 || n == 0) return FMD_OK;
  FMD_REQUIRE(k == 0 || (a && b && lda >= k && ldb >= (b_layout == 0 ? k : n)));
  FMD_REQUIRE(fmd_cdiv(m, BM) < (int64_t(1) << 31) && fmd_cdiv(n, BN) < 65536);
  if (b_layout == 0 && k > 0 && k % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned16(a) && aligned16(b) &&
      fmd_cdiv(m, 128) * fmd_cdiv(n, 128) < (int64_t(1) << 31)) {
    const int64_t nks = fmd_cdiv(k, 16);
    if (m >= kBresMinRows && nks <= 34) {
      // tall A, K <= 272 (A's whole K extent in a wave's registers beside its accumulators):
      // B's column slabs resident in LDS. Two 128-column slabs per workgroup (A loaded once for
      // both) when there are row blocks enough for every workgroup at half the slab count, else one
      const int nsl = nks <= 17 && fmd_cdiv(m, BR_ROWS) >= 2 * kBresWorkgroups ? 2 : 1;
      const int n_slabs = (int)fmd_cdiv(n, nsl * 32 * 4);
      const int walkers = max(8, (kBresWorkgroups / n_slabs) & ~7);
      const dim3 grid((unsigned)(walkers * n_slabs)), block(64 * BR_WAVES);
      const __bf16 *ab = reinterpret_cast<const __bf16*>(a), *bb = reinterpret_cast<const __bf16*>(b);
#define BRES_LAUNCH(KS, SL, KR)                                                                              \
  hipLaunchKernelGGL((gemm_bf16_bres_kernel<4, KS, SL, KR>), grid, block, 0, stream, ab, lda, bb, ldb, bias, c, ldc, \
                     m, n, k, accumulate, epilogue_kind, n_slabs, walkers)
      if (nks <= 9) {
        if (nsl == 2) BRES_LAUNCH(9, 2, 1); else BRES_LAUNCH(9, 1, 1);
      } else if (nks <= 17) {
        if (nsl == 2) BRES_LAUNCH(17, 2, 1); else BRES_LAUNCH(17, 1, 1);
      } else {
        BRES_LAUNCH(17, 1, 2);  // K <= 544: one 128-column slab (137-140 KB of LDS), two k-rounds
      }
#undef BRES_LAUNCH
      FMD_CHECK_LAUNCH();
      return FMD_OK;
    }
    // K-contiguous operands with 16-byte aligned rows: the direct-to-LDS pipeline
    const int64_t n_tiles = fmd_cdiv(n, 128), tiles = fmd_cdiv(m, 128) * n_tiles;
    hipLaunchKernelGGL(gemm_bf16_dma_kernel, dim3((unsigned)tiles), dim3(kThreads), 0, stream,
                       reinterpret_cast<const __bf16*>(a), lda, reinterpret_cast<const __bf16*>(b), ldb, bias, c, ldc,
                       m, n, k, accumulate, epilogue_kind, n_tiles);
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  dim3 grid((unsigned)fmd_cdiv(m, BM), (unsigned)fmd_cdiv(n, BN));
  if (b_layout == 0)
    hipLaunchKernelGGL(gemm_bf16_kernel<0>, grid, dim3(kThreads), 0, stream, a, lda, b, ldb, bias, c, ldc, m, n, k,
                       accumulate, epilogue_kind);
  else
    hipLaunchKernelGGL(gemm_bf16_kernel<1>, grid, dim3(kThreads), 0, stream, a, lda, b, ldb, bias, c, ldc, m, n, k,
                       accumulate, epilogue_kind);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
