// GEMMs with a thin side, on the vector ALUs as fp32 FMA chains (no matrix-core split):
//   K <= 16 (outer-product form): C[r, c] = sum_k A[r, k] B(k, c) with the lanes across the
//     columns (<= 256, up to four per lane), the lane's K x 4 values of B in registers and A's
//     values for 16 rows loaded one per lane and read back per row; one wave per 16 rows.
//   N <= 16 (row-dot form): four lanes per row (16 rows per wave), each over every fourth 16-byte
//     chunk of K, B staged in LDS [K][N], the four partial sums added in a fixed butterfly.
// Both store C = A op(B) (+ bias) (+ the old C) and then the activation (1: SiLU), the epilogue of
// the matrix-core kernels. These shapes (a Fourier or radial basis times a weight, its VJP) move
// far more bytes than they do flops: the tiles of the matrix-core kernels, sized for K and N in
// the hundreds, leave them latency-bound.
#include "common.h"

namespace {

constexpr int kThinMaxK = 16, kThinMaxN = 16, kThinRows = 16;
constexpr int kThinNLds = 16384;  // floats of B in LDS for the row-dot form (64 KB)

__device__ __forceinline__ float thin_silu(float x) { return x / (1.0f + __expf(-x)); }

__device__ __forceinline__ float thin_finish(float acc, float bias, const float* dst, int accumulate, int act) {
  float x = acc + bias;
  if (accumulate) x = *dst + x;
  if (act == 1) x = thin_silu(x);
  return x;
}

// op(B)(kk, col): b [K, N] (layout 1) or [N, K] (layout 0)
__device__ __forceinline__ float b_at(const float* b, int64_t ldb, int b_layout, int64_t kk, int64_t col) {
  return b_layout == 1 ? b[kk * ldb + col] : b[col * ldb + kk];
}

// K <= KB (KB a multiple of 4 up to 16; the columns past K hold zeros in A and B), N <= 64 NJ:
// wave w takes rows [16 w, 16 w + 16)
template <int NJ, int KB>
__global__ void __launch_bounds__(256) gemm_thin_k_kernel(const float* a, int64_t lda, const float* b, int64_t ldb,
                                                           int b_layout, const float* bias, float* c, int64_t ldc,
                                                           int64_t m, int64_t n, int k, int accumulate, int act) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64)) * kThinRows;
  if (row0 >= m) return;
  // A: lane l holds A[row0 + 4 g + l / 16, l % 16] in av[g] (zero past K; rows clamped to M)
  float av[kThinRows / 4];
#pragma unroll
  for (int g = 0; g < kThinRows / 4; ++g) {
    const int64_t r = row0 + 4 * g + lane / 16;
    const int kk = lane % 16;
    const float v = a[(r < m ? r : m - 1) * lda + (kk < k ? kk : k - 1)];
    av[g] = kk < k ? v : 0.f;
  }
  // B: the lane's columns lane + 64 j (lanes past N read column N - 1 and store nothing)
  int64_t col[NJ];
  bool live[NJ];
  float bv[KB][NJ], bs[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t cj = lane + 64 * j;
    live[j] = cj < n;
    col[j] = cj < n ? cj : n - 1;
    bs[j] = bias ? bias[col[j]] : 0.f;
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) bv[kk][j] = kk < k ? b_at(b, ldb, b_layout, kk, col[j]) : 0.f;
  }
  const int rows = m - row0 < kThinRows ? (int)(m - row0) : kThinRows;
#pragma unroll 1
  for (int i = 0; i < rows; ++i) {
    const int g = i / 4;  // (a select, not an indexed register array)
    const float ai = g == 0 ? av[0] : g == 1 ? av[1] : g == 2 ? av[2] : av[3];
    float acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
      const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ai), (i % 4) * 16 + kk));
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] = __builtin_fmaf(x, bv[kk][j], acc[j]);
    }
    float* dst = c + (row0 + i) * ldc;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (live[j]) dst[col[j]] = thin_finish(acc[j], bs[j], dst + col[j], accumulate, act);
  }
}

// N <= 4 NQ: a workgroup takes 64 rows, lane l of wave w row 64 blockIdx + 16 w + l / 4 and the
// chunks q, q + 4, ... (q = l % 4) of four K columns, CH chunks per lane and pass (all in flight
// together). VEC: 16-byte loads (K and lda multiples of 4, a aligned).
template <int NQ, int CH, bool VEC>
__global__ void __launch_bounds__(256) gemm_thin_n_kernel(const float* a, int64_t lda, const float* b, int64_t ldb,
                                                           int b_layout, const float* bias, float* c, int64_t ldc,
                                                           int64_t m, int64_t n, int64_t k, int accumulate, int act) {
  // LDS row pitch: the four K rows a quad reads at once (4 apart) start 16 banks apart (64 banks)
  constexpr int NB = 4 * NQ, PITCH = NQ == 1 ? 4 : 20;
  extern __shared__ float4 thin_lds4[];
  float* bsh = reinterpret_cast<float*>(thin_lds4);
  for (int64_t idx = threadIdx.x; idx < k * NB; idx += 256) {
    const int64_t kk = idx / NB, cc = idx % NB;
    bsh[kk * PITCH + cc] = cc < n ? b_at(b, ldb, b_layout, kk, cc) : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, q = lane & 3;
  const int64_t r = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);
  const float* ar = a + (r < m ? r : m - 1) * lda;
  float acc[NB];
#pragma unroll
  for (int cc = 0; cc < NB; ++cc) acc[cc] = 0.f;
  const int64_t chunks = fmd_cdiv(k, 4);
  for (int64_t ch0 = q; ch0 < chunks; ch0 += 4 * CH) {
    // the pass's chunks all in flight before their arithmetic
    float4 av[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int64_t ch = ch0 + 4 * u;
      const int64_t cl = ch < chunks ? ch : chunks - 1;
      if (VEC) {
        av[u] = *reinterpret_cast<const float4*>(ar + 4 * cl);
      } else {
        float e[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t kk = 4 * cl + t;
          e[t] = ar[kk < k ? kk : k - 1];
        }
        av[u] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int64_t ch = ch0 + 4 * u;
      if (ch >= chunks) break;
      const float e[4] = {av[u].x, av[u].y, av[u].z, av[u].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t kk = 4 * ch + t;
        if (kk >= k) break;
        const float4* brow = reinterpret_cast<const float4*>(bsh + kk * PITCH);
#pragma unroll
        for (int g = 0; g < NQ; ++g) {
          const float4 bq = brow[g];
          acc[4 * g + 0] = __builtin_fmaf(e[t], bq.x, acc[4 * g + 0]);
          acc[4 * g + 1] = __builtin_fmaf(e[t], bq.y, acc[4 * g + 1]);
          acc[4 * g + 2] = __builtin_fmaf(e[t], bq.z, acc[4 * g + 2]);
          acc[4 * g + 3] = __builtin_fmaf(e[t], bq.w, acc[4 * g + 3]);
        }
      }
    }
  }
  // the quad's four partial sums, (q0 + q1) + (q2 + q3) on every lane of the quad
#pragma unroll
  for (int cc = 0; cc < NB; ++cc) {
    acc[cc] += dpp_read<kDppQuadXor1>(acc[cc]);
    acc[cc] += dpp_read<kDppQuadXor2>(acc[cc]);
  }
  if (r >= m) return;
  float* dst = c + r * ldc;
#pragma unroll
  for (int cc = 0; cc < NB; ++cc)
    if (cc % 4 == q && cc < n) dst[cc] = thin_finish(acc[cc], bias ? bias[cc] : 0.f, dst + cc, accumulate, act);
}

}  // namespace

// Launches for fmd_gemm_f32: FMD_EUNSUPPORTED when the shape is not thin.
__attribute__((visibility("hidden"))) int launch_gemm_thin(const float* a, int64_t lda, const float* b, int64_t ldb, int32_t b_layout, const float* bias,
                     float* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t act,
                     hipStream_t stream) {
  if (m <= 0 || n <= 0 || k <= 0) return FMD_EUNSUPPORTED;
  if (k <= kThinMaxK && n <= 256) {
    const unsigned grid = (unsigned)fmd_cdiv(m, 4 * kThinRows);
    const int nj = (int)fmd_cdiv(n, 64), kb = (int)fmd_cdiv(k, 4);
#define THIN_K(NJ, KB)                                                                                          \
  hipLaunchKernelGGL((gemm_thin_k_kernel<NJ, KB>), dim3(grid), dim3(256), 0, stream, a, lda, b, ldb, b_layout,   \
                     bias, c, ldc, m, n, (int)k, accumulate, act)
#define THIN_K_B(NJ)      \
  do {                    \
    if (kb == 1)          \
      THIN_K(NJ, 4);      \
    else if (kb == 2)     \
      THIN_K(NJ, 8);      \
    else if (kb == 3)     \
      THIN_K(NJ, 12);     \
    else                  \
      THIN_K(NJ, 16);     \
  } while (0)
    if (nj == 1)
      THIN_K_B(1);
    else if (nj == 2)
      THIN_K_B(2);
    else if (nj == 3)
      THIN_K_B(3);
    else
      THIN_K_B(4);
#undef THIN_K_B
#undef THIN_K
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  const int nq = (int)fmd_cdiv(n, 4);
  const int64_t pitch = nq == 1 ? 4 : 20;
  if (n <= kThinMaxN && k * pitch <= kThinNLds) {
    const unsigned grid = (unsigned)fmd_cdiv(m, 64);
    const size_t lds = (size_t)k * pitch * sizeof(float);
    const bool vec = k % 4 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
    const bool short_k = k <= 64;  // four chunks per lane cover the row
#define THIN_N(NQ, CH, V)                                                                                        \
  hipLaunchKernelGGL((gemm_thin_n_kernel<NQ, CH, V>), dim3(grid), dim3(256), lds, stream, a, lda, b, ldb,        \
                     b_layout, bias, c, ldc, m, n, k, accumulate, act)
#define THIN_N_Q(NQ)           \
  do {                         \
    if (short_k && vec)        \
      THIN_N(NQ, 4, true);     \
    else if (short_k)          \
      THIN_N(NQ, 4, false);    \
    else if (vec)              \
      THIN_N(NQ, 16, true);    \
    else                       \
      THIN_N(NQ, 16, false);   \
  } while (0)
    if (nq == 1)
      THIN_N_Q(1);
    else if (nq == 2)
      THIN_N_Q(2);
    else if (nq == 3)
      THIN_N_Q(3);
    else
      THIN_N_Q(4);
#undef THIN_N_Q
#undef THIN_N
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  return FMD_EUNSUPPORTED;
}
