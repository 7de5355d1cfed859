// (b) gather-cat and (c) deterministic CSR segment sums (+ transpose), fp32, HBM-bound.
//
// Layout: row-major matrices with a row stride; a wavefront owns a row (gather-cat) or a
// segment (segment sum) and its lanes cover the columns in float4 units when every operand
// is 16-byte aligned with a stride and width divisible by 4 (host checked), else in floats.
// No float atomics anywhere: a segment's rows are added in the order of its CSR run, split
// over a fixed number of lane groups that are combined in a fixed order at the end, so the
// result is a function of the CSR only (bitwise reproducible run to run).
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxParts = 4;
constexpr int kMaxTerms = 2;

struct CatParts {
  const float* src[kMaxParts];
  const int32_t* idx[kMaxParts];
  int64_t istride[kMaxParts];
  int64_t ld[kMaxParts];
  int32_t width[kMaxParts];  // in VEC units
  int32_t start[kMaxParts + 1];
  int32_t n;
};

template <int VEC>
struct VecT;
template <>
struct VecT<1> {
  using T = float;
  __device__ static T zero() { return 0.f; }
  __device__ static void add(T& a, T b) { a = a + b; }
  __device__ static T mul(T a, T b) { return a * b; }
  __device__ static T scale(T a, float s) { return a * s; }
};
template <>
struct VecT<4> {
  using T = float4;
  __device__ static T zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ static void add(T& a, T b) {
    a.x = a.x + b.x;
    a.y = a.y + b.y;
    a.z = a.z + b.z;
    a.w = a.w + b.w;
  }
  __device__ static T mul(T a, T b) { return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w); }
  __device__ static T scale(T a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
};

// out[e, :] = cat(parts) over tiles of RPW rows per wave. A wave first stages the gathered row
// numbers of its tile in LDS (one coalesced index load per part), then walks the tile's
// RPW x total output units as one flat range: unit u = it * 64 + lane is (row u / total, column
// u % total), so every lane stores on every pass and consecutive lanes store consecutive
// 16-byte units (full-width coalesced stores, no idle lanes at the end of a row). U passes are
// issued before their stores so each lane keeps U loads in flight; the stores are streaming.
template <int VEC, int RPW>
__global__ void __launch_bounds__(kThreads) gather_cat_kernel(CatParts p, int64_t rows, float* out, int64_t ld_out) {
  using V = typename VecT<VEC>::T;
  constexpr int U = 4;
  constexpr int kWaves = kThreads / FMD_WAVE;
  __shared__ int32_t s_idx[kWaves][kMaxParts][RPW];
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const int w = threadIdx.x / FMD_WAVE;
  const int total = p.start[p.n];
  // advance of (row, column) per pass of 64 units
  const int q = FMD_WAVE / total, rem = FMD_WAVE % total;
  const int64_t ntiles = (rows + RPW - 1) / RPW;
  for (int64_t tile = (int64_t)blockIdx.x * kWaves + w; tile < ntiles; tile += (int64_t)gridDim.x * kWaves) {
    const int64_t e0 = tile * RPW;
    const int nrow = (int)((rows - e0) < RPW ? (rows - e0) : RPW);
    for (int l = lane; l < RPW; l += FMD_WAVE) {
#pragma unroll
      for (int k = 0; k < kMaxParts; ++k) {
        int32_t v = 0;
        if (k < p.n && l < nrow) v = p.idx[k] ? p.idx[k][(e0 + l) * p.istride[k]] : (int32_t)(e0 + l);
        s_idx[w][k][l] = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int T = nrow * total;
    int r = lane / total, c = lane % total;
    for (int base = 0; base < T; base += FMD_WAVE * U) {
      V val[U];
      int rr[U], cc[U];
#pragma unroll
      for (int j = 0; j < U; ++j) {
        rr[j] = r;
        cc[j] = c;
        if (base + j * FMD_WAVE + lane < T) {
          int k = 0;
#pragma unroll
          for (int m = 1; m < kMaxParts; ++m) k += (m < p.n && c >= p.start[m]) ? 1 : 0;
          const int64_t srow = s_idx[w][k][r];
          val[j] = reinterpret_cast<const V*>(p.src[k] + srow * p.ld[k])[c - p.start[k]];
        }
        r += q;
        c += rem;
        if (c >= total) {
          c -= total;
          r += 1;
        }
      }
#pragma unroll
      for (int j = 0; j < U; ++j)
        if (base + j * FMD_WAVE + lane < T) store_stream(reinterpret_cast<V*>(out + (e0 + rr[j]) * ld_out) + cc[j], val[j]);
    }
    __builtin_amdgcn_wave_barrier();  // s_idx is rewritten for the next tile
  }
}

struct SegTerms {
  const float* v[kMaxTerms];
  const float* w[kMaxTerms];
  const int32_t* perm[kMaxTerms];
  const int64_t* off[kMaxTerms];
  int64_t ld[kMaxTerms];
  int64_t col[kMaxTerms];
  int64_t rows[kMaxTerms];
  float scale[kMaxTerms];
  int32_t n;
};

// out[s, tile] = sum_t sum_{j in run_t(s)} [w] v[r_j, col_t + tile]. One wave per (segment,
// column tile of 64*VEC floats). When the tile is narrower than 64 lanes, R = 64 / lpr lane
// groups take rows j = run_start + g, + R, ... and are combined in slot order at the end.
template <int VEC>
__global__ void __launch_bounds__(kThreads) segsum_kernel(SegTerms t, int64_t num_segment, int64_t dimv,
                                                          int64_t skip, int accumulate, float* out, int64_t ld_out,
                                                          int lpr) {
  using V = typename VecT<VEC>::T;
  using Op = VecT<VEC>;
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const int64_t s = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / FMD_WAVE;
  if (s >= num_segment) return;
  const int64_t c = (int64_t)blockIdx.y * FMD_WAVE + (lane % lpr);
  const int g = lane / lpr, R = FMD_WAVE / lpr;
  const bool live = c < dimv && ((int64_t)blockIdx.y * FMD_WAVE + lpr > c);
  V acc = Op::zero();
  if (s != skip && live) {
    for (int k = 0; k < t.n; ++k) {
      int64_t lo = t.off[k][s], hi = t.off[k][s + 1];
      hi = hi < t.rows[k] ? hi : t.rows[k];
      lo = lo < hi ? lo : hi;
      const float* base = t.v[k] + t.col[k];
      const float* wb = t.w[k] ? t.w[k] + t.col[k] : nullptr;
      const float sc = t.scale[k];
      V part = Op::zero();
      // four rows of the group's run loaded before they are added (in run order, so the sum is
      // the same as a row-by-row loop; a missing row adds +0, which leaves the +0-started sum
      // unchanged bit for bit)
      for (int64_t j = lo + g; j < hi; j += 4 * R) {
        V val[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t jj = j + (int64_t)i * R;
          val[i] = Op::zero();
          if (jj < hi) {
            const int64_t r = t.perm[k] ? (int64_t)t.perm[k][jj] : jj;
            if (r >= 0) {
              val[i] = reinterpret_cast<const V*>(base + r * t.ld[k])[c];
              if (wb) val[i] = Op::mul(val[i], reinterpret_cast<const V*>(wb + r * t.ld[k])[c]);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) Op::add(part, val[i]);
      }
      Op::add(acc, sc == 1.0f ? part : Op::scale(part, sc));
    }
  }
  // combine the R lane groups in fixed order: groups 0..R-1 of the same column
  for (int step = 1; step < R; step <<= 1) {
    V o;
    if constexpr (VEC == 4) {
      o.x = __shfl_down(acc.x, step * lpr, FMD_WAVE);
      o.y = __shfl_down(acc.y, step * lpr, FMD_WAVE);
      o.z = __shfl_down(acc.z, step * lpr, FMD_WAVE);
      o.w = __shfl_down(acc.w, step * lpr, FMD_WAVE);
    } else {
      o = __shfl_down(acc, step * lpr, FMD_WAVE);
    }
    if ((g % (2 * step)) == 0 && g + step < R) Op::add(acc, o);
  }
  if (g == 0 && live) {
    V* dst = reinterpret_cast<V*>(out + s * ld_out) + c;
    if (accumulate && s != skip) {
      V cur = *dst;
      Op::add(cur, acc);
      *dst = cur;
    } else {
      *dst = acc;
    }
  }
}

// Transpose of one CSR term: gv[r] = gout[s] (* w[r]), gw[r] = gout[s] * v[r] for r in run(s).
template <int VEC>
__global__ void __launch_bounds__(kThreads) segsum_t_kernel(const float* gout, int64_t ld_gout, const float* value,
                                                            const float* weight, int64_t ld_value,
                                                            const int32_t* perm, const int64_t* off,
                                                            int64_t num_segment, int64_t n_rows, int64_t dimv,
                                                            int64_t skip, float* gv, float* gw, int lpr) {
  using V = typename VecT<VEC>::T;
  using Op = VecT<VEC>;
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  const int64_t s = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / FMD_WAVE;
  if (s >= num_segment) return;
  const int64_t c = (int64_t)blockIdx.y * FMD_WAVE + (lane % lpr);
  const int g = lane / lpr, R = FMD_WAVE / lpr;
  if (!(c < dimv && ((int64_t)blockIdx.y * FMD_WAVE + lpr > c))) return;
  int64_t lo = off[s], hi = off[s + 1];
  hi = hi < n_rows ? hi : n_rows;
  lo = lo < hi ? lo : hi;
  const V go = (s == skip) ? Op::zero() : reinterpret_cast<const V*>(gout + s * ld_gout)[c];
  for (int64_t j = lo + g; j < hi; j += R) {
    const int64_t r = perm ? (int64_t)perm[j] : j;
    if (r < 0) continue;
    if (gv) {
      V val = go;
      if (weight) val = Op::mul(val, reinterpret_cast<const V*>(weight + r * ld_value)[c]);
      store_stream(reinterpret_cast<V*>(gv + r * dimv * VEC) + c, val);
    }
    if (gw)
      store_stream(reinterpret_cast<V*>(gw + r * dimv * VEC) + c,
                   Op::mul(go, reinterpret_cast<const V*>(value + r * ld_value)[c]));
  }
}

// Rows [first, n_rows) of gv/gw (contiguous, width dim) set to 0: the rows no run covers.
__global__ void zero_rows_kernel(float* a, float* b, const int64_t* first_ptr, int64_t n_rows, int64_t dim) {
  const int64_t first = first_ptr ? (first_ptr[0] < n_rows ? first_ptr[0] : n_rows) : 0;
  const int64_t total = (n_rows - first) * dim;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (int64_t)gridDim.x * blockDim.x) {
    if (a) a[first * dim + k] = 0.f;
    if (b) b[first * dim + k] = 0.f;
  }
}

// Fixed-order FP64 sum in one workgroup: per-thread strided sums, then a tree over threads.
template <typename T>
__global__ void __launch_bounds__(1024) sum_f64_kernel(const T* x, int64_t n, double* out) {
  __shared__ double part[1024];
  // the same adds in the same order; eight loads in flight before their adds
  constexpr int kU = 8;
  const int64_t step = blockDim.x;
  double s = 0.0;
  int64_t k = threadIdx.x;
  for (; k + (kU - 1) * step < n; k += kU * step) {
    T t[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) t[u] = x[k + u * step];
#pragma unroll
    for (int u = 0; u < kU; ++u) s = s + (double)t[u];
  }
  for (; k < n; k += step) s = s + (double)x[k];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int width = blockDim.x / 2; width > 0; width >>= 1) {
    if ((int)threadIdx.x < width) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + width];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = part[0];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int lanes_per_row(int64_t dimv) {
  int lpr = 1;
  while (lpr < dimv && lpr < FMD_WAVE) lpr <<= 1;
  return lpr;
}

}  // namespace

extern "C" {

int fmd_gather_cat_f32(int32_t n_parts, const float* const* srcs, const int32_t* const* indices,
                       const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t rows,
                       float* out, int64_t ld_out, hipStream_t stream) {
  FMD_REQUIRE(n_parts >= 1 && n_parts <= kMaxParts && rows >= 0 && out && srcs && lds && widths);
  if (rows == 0) return FMD_OK;
  bool vec = aligned16(out) && ld_out % 4 == 0;
  int64_t total = 0;
  for (int k = 0; k < n_parts; ++k) {
    FMD_REQUIRE(srcs[k] && widths[k] >= 0 && lds[k] >= 0);
    vec = vec && aligned16(srcs[k]) && lds[k] % 4 == 0 && widths[k] % 4 == 0;
    total += widths[k];
  }
  FMD_REQUIRE(total <= ld_out);
  CatParts p{};
  p.n = n_parts;
  const int div = vec ? 4 : 1;
  p.start[0] = 0;
  for (int k = 0; k < n_parts; ++k) {
    p.src[k] = srcs[k];
    p.idx[k] = indices ? indices[k] : nullptr;
    p.istride[k] = index_strides ? index_strides[k] : 1;
    FMD_REQUIRE(p.istride[k] >= 1);
    p.ld[k] = lds[k];
    p.width[k] = widths[k] / div;
    p.start[k + 1] = p.start[k] + p.width[k];
  }
  for (int k = n_parts; k < kMaxParts; ++k) p.start[k + 1] = p.start[n_parts];
  if (p.start[n_parts] == 0) return FMD_OK;
  constexpr int kRpw = 16;
  int64_t blocks = fmd_cdiv(fmd_cdiv(rows, kRpw), kThreads / FMD_WAVE);
  blocks = blocks > (1 << 20) ? (1 << 20) : blocks;
  if (vec)
    hipLaunchKernelGGL((gather_cat_kernel<4, kRpw>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, p, rows, out,
                       ld_out);
  else
    hipLaunchKernelGGL((gather_cat_kernel<1, kRpw>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, p, rows, out,
                       ld_out);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_segsum_csr_f32(int32_t n_terms, const float* const* values, const int64_t* ld_values,
                       const int64_t* col_offsets, const float* const* weights, const float* scales,
                       const int32_t* const* perms, const int64_t* const* offs, const int64_t* rows,
                       int64_t num_segment, int64_t dim,
                       int64_t skip_segment, int32_t accumulate, float* out, int64_t ld_out, hipStream_t stream) {
  FMD_REQUIRE(n_terms >= 0 && n_terms <= kMaxTerms && num_segment >= 0 && dim >= 0 && out);
  FMD_REQUIRE(ld_out >= dim);
  if (num_segment == 0 || dim == 0) return FMD_OK;
  SegTerms t{};
  t.n = n_terms;
  bool vec = aligned16(out) && ld_out % 4 == 0 && dim % 4 == 0;
  for (int k = 0; k < n_terms; ++k) {
    FMD_REQUIRE(values[k] && offs[k] && rows[k] >= 0 && ld_values[k] >= 0 && col_offsets[k] >= 0);
    t.v[k] = values[k];
    t.w[k] = weights ? weights[k] : nullptr;
    t.perm[k] = perms ? perms[k] : nullptr;
    t.off[k] = offs[k];
    t.ld[k] = ld_values[k];
    t.col[k] = col_offsets[k];
    t.rows[k] = rows[k];
    t.scale[k] = scales ? scales[k] : 1.0f;
    vec = vec && aligned16(values[k]) && ld_values[k] % 4 == 0 && col_offsets[k] % 4 == 0;
    if (t.w[k]) vec = vec && aligned16(t.w[k]);
  }
  const int div = vec ? 4 : 1;
  const int64_t dimv = dim / div;
  const int lpr = lanes_per_row(dimv);
  dim3 grid((unsigned)fmd_cdiv(num_segment, kThreads / FMD_WAVE), (unsigned)fmd_cdiv(dimv, FMD_WAVE));
  if (vec)
    hipLaunchKernelGGL(segsum_kernel<4>, grid, dim3(kThreads), 0, stream, t, num_segment, dimv, skip_segment,
                       accumulate, out, ld_out, lpr);
  else
    hipLaunchKernelGGL(segsum_kernel<1>, grid, dim3(kThreads), 0, stream, t, num_segment, dimv, skip_segment,
                       accumulate, out, ld_out, lpr);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_segsum_csr_t_f32(const float* gout, int64_t ld_gout, const float* value, const float* weight, int64_t ld_value,
                         const int32_t* perm, const int64_t* off, int64_t num_segment, int64_t n_rows, int64_t dim,
                         int64_t skip_segment, float* gvalue, float* gweight, hipStream_t stream) {
  FMD_REQUIRE(gout && off && num_segment >= 0 && n_rows >= 0 && dim >= 0);
  FMD_REQUIRE(gvalue || gweight);
  FMD_REQUIRE(!gweight || value);
  if (n_rows == 0 || dim == 0) return FMD_OK;
  // rows no run covers: identity CSR -> the rows past off[num_segment]; a permutation CSR
  // covers every row by contract, but its rows are zeroed first anyway (cheap, and safe)
  {
    int64_t blocks = fmd_cdiv(n_rows * dim, 256);
    blocks = blocks > 4096 ? 4096 : blocks;
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, gvalue, gweight,
                       perm ? (const int64_t*)nullptr : off + num_segment, n_rows, dim);
    FMD_CHECK_LAUNCH();
  }
  if (num_segment == 0) return FMD_OK;
  bool vec = aligned16(gout) && ld_gout % 4 == 0 && dim % 4 == 0 && (!gvalue || aligned16(gvalue)) &&
             (!gweight || aligned16(gweight));
  if (value) vec = vec && aligned16(value) && ld_value % 4 == 0;
  if (weight) vec = vec && aligned16(weight);
  const int div = vec ? 4 : 1;
  const int64_t dimv = dim / div;
  const int lpr = lanes_per_row(dimv);
  dim3 grid((unsigned)fmd_cdiv(num_segment, kThreads / FMD_WAVE), (unsigned)fmd_cdiv(dimv, FMD_WAVE));
  if (vec)
    hipLaunchKernelGGL(segsum_t_kernel<4>, grid, dim3(kThreads), 0, stream, gout, ld_gout, value, weight, ld_value, perm,
                       off, num_segment, n_rows, dimv, skip_segment, gvalue, gweight, lpr);
  else
    hipLaunchKernelGGL(segsum_t_kernel<1>, grid, dim3(kThreads), 0, stream, gout, ld_gout, value, weight, ld_value, perm,
                       off, num_segment, n_rows, dimv, skip_segment, gvalue, gweight, lpr);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_sum_f64(const void* x, int32_t x_is_f64, int64_t n, double* out, hipStream_t stream) {
  FMD_REQUIRE(x && out && n >= 0);
  if (x_is_f64)
    hipLaunchKernelGGL(sum_f64_kernel<double>, dim3(1), dim3(1024), 0, stream, static_cast<const double*>(x), n, out);
  else
    hipLaunchKernelGGL(sum_f64_kernel<float>, dim3(1), dim3(1024), 0, stream, static_cast<const float*>(x), n, out);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
