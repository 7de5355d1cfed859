// Three-body line graph of the fixed-capacity builder: undirected pairs of the directed edge rows,
// the short-bond lists per atom and the triplet rows (fixed_capacity_builder.py:2001-2161, the
// torch steps of _materialize_pairs / _materialize_line_graph and _line_graph_kernel :680-753).
// Integer work, bit-exact with the reference's rules on the same rows:
//   pair leader: a real row e whose reverse row r exists and e <= r; the pair id of e is the
//     number of leaders up to min(e, r), minus one (d2u); u2d[u] = the leader row of pair u;
//     padding rows / pairs follow the far self-loop rule (pair u >= real_u is the rows
//     ec + 2 (u - real_u) and ec + 2 (u - real_u) + 1); invalid_pairs = odd edge count, a leader
//     count other than half the edges, or a real row without a reverse row
//   short lists: the rows of atom i with the short-bond flag, in row order, in
//     short_edge_matrix[i, 0..s_i) (the rest e_cap); pair_offsets = exclusive scan of s (s - 1)
//   overflow = edges >= e_cap | triplets > t_cap | invalid_pairs | !candidate_valid
//   triplet row t (< min(triplets, t_cap)): atom a = the last atom with pair_offsets[a] <= t,
//     local = t - pair_offsets[a], first = local / (s_a - 1), second = local % (s_a - 1) skipping
//     first; (a, d2u[row1], row1, d2u[row2], row2) with row = short_edge_matrix[a, .]; padding
//     triplets use padding pair real_u + (t - t_real) % (u_cap - real_u) on atom pair % n;
//     on overflow every triplet is the all-loop topology (u = t u_cap / t_cap, row 2 u, atom u % n)
//     and d2u / u2d are the all-loop pairs (e / 2, 2 u).
//   Sink padding (n_dummy > 0): a padding triplet sits on sink n + pad_id n_dummy / (t_cap - t_real)
//     and the overflow topology is all-sink (u = ceil(d u_cap / n_dummy) for d = t n_dummy / t_cap,
//     atom n + u n_dummy / u_cap); fmd_nl_overflow_rows writes the matching edge rows.
// The scans are multi-block (block sums, one workgroup over the blocks, block-local scans):
// deterministic, no atomics.
#include "common.h"

namespace {

constexpr int kLgBlock = 1024;

__device__ __forceinline__ int64_t real_rows_of(const int64_t* edge_offsets, int64_t n, int64_t e_cap) {
  const int64_t t = edge_offsets[n];
  return t < e_cap ? t : e_cap;
}

// wave-wide inclusive scan of one int64 per lane (six shuffle steps)
__device__ __forceinline__ int64_t wave_inclusive_scan(int64_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t u = __shfl_up(v, off, 64);
    v += lane >= off ? u : 0;
  }
  return v;
}

// block-wide inclusive scan of one int64 per thread (1024 threads): scans within the waves, the
// wave totals through LDS (sh: at least 16 entries), two barriers; integer sums, so the result is
// the serial prefix whatever the order. `total` (optional): the block's sum.
__device__ __forceinline__ int64_t block_inclusive_scan(int64_t v, int64_t* sh, int64_t* total = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_inclusive_scan(v);
  if (lane == 63) sh[wave] = v;
  __syncthreads();
  int64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kLgBlock / 64; ++w) {
    const int64_t t = sh[w];
    before += w < wave ? t : 0;
    all += t;
  }
  if (total) *total = all;
  __syncthreads();
  return before + v;
}

__device__ __forceinline__ void leader_of(const int32_t* reverse, int64_t e, int64_t ec, bool& leader, bool& unmatched,
                                          int64_t& canon) {
  const bool real = e < ec;
  const int64_t r = real ? (int64_t)reverse[e] : -1;
  const bool matched = real && r >= 0;
  leader = matched && e <= r;
  unmatched = real && !matched;
  canon = matched && r < e ? r : e;
}

// K1: per block of rows, the leader and unmatched counts -> work[b], work[nb + b]
__global__ void __launch_bounds__(kLgBlock) lg_leader_count_kernel(const int32_t* reverse, const int64_t* edge_offsets,
                                                                    int64_t n, int64_t e_cap, int64_t nb,
                                                                    int64_t* work) {
  __shared__ int64_t sh[kLgBlock / 64];
  const int64_t e = (int64_t)blockIdx.x * kLgBlock + threadIdx.x;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  bool leader, unmatched;
  int64_t canon;
  leader_of(reverse, e, ec, leader, unmatched, canon);
  const int64_t packed = (leader ? 1 : 0) + (unmatched ? (int64_t(1) << 32) : 0);
  const int64_t tot = block_inclusive_scan(packed, sh);
  if (threadIdx.x == kLgBlock - 1) {
    work[blockIdx.x] = tot & 0xffffffffLL;
    work[nb + blockIdx.x] = tot >> 32;
  }
}

// K2: one workgroup: exclusive scan of the block leader counts (in place), the invalid-pairs flag
__global__ void __launch_bounds__(kLgBlock) lg_leader_scan_kernel(const int64_t* edge_offsets, int64_t n, int64_t nb,
                                                                   int64_t* work, uint8_t* invalid_pairs) {
  __shared__ int64_t sh[kLgBlock / 64];
  __shared__ int64_t chunk;
  int64_t carry = 0, unmatched = 0;
  for (int64_t base = 0; base < nb; base += kLgBlock) {
    const int64_t b = base + threadIdx.x;
    const int64_t v = b < nb ? work[b] : 0;
    unmatched += b < nb ? work[nb + b] : 0;
    const int64_t inc = block_inclusive_scan(v, sh);
    if (b < nb) work[b] = carry + inc - v;
    if (threadIdx.x == kLgBlock - 1) chunk = inc;  // the chunk's total
    __syncthreads();
    carry += chunk;
    __syncthreads();
  }
  const int64_t um = block_inclusive_scan(unmatched, sh);
  if (threadIdx.x == kLgBlock - 1) {
    const int64_t total = edge_offsets[n];
    work[2 * nb] = carry;  // number of leaders
    invalid_pairs[0] = (total % 2 != 0) || (carry != total / 2) || (um > 0) ? 1 : 0;
  }
}

// K3: per block: the inclusive leader prefix of every row -> pfx[e] (int64)
__global__ void __launch_bounds__(kLgBlock) lg_leader_apply_kernel(const int32_t* reverse, const int64_t* edge_offsets,
                                                                    int64_t n, int64_t e_cap, const int64_t* work,
                                                                    int64_t* pfx) {
  __shared__ int64_t sh[kLgBlock / 64];
  const int64_t e = (int64_t)blockIdx.x * kLgBlock + threadIdx.x;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  bool leader, unmatched;
  int64_t canon;
  leader_of(reverse, e, ec, leader, unmatched, canon);
  const int64_t inc = block_inclusive_scan(leader ? 1 : 0, sh);
  if (e < e_cap) pfx[e] = work[blockIdx.x] + inc;
}

// K4: one wave per atom: its short rows in row order, their count
__global__ void __launch_bounds__(256) lg_short_kernel(const uint8_t* short_flags, const int64_t* edge_offsets,
                                                       int64_t n, int64_t e_cap, int32_t bmax, int64_t* short_counts,
                                                       int32_t* sem, int32_t* short_rank) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  if (i >= n) return;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  int64_t lo = edge_offsets[i], hi = edge_offsets[i + 1];
  hi = hi < ec ? hi : ec;
  lo = lo < hi ? lo : hi;
  int64_t s = 0;
  int32_t* row = sem + i * bmax;
  for (int64_t base = lo; base < hi; base += 64) {
    const int64_t e = base + lane;
    const bool f = e < hi && short_flags[e] != 0;
    const uint64_t mask = __ballot(f);
    const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
    if (f && s + rank < bmax) row[s + rank] = (int32_t)e;
    if (e < hi) short_rank[e] = (int32_t)(s + rank);  // short rows of the atom before e
    s += __popcll(mask);
  }
  for (int64_t k = (s < bmax ? s : bmax) + lane; k < bmax; k += 64) row[k] = (int32_t)e_cap;
  if (lane == 0) short_counts[i] = s;
}

// K5: one workgroup: exclusive scans of s and s (s - 1) over the atoms, the overflow flag. Each
// thread takes kPairsPer consecutive atoms per pass (their loads in flight together), the block
// scans the per-thread sums.
constexpr int kPairsPer = 8;

__global__ void __launch_bounds__(kLgBlock) lg_pairs_scan_kernel(const int64_t* short_counts, const int64_t* edge_offsets,
                                                                  const uint8_t* invalid_pairs,
                                                                  const uint8_t* candidate_valid, int64_t n,
                                                                  int64_t e_cap, int64_t t_cap, int64_t* short_offsets,
                                                                  int64_t* pair_offsets, uint8_t* overflow) {
  __shared__ int64_t sh[2][kLgBlock / 64];
  int64_t carry_s = 0, carry_p = 0;
  for (int64_t base = 0; base < n; base += (int64_t)kLgBlock * kPairsPer) {
    const int64_t i0 = base + (int64_t)threadIdx.x * kPairsPer;
    int64_t sv[kPairsPer], ts = 0, tp = 0;
#pragma unroll
    for (int k = 0; k < kPairsPer; ++k) sv[k] = i0 + k < n ? short_counts[i0 + k] : 0;
#pragma unroll
    for (int k = 0; k < kPairsPer; ++k) {
      ts += sv[k];
      tp += sv[k] * (sv[k] - 1);
    }
    int64_t tot_s, tot_p;
    int64_t ex_s = carry_s + block_inclusive_scan(ts, sh[0], &tot_s) - ts;
    int64_t ex_p = carry_p + block_inclusive_scan(tp, sh[1], &tot_p) - tp;
#pragma unroll
    for (int k = 0; k < kPairsPer; ++k)
      if (i0 + k < n) {
        short_offsets[i0 + k] = ex_s;
        pair_offsets[i0 + k] = ex_p;
        ex_s += sv[k];
        ex_p += sv[k] * (sv[k] - 1);
      }
    carry_s += tot_s;
    carry_p += tot_p;
  }
  if (threadIdx.x == 0) {
    short_offsets[n] = carry_s;
    pair_offsets[n] = carry_p;
    const int64_t total = edge_offsets[n];
    overflow[0] = (total >= e_cap) || (carry_p > t_cap) || invalid_pairs[0] || !candidate_valid[0] ? 1 : 0;
  }
}

// K6: d2u per row and u2d per pair (written by the pair's leader row, padding pairs by index)
__global__ void lg_pairs_index_kernel(const int32_t* reverse, const int64_t* edge_offsets, const int64_t* pfx,
                                      const uint8_t* overflow, int64_t n, int64_t e_cap, int64_t u_cap, int32_t* d2u,
                                      int32_t* u2d) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool ovf = overflow[0] != 0;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  const int64_t real_u = ec / 2;
  if (k < e_cap) {
    const int64_t e = k;
    bool leader, unmatched;
    int64_t canon;
    leader_of(reverse, e, ec, leader, unmatched, canon);
    int64_t u;
    if (ovf) {
      u = e / 2;
    } else if (e < ec) {
      u = pfx[canon] - 1;
    } else {
      u = real_u + (e - ec) / 2;
    }
    u = u < 0 ? 0 : (u > u_cap - 1 ? u_cap - 1 : u);
    d2u[e] = (int32_t)u;
    if (!ovf && leader) {
      const int64_t id = pfx[e] - 1;
      if (id >= 0 && id < u_cap) u2d[id] = (int32_t)(e < e_cap - 1 ? e : e_cap - 1);
    }
  }
  if (k < u_cap) {
    int64_t v = -1;
    if (ovf)
      v = 2 * k;
    else if (k >= real_u)
      v = ec + 2 * (k - real_u);
    if (v >= 0) u2d[k] = (int32_t)(v < e_cap - 1 ? v : e_cap - 1);
  }
}

// K8: the angle -> bond CSR over the directed rows (row e's triplets as first bond:
// [off[e], off[e + 1]) = pair_offsets[i] + rank_e (s_i - 1) + [0, s_i - 1) for a short row, empty
// otherwise; padding rows empty at the end; clamped to t_cap) and the compact short-bond rows
// (bond_rows[short_offsets[i] + rank_e] = e, the rest -1)
__global__ void lg_edge_offsets_kernel(const int32_t* center, const uint8_t* short_flags, const int32_t* short_rank,
                                       const int64_t* short_counts, const int64_t* short_offsets,
                                       const int64_t* pair_offsets, const int64_t* edge_offsets, int64_t n,
                                       int64_t e_cap, int64_t t_cap, int64_t* edge_tri_off, int32_t* bond_rows) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e > e_cap) return;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  int64_t o;
  if (e < ec) {
    const int64_t i = center[e];
    const int64_t sc = short_counts[i];
    o = pair_offsets[i] + (int64_t)short_rank[e] * (sc > 0 ? sc - 1 : 0);
  } else {
    o = pair_offsets[n];
  }
  edge_tri_off[e] = o < t_cap ? o : t_cap;
  if (e < e_cap) {
    const int64_t nshort = short_offsets[n];
    if (e < ec && short_flags[e]) {
      const int64_t b = short_offsets[center[e]] + short_rank[e];
      if (b < e_cap) bond_rows[b] = (int32_t)e;
    }
    if (e >= nshort) bond_rows[e] = -1;
  }
}

// K7: the triplet rows
__global__ void lg_line_graph_kernel(const int64_t* pair_offsets, const int64_t* short_counts, const int32_t* sem,
                                     const int32_t* d2u, const int64_t* edge_offsets, const uint8_t* overflow,
                                     int64_t n, int64_t e_cap, int64_t u_cap, int64_t t_cap, int32_t bmax,
                                     int32_t n_dummy, int32_t* line_graph, int32_t* second_perm) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= t_cap) return;
  int32_t* out = line_graph + t * 5;
  // the second-bond CSR: its entries past the real triplets (and all of an overflowed build's) are
  // -1; a real triplet's own entry is written below
  const int64_t total_all = pair_offsets[n];
  if (overflow[0] || t >= (total_all < t_cap ? total_all : t_cap)) second_perm[t] = -1;
  if (overflow[0]) {
    int64_t u;
    if (n_dummy > 0) {
      const int64_t d = t * n_dummy / t_cap;
      u = (d * u_cap + n_dummy - 1) / n_dummy;
    } else {
      u = t * u_cap / t_cap;
    }
    u = u < u_cap - 1 ? u : u_cap - 1;
    const int32_t atom = (int32_t)(n_dummy > 0 ? n + u * n_dummy / u_cap : u % n);
    out[0] = atom;
    out[1] = (int32_t)u;
    out[2] = (int32_t)(2 * u);
    out[3] = (int32_t)u;
    out[4] = (int32_t)(2 * u);
    return;
  }
  const int64_t total_t = pair_offsets[n];
  const int64_t t_real = total_t < t_cap ? total_t : t_cap;
  const int64_t ec = real_rows_of(edge_offsets, n, e_cap);
  if (t < t_real) {
    // the last atom with pair_offsets[atom] <= t
    int64_t lo = 0, hi = n;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (pair_offsets[mid] <= t)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int64_t atom = lo < n - 1 ? lo : n - 1;
    const int64_t local = t - pair_offsets[atom];
    int64_t denom = short_counts[atom] - 1;
    denom = denom > 1 ? denom : 1;
    const int64_t first = local / denom;
    const int64_t second_raw = local - first * denom;
    const int64_t second = second_raw + (second_raw >= first ? 1 : 0);
    const int64_t de1 = sem[atom * bmax + (first < bmax - 1 ? first : bmax - 1)];
    const int64_t de2 = sem[atom * bmax + (second < bmax - 1 ? second : bmax - 1)];
    const int64_t c1 = de1 < 0 ? 0 : (de1 > e_cap - 1 ? e_cap - 1 : de1);
    const int64_t c2 = de2 < 0 ? 0 : (de2 > e_cap - 1 ? e_cap - 1 : de2);
    out[0] = (int32_t)atom;
    out[1] = d2u[c1];
    out[2] = (int32_t)de1;
    out[3] = d2u[c2];
    out[4] = (int32_t)de2;
    // triplets with bond (atom, second) as their second bond, by first bond: slot first (or
    // first - 1 past the bond itself) of that bond's run pair_offsets + second (s - 1)
    second_perm[pair_offsets[atom] + second * denom + (first < second ? first : first - 1)] = (int32_t)t;
  } else {
    const int64_t real_u = ec / 2;
    const int64_t pad_id = t - t_real;
    const int64_t free_u = u_cap - real_u > 1 ? u_cap - real_u : 1;
    const int64_t pad_pair = pad_id % free_u;
    const int32_t pu = (int32_t)(real_u + pad_pair), pde = (int32_t)(ec + 2 * pad_pair);
    if (n_dummy > 0) {
      const int64_t free_t = t_cap - t_real > 1 ? t_cap - t_real : 1;
      out[0] = (int32_t)(n + pad_id * n_dummy / free_t);
    } else {
      out[0] = (int32_t)(pad_pair % n);
    }
    out[1] = pu;
    out[2] = pde;
    out[3] = pu;
    out[4] = pde;
  }
}

// The all-padding edge rows of an overflowed line-graph build (_allocate_overflow_topology /
// _substitute_overflow_topology, fixed_capacity_builder.py:1474-1513,2163-2177): row e is a loop
// of pair u = e / 2's atom (u mod n, or sink n + u n_dummy / u_cap) with image +/- the pad image
// (+/- (3, 3, 3) for sinks) for even / odd rows. Rows untouched without overflow.
__global__ void lg_overflow_rows_kernel(const uint8_t* overflow, int64_t n, int64_t e_cap, int32_t n_dummy, int pix,
                                        int piy, int piz, int32_t* center, int32_t* neighbor, int32_t* images,
                                        int32_t* edge_index, float* edge_image) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= e_cap || overflow[0] == 0) return;
  const int64_t u = e / 2, u_cap = e_cap / 2;
  const int32_t atom = (int32_t)(n_dummy > 0 ? n + u * n_dummy / u_cap : u % n);
  const int sign = (e % 2 == 0) ? 1 : -1;
  const int im[3] = {sign * (n_dummy > 0 ? 3 : pix), sign * (n_dummy > 0 ? 3 : piy), sign * (n_dummy > 0 ? 3 : piz)};
  center[e] = atom;
  neighbor[e] = atom;
#pragma unroll
  for (int k = 0; k < 3; ++k) images[3 * e + k] = im[k];
  if (edge_index) {
    edge_index[2 * e] = atom;
    edge_index[2 * e + 1] = atom;
  }
  if (edge_image)
#pragma unroll
    for (int k = 0; k < 3; ++k) edge_image[3 * e + k] = (float)im[k];
}

}  // namespace

extern "C" {

int fmd_nl_overflow_rows(const uint8_t* overflow, int64_t n_atoms, int64_t e_cap, int32_t n_dummy, int32_t pad_ix,
                         int32_t pad_iy, int32_t pad_iz, int32_t* center, int32_t* neighbor, int32_t* images,
                         int32_t* edge_index, float* edge_image, hipStream_t stream) {
  FMD_REQUIRE(overflow && center && neighbor && images && n_atoms > 0 && e_cap > 0 && e_cap % 2 == 0 && n_dummy >= 0);
  FMD_REQUIRE(n_atoms + n_dummy < (int64_t(1) << 31));
  hipLaunchKernelGGL(lg_overflow_rows_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, overflow,
                     n_atoms, e_cap, n_dummy, pad_ix, pad_iy, pad_iz, center, neighbor, images, edge_index, edge_image);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int64_t fmd_nl_line_graph_work_size(int64_t n_atoms, int64_t e_cap) {
  const int64_t nb = fmd_cdiv(e_cap, kLgBlock);
  return 2 * nb + 8 + e_cap + fmd_cdiv(e_cap, 2);  // block sums, leader prefix, short ranks (int32)
}

int fmd_nl_line_graph(const int32_t* center, const int32_t* edge_reverse, const uint8_t* short_flags,
                      const int64_t* edge_offsets, const uint8_t* candidate_valid, int64_t n_atoms, int64_t e_cap,
                      int64_t u_cap, int64_t t_cap, int32_t bmax, int64_t* work, int32_t* d2u, int32_t* u2d,
                      uint8_t* invalid_pairs, int64_t* short_counts, int64_t* short_offsets,
                      int32_t* short_edge_matrix, int64_t* pair_offsets, uint8_t* overflow, int32_t* line_graph,
                      int64_t* edge_triplet_offsets, int32_t* bond_rows, int32_t* second_perm, int32_t n_dummy,
                      hipStream_t stream) {
  FMD_REQUIRE(n_atoms > 0 && e_cap > 0 && u_cap > 0 && t_cap > 0 && bmax > 0 && e_cap == 2 * u_cap);
  FMD_REQUIRE(n_dummy >= 0 && n_atoms + n_dummy < (int64_t(1) << 31));
  FMD_REQUIRE(e_cap < (int64_t(1) << 31) && t_cap < (int64_t(1) << 31) && n_atoms < (int64_t(1) << 31));
  FMD_REQUIRE(edge_reverse && short_flags && edge_offsets && candidate_valid && work && d2u && u2d && invalid_pairs);
  FMD_REQUIRE(short_counts && short_offsets && short_edge_matrix && pair_offsets && overflow && line_graph);
  FMD_REQUIRE(center && edge_triplet_offsets && bond_rows && second_perm);
  const int64_t nb = fmd_cdiv(e_cap, kLgBlock);
  int64_t* pfx = work + 2 * nb + 8;
  int32_t* short_rank = reinterpret_cast<int32_t*>(pfx + e_cap);
  hipLaunchKernelGGL(lg_leader_count_kernel, dim3((unsigned)nb), dim3(kLgBlock), 0, stream, edge_reverse, edge_offsets,
                     n_atoms, e_cap, nb, work);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_leader_scan_kernel, dim3(1), dim3(kLgBlock), 0, stream, edge_offsets, n_atoms, nb, work,
                     invalid_pairs);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_leader_apply_kernel, dim3((unsigned)nb), dim3(kLgBlock), 0, stream, edge_reverse, edge_offsets,
                     n_atoms, e_cap, work, pfx);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_short_kernel, dim3((unsigned)fmd_cdiv(n_atoms, 4)), dim3(256), 0, stream, short_flags,
                     edge_offsets, n_atoms, e_cap, bmax, short_counts, short_edge_matrix, short_rank);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_pairs_scan_kernel, dim3(1), dim3(kLgBlock), 0, stream, short_counts, edge_offsets,
                     invalid_pairs, candidate_valid, n_atoms, e_cap, t_cap, short_offsets, pair_offsets, overflow);
  FMD_CHECK_LAUNCH();
  const int64_t idx = e_cap > u_cap ? e_cap : u_cap;
  hipLaunchKernelGGL(lg_pairs_index_kernel, dim3((unsigned)fmd_cdiv(idx, 256)), dim3(256), 0, stream, edge_reverse,
                     edge_offsets, pfx, overflow, n_atoms, e_cap, u_cap, d2u, u2d);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_edge_offsets_kernel, dim3((unsigned)fmd_cdiv(e_cap + 1, 256)), dim3(256), 0, stream, center,
                     short_flags, short_rank, short_counts, short_offsets, pair_offsets, edge_offsets, n_atoms, e_cap,
                     t_cap, edge_triplet_offsets, bond_rows);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(lg_line_graph_kernel, dim3((unsigned)fmd_cdiv(t_cap, 256)), dim3(256), 0, stream, pair_offsets,
                     short_counts, short_edge_matrix, d2u, edge_offsets, overflow, n_atoms, e_cap, u_cap, t_cap, bmax,
                     n_dummy, line_graph, second_perm);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
