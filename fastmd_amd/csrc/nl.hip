// (a) Neighbour list of the GPU-resident MD step: candidate cell list (rare refresh path) and
// the per-step exact re-filter build over the candidates (count -> offsets + materialize + pad ->
// reverse rows + flags), bit-exact against the CPU oracle.
//
// Arithmetic contract (shared with oracle/nl.py): every float32 operation below is a single
// IEEE round-to-nearest operation in the written order, with no contraction into FMAs (this
// file is compiled with -ffp-contract=off and the pragma below):
//   frac_a   = (x*inv[0][a] + y*inv[1][a]) + z*inv[2][a]          (small_matmul, geometry.py:7-34)
//   wrap_a   = floor(frac_a);  frac_a -= wrap_a
//   wrapped_c = (f0*cell[0][c] + f1*cell[1][c]) + f2*cell[2][c]
//   d_c      = (((p_j,c - p_i,c) + sx*cell[0][c]) + sy*cell[1][c]) + sz*cell[2][c]
//   d2       = (dx*dx + dy*dy) + dz*dz,    edge iff d2 < rc2        (fixed_capacity_builder.py:163-171)
// Candidates are stored per atom in ascending (neighbour, sx, sy, sz) order, so the rows the
// build materializes at edge_offsets[i] + rank are already in the canonical (centre,
// neighbour, image) order that the reference obtains with a global torch.sort
// (fixed_capacity_builder.py:1968-1999): image = shift + wrap_delta[j] - wrap_delta[i] is a
// per-neighbour constant offset of the shift, so the per-row order is preserved.
#pragma clang fp contract(off)

#include <mutex>

#include "common.h"

namespace {

constexpr int kSmallThreads = 1024;   // fused single-workgroup build
constexpr int kSmallMaxAtoms = 1024;  // LDS-resident wrapped coordinates up to this many atoms
constexpr int kSmallBatch = 4;        // atoms per wave whose candidate loads are issued together
constexpr int kSmallMaxEdges = 8192;  // rows whose reverse search runs on LDS copies of their keys
constexpr int kImageBias = 512;       // packed image fields: component + 512 in 10 bits
constexpr int kBlock = 256;           // multi-block kernels: 4 waves, one atom per wave

struct Mat3 {
  float m[9];
};

__device__ __forceinline__ Mat3 load_mat3(const float* p) {
  Mat3 r;
#pragma unroll
  for (int k = 0; k < 9; ++k) r.m[k] = p[k];
  return r;
}

__device__ __forceinline__ void load_position(const void* positions, int is64, int64_t i, float& x,
                                              float& y, float& z) {
  if (is64) {
    const double* p = static_cast<const double*>(positions) + 3 * i;
    x = (float)p[0];
    y = (float)p[1];
    z = (float)p[2];
  } else {
    const float* p = static_cast<const float*>(positions) + 3 * i;
    x = p[0];
    y = p[1];
    z = p[2];
  }
}

// pos -> fractional coordinates in [0,1), integer wraps and the wrapped Cartesian position.
__device__ __forceinline__ void wrap_position(float x, float y, float z, const Mat3& inv, const Mat3& cell,
                                              float f[3], int w[3], float wr[3]) {
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    float t = x * inv.m[a];
    t = t + y * inv.m[3 + a];
    t = t + z * inv.m[6 + a];
    float fl = floorf(t);
    w[a] = (int)fl;
    f[a] = t - fl;
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float t = f[0] * cell.m[c];
    t = t + f[1] * cell.m[3 + c];
    t = t + f[2] * cell.m[6 + c];
    wr[c] = t;
  }
}

__device__ __forceinline__ float pair_d2(float xi, float yi, float zi, float xj, float yj, float zj, float sx,
                                         float sy, float sz, const Mat3& cell) {
  float dx = xj - xi;
  dx = dx + sx * cell.m[0];
  dx = dx + sy * cell.m[3];
  dx = dx + sz * cell.m[6];
  float dy = yj - yi;
  dy = dy + sx * cell.m[1];
  dy = dy + sy * cell.m[4];
  dy = dy + sz * cell.m[7];
  float dz = zj - zi;
  dz = dz + sx * cell.m[2];
  dz = dz + sy * cell.m[5];
  dz = dz + sz * cell.m[8];
  float d2 = dx * dx;
  d2 = d2 + dy * dy;
  d2 = d2 + dz * dz;
  return d2;
}

__device__ __forceinline__ float displacement_norm(float x, float y, float z, const float* ref) {
  float dx = x - ref[0], dy = y - ref[1], dz = z - ref[2];
  float s = dx * dx;
  s = s + dy * dy;
  s = s + dz * dz;
  return sqrtf(s);
}

// ------------------------------------------------------------------------------------------
// wrap (refresh flavour)
// ------------------------------------------------------------------------------------------
__global__ void nl_wrap_kernel(const void* positions, int is64, const float* inv_cell, const float* cell,
                               int64_t n, float* frac, int32_t* wraps, float* wrapped, float* ref_pos,
                               int32_t* ref_wraps, int32_t* wrap_delta) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  Mat3 inv = load_mat3(inv_cell), cm = load_mat3(cell);
  float x, y, z, f[3], wr[3];
  int w[3];
  load_position(positions, is64, i, x, y, z);
  wrap_position(x, y, z, inv, cm, f, w, wr);
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    if (frac) frac[3 * i + a] = f[a];
    if (wraps) wraps[3 * i + a] = w[a];
    if (wrapped) wrapped[3 * i + a] = wr[a];
    if (ref_wraps) ref_wraps[3 * i + a] = w[a];
    if (wrap_delta) wrap_delta[3 * i + a] = 0;
  }
  if (ref_pos) {
    ref_pos[3 * i] = x;
    ref_pos[3 * i + 1] = y;
    ref_pos[3 * i + 2] = z;
  }
}

// ------------------------------------------------------------------------------------------
// candidate cell list
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ int cell_coord(float f, int nc) {
  int c = (int)floorf(f * (float)nc);
  c = c < 0 ? 0 : c;
  return c >= nc ? nc - 1 : c;
}

__global__ void cells_reset_kernel(int32_t* cell_count, int64_t ncell, uint8_t* capacity_valid) {
  int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c < ncell) cell_count[c] = 0;
  if (c == 0) capacity_valid[0] = 1;
}

__global__ void cells_count_kernel(const float* frac, int64_t n, int n0, int n1, int n2, int32_t* cell_count) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int c0 = cell_coord(frac[3 * i], n0), c1 = cell_coord(frac[3 * i + 1], n1), c2 = cell_coord(frac[3 * i + 2], n2);
  atomicAdd(&cell_count[(c0 * n1 + c1) * n2 + c2], 1);
}

// Exclusive scan of the cell counts (one workgroup); leaves the counts zeroed as cursors.
__global__ void cells_scan_kernel(int32_t* cell_count, int32_t* cell_start, int64_t ncell) {
  __shared__ int32_t partial[1024];
  const int t = threadIdx.x, T = blockDim.x;
  const int64_t chunk = fmd_cdiv(ncell, T);
  const int64_t lo = t * chunk, hi = lo + chunk < ncell ? lo + chunk : ncell;
  int32_t s = 0;
  for (int64_t c = lo; c < hi; ++c) s += cell_count[c];
  partial[t] = s;
  __syncthreads();
  if (t == 0) {
    int32_t run = 0;
    for (int k = 0; k < T; ++k) {
      int32_t v = partial[k];
      partial[k] = run;
      run += v;
    }
    cell_start[ncell] = run;
  }
  __syncthreads();
  int32_t run = partial[t];
  for (int64_t c = lo; c < hi; ++c) {
    int32_t v = cell_count[c];
    cell_start[c] = run;
    run += v;
    cell_count[c] = 0;
  }
}

__global__ void cells_place_kernel(const float* frac, int64_t n, int n0, int n1, int n2, int32_t* cursor,
                                   const int32_t* cell_start, int32_t* cell_atoms) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int c0 = cell_coord(frac[3 * i], n0), c1 = cell_coord(frac[3 * i + 1], n1), c2 = cell_coord(frac[3 * i + 2], n2);
  int cid = (c0 * n1 + c1) * n2 + c2;
  int slot = atomicAdd(&cursor[cid], 1);
  cell_atoms[cell_start[cid] + slot] = (int32_t)i;
}

__device__ __forceinline__ uint64_t cand_key(int32_t j, int sx, int sy, int sz) {
  return ((uint64_t)(uint32_t)j << 24) | ((uint64_t)(sx + 128) << 16) | ((uint64_t)(sy + 128) << 8) |
         (uint64_t)(sz + 128);
}

// One workgroup per atom: test every atom of the cells within reach (all periodic images),
// collect the candidate keys in LDS, bitonic-sort them and write the row.
__global__ void __launch_bounds__(256) cells_query_kernel(const float* wrapped, const float* frac, const float* cell,
                                                          int64_t n, float cutoff2, int n0, int n1, int n2, int r0,
                                                          int r1, int r2, int32_t bmax, int lcap,
                                                          const int32_t* cell_start, const int32_t* cell_atoms,
                                                          int32_t* neighbor_matrix, int32_t* neighbor_shifts,
                                                          int32_t* num_neighbors, uint8_t* capacity_valid,
                                                          int64_t system_size, int64_t index_offset) {
  extern __shared__ uint64_t keys[];
  __shared__ int counter;
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;
  if (t == 0) counter = 0;
  __syncthreads();
  Mat3 cm = load_mat3(cell);
  const float xi = wrapped[3 * i], yi = wrapped[3 * i + 1], zi = wrapped[3 * i + 2];
  const int c0 = cell_coord(frac[3 * i], n0), c1 = cell_coord(frac[3 * i + 1], n1), c2 = cell_coord(frac[3 * i + 2], n2);
  const int span0 = 2 * r0 + 1, span1 = 2 * r1 + 1, span2 = 2 * r2 + 1;
  const int noff = span0 * span1 * span2;
  for (int q = t; q < noff; q += blockDim.x) {
    const int d0 = q / (span1 * span2) - r0;
    const int d1 = (q / span2) % span1 - r1;
    const int d2 = q % span2 - r2;
    int t0 = c0 + d0, t1 = c1 + d1, t2 = c2 + d2;
    // floor division into (cell, image shift)
    int s0 = (t0 >= 0) ? t0 / n0 : -((-t0 + n0 - 1) / n0);
    int s1 = (t1 >= 0) ? t1 / n1 : -((-t1 + n1 - 1) / n1);
    int s2 = (t2 >= 0) ? t2 / n2 : -((-t2 + n2 - 1) / n2);
    t0 -= s0 * n0;
    t1 -= s1 * n1;
    t2 -= s2 * n2;
    const int cid = (t0 * n1 + t1) * n2 + t2;
    const float sx = (float)s0, sy = (float)s1, sz = (float)s2;
    for (int p = cell_start[cid]; p < cell_start[cid + 1]; ++p) {
      const int32_t j = cell_atoms[p];
      if (j == i && s0 == 0 && s1 == 0 && s2 == 0) continue;
      // replicas of one system side by side (atoms [k S, (k+1) S) each): no pair across them
      if (system_size > 0 && (int64_t)j / system_size != i / system_size) continue;
      const float d2v = pair_d2(xi, yi, zi, wrapped[3 * j], wrapped[3 * j + 1], wrapped[3 * j + 2], sx, sy, sz, cm);
      if (d2v < cutoff2) {
        int slot = atomicAdd(&counter, 1);
        if (slot < lcap) keys[slot] = cand_key(j, s0, s1, s2);
      }
    }
  }
  __syncthreads();
  const int count = counter;
  // a row whose candidates overflowed the LDS keys holds an arrival-order subset of them: it is
  // stored empty instead (deterministic; the row is flagged invalid below since lcap >= bmax)
  const int stored = count <= lcap ? count : 0;
  int P = 1;
  while (P < stored) P <<= 1;
  for (int k = stored + t; k < P; k += blockDim.x) keys[k] = ~0ull;
  __syncthreads();
  // bitonic sort of keys[0, P)
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int k = t; k < P / 2; k += blockDim.x) {
        const int lo = 2 * k - (k & (stride - 1));
        const int hi = lo + stride;
        const bool up = ((lo & size) == 0);
        const uint64_t a = keys[lo], b = keys[hi];
        if ((a > b) == up) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  int32_t* nrow = neighbor_matrix + i * bmax;
  int32_t* srow = neighbor_shifts + i * bmax * 3;
  for (int s = t; s < bmax; s += blockDim.x) {
    int32_t j = (int32_t)(n + index_offset);
    int sx = 0, sy = 0, sz = 0;
    if (s < stored) {
      const uint64_t key = keys[s];
      j = (int32_t)((int64_t)(key >> 24) + index_offset);
      sx = (int)((key >> 16) & 0xff) - 128;
      sy = (int)((key >> 8) & 0xff) - 128;
      sz = (int)(key & 0xff) - 128;
    }
    nrow[s] = j;
    srow[3 * s] = sx;
    srow[3 * s + 1] = sy;
    srow[3 * s + 2] = sz;
  }
  if (t == 0) {
    num_neighbors[i] = count;
    if (count > bmax) capacity_valid[0] = 0;
  }
}

// ------------------------------------------------------------------------------------------
// per-step build
// ------------------------------------------------------------------------------------------
struct BuildArgs {
  const void* positions;
  int pos64;
  const float* inv_cell;
  const float* cell;
  int64_t n;
  const int32_t* nbr;
  const int32_t* shifts;
  const int32_t* num;
  int32_t bmax;
  const float* ref_pos;
  const int32_t* ref_wraps;
  const uint8_t* capacity_valid;
  float rc2;
  float skin_limit;
  int minimum_image;  // a lattice jump since the refresh is no motion (see atom_motion)
  int pad_ix, pad_iy, pad_iz;
  // sink padding (> 0): padded rows are self-loops of the sink rows n .. n + n_dummy - 1 (image
  // (3, 3, 3), distance 1e6), a padded pair's two rows on one sink, the pairs spread evenly over
  // the sinks (fixed_capacity_builder.py:291-320); 0: far self-loops with the pad image
  int n_dummy;
  // several systems in one union (null: one system): the system of each row; then inv_cell and
  // cell are [systems, 9] tables and pad_images [systems, 3] the far self-loop image of each
  const int32_t* system_of;
  const int32_t* pad_images;
  int64_t e_cap;
  int64_t* work;
  float* frac;
  int32_t* wrap_delta;
  float* wrapped_out;
  int64_t* edge_counts;
  int64_t* edge_offsets;
  int32_t* center;
  int32_t* neighbor;
  int32_t* images;
  float* distances;
  int32_t* edge_index;
  float* edge_image;
  float* max_disp;
  uint8_t* cand_valid;
  uint8_t* overflow;
  int32_t* isolated;
  float line2;           // line-graph (bond) cutoff squared, float32
  uint8_t* short_flags;  // [e_cap]: real row with d2 < line2 (null: not written)
  int32_t* reverse;      // [e_cap]: the reverse row of every real row, -1 past them (null: not formed)
  // a whole-step window's flags, folded with this build's status (w_over null: not folded)
  uint8_t* w_over;
  uint8_t* w_cap;
  int64_t* w_edges;
  int32_t* w_iso;
  double* w_stats;
  int w_check_iso;
};

// The cell and inverse cell of atom i (its system's, in a union of systems).
__device__ __forceinline__ void atom_frame(const BuildArgs& a, int64_t i, Mat3& inv, Mat3& cm) {
  const int64_t base = a.system_of ? 9 * (int64_t)a.system_of[i] : 0;
  inv = load_mat3(a.inv_cell + base);
  cm = load_mat3(a.cell + base);
}

// Skin-test motion of atom i since the refresh and its wrap delta wd = wraps - reference_wraps
// (fixed_capacity_builder.py:2219-2251). With minimum_image a lattice jump L since the refresh
// (the caller wrapped the atom, e.g. ASE's atoms.wrap()) is no motion: the displacement
// d = pos - ref loses jumps = rint(d inv) (small_matmul order, round half to even), d -= jumps
// cell, and the jump leaves the wrap delta, so the candidates' images stay exact.
__device__ __forceinline__ float atom_motion(const BuildArgs& a, int64_t i, float x, float y, float z,
                                             const int w[3], const Mat3& inv, const Mat3& cm, int wd[3]) {
  const float* ref = a.ref_pos + 3 * i;
  float d[3] = {x - ref[0], y - ref[1], z - ref[2]};
#pragma unroll
  for (int k = 0; k < 3; ++k) wd[k] = w[k] - a.ref_wraps[3 * i + k];
  if (a.minimum_image) {
    float jump[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float t = d[0] * inv.m[c];
      t = t + d[1] * inv.m[3 + c];
      t = t + d[2] * inv.m[6 + c];
      jump[c] = rintf(t);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float t = jump[0] * cm.m[c];
      t = t + jump[1] * cm.m[3 + c];
      t = t + jump[2] * cm.m[6 + c];
      d[c] = d[c] - t;
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) wd[k] -= (int)jump[k];
  }
  float sq = d[0] * d[0];
  sq = sq + d[1] * d[1];
  sq = sq + d[2] * d[2];
  return sqrtf(sq);
}

// d2: the row's squared distance (the edge decision's own value: the short-bond decision uses the
// same bits, fixed_capacity_builder.py:258-260)
__device__ __forceinline__ void write_row(const BuildArgs& a, int64_t row, int32_t c, int32_t j, int ix, int iy,
                                          int iz, float d2, bool real) {
  a.center[row] = c;
  a.neighbor[row] = j;
  a.images[3 * row] = ix;
  a.images[3 * row + 1] = iy;
  a.images[3 * row + 2] = iz;
  if (real) a.distances[row] = sqrtf(d2);
  if (a.short_flags) a.short_flags[row] = real && d2 < a.line2 ? 1 : 0;
  if (a.edge_index) {
    a.edge_index[2 * row] = c;
    a.edge_index[2 * row + 1] = j;
  }
  if (a.edge_image) {
    a.edge_image[3 * row] = (float)ix;
    a.edge_image[3 * row + 1] = (float)iy;
    a.edge_image[3 * row + 2] = (float)iz;
  }
}

// Validity of candidate slot s of atom i, given the atom's wrapped position and wrap delta and
// a functor giving (wrapped_j, wrap_delta_j).
// The same test from the slot's candidate entry (j_raw) and lattice shift (sh), loaded beforehand.
template <typename NeighborFn>
__device__ __forceinline__ bool slot_edge_of(const BuildArgs& a, const Mat3& cm, int32_t j_raw, const int32_t sh[3],
                                             float xi, float yi, float zi, const int wdi[3], NeighborFn nbr_state,
                                             int32_t& j, int img[3], float& d2) {
  j = j_raw < (int32_t)a.n - 1 ? j_raw : (int32_t)a.n - 1;
  float xj, yj, zj;
  int wdj[3];
  nbr_state(j, xj, yj, zj, wdj);
#pragma unroll
  for (int k = 0; k < 3; ++k) img[k] = sh[k] + wdj[k] - wdi[k];
  d2 = pair_d2(xi, yi, zi, xj, yj, zj, (float)img[0], (float)img[1], (float)img[2], cm);
  return d2 < a.rc2;
}

template <typename NeighborFn>
__device__ __forceinline__ bool slot_edge(const BuildArgs& a, const Mat3& cm, int64_t i, int s, float xi, float yi,
                                          float zi, const int wdi[3], NeighborFn nbr_state, int32_t& j, int img[3],
                                          float& d2) {
  const int32_t* sh = a.shifts + (i * a.bmax + s) * 3;
  const int32_t shv[3] = {sh[0], sh[1], sh[2]};
  return slot_edge_of(a, cm, a.nbr[i * a.bmax + s], shv, xi, yi, zi, wdi, nbr_state, j, img, d2);
}

// Reverse rows of a build (the search of nl_reverse_kernel) over rows start, start + step, ...:
// row e (i -> j, image) finds the first row of j's block [off[j], off[j + 1]) at or after
// (i, -image) in (neighbor, image) order and takes it when it is that pair, else -1; rows past
// the real ones get -1. Four rows per thread at a time, so that their loads overlap.
template <typename OffFn>
__device__ __forceinline__ void reverse_rows(const BuildArgs& a, int64_t ec, OffFn off_of, int64_t start,
                                             int64_t step) {
  constexpr int R = 4;
  for (int64_t e0 = start; e0 < a.e_cap; e0 += R * step) {
    int64_t e[R], lo[R], hi[R], end[R];
    int32_t c[R];
    int ix[R], iy[R], iz[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      e[k] = e0 + k * step;
      lo[k] = hi[k] = end[k] = 0;
      c[k] = 0;
      ix[k] = iy[k] = iz[k] = 0;
      if (e[k] < ec) {
        c[k] = a.center[e[k]];
        const int32_t j = a.neighbor[e[k]];
        ix[k] = -a.images[3 * e[k]];
        iy[k] = -a.images[3 * e[k] + 1];
        iz[k] = -a.images[3 * e[k] + 2];
        const int64_t o1 = off_of(j + 1);
        end[k] = o1 < ec ? o1 : ec;
        hi[k] = end[k];
        const int64_t o0 = off_of(j);
        lo[k] = o0 < hi[k] ? o0 : hi[k];
      }
    }
    bool any = true;
    while (any) {
      any = false;
#pragma unroll
      for (int k = 0; k < R; ++k) {
        if (lo[k] < hi[k]) {
          const int64_t mid = (lo[k] + hi[k]) >> 1;
          const int32_t mj = a.neighbor[mid];
          const int mx = a.images[3 * mid], my = a.images[3 * mid + 1], mz = a.images[3 * mid + 2];
          const bool less = (mj < c[k]) || (mj == c[k] && (mx < ix[k] || (mx == ix[k] && (my < iy[k] ||
                                                                                       (my == iy[k] && mz < iz[k])))));
          if (less)
            lo[k] = mid + 1;
          else
            hi[k] = mid;
          any = true;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      if (e[k] >= a.e_cap) continue;
      int32_t r = -1;
      if (e[k] < ec && lo[k] < end[k] && a.neighbor[lo[k]] == c[k] && a.images[3 * lo[k]] == ix[k] &&
          a.images[3 * lo[k] + 1] == iy[k] && a.images[3 * lo[k] + 2] == iz[k])
        r = (int32_t)lo[k];
      a.reverse[e[k]] = r;
    }
  }
}

__device__ __forceinline__ void pad_rows(const BuildArgs& a, int64_t total, int64_t start, int64_t step) {
  const int64_t ec = total < a.e_cap ? total : a.e_cap;
  if (a.n_dummy > 0) {
    const int64_t free_u = a.e_cap / 2 - ec / 2;
    for (int64_t row = ec + start; row < a.e_cap; row += step) {
      const int64_t pair = (row - ec) / 2;
      const int32_t sink = (int32_t)(a.n + pair * a.n_dummy / (free_u > 1 ? free_u : 1));
      write_row(a, row, sink, sink, 3, 3, 3, 0.f, false);
      a.distances[row] = 1.0e6f;
    }
    return;
  }
  for (int64_t row = ec + start; row < a.e_cap; row += step) {
    const int32_t atom = (int32_t)((row - ec) % a.n);
    if (a.system_of) {
      const int32_t* im = a.pad_images + 3 * a.system_of[atom];
      write_row(a, row, atom, atom, im[0], im[1], im[2], 0.f, false);
    } else {
      write_row(a, row, atom, atom, a.pad_ix, a.pad_iy, a.pad_iz, 0.f, false);
    }
  }
}

// One build's status folded into a whole-step window's flags (one thread).
__device__ __forceinline__ void window_fold(int64_t edges, int32_t iso, bool overflowed, const uint8_t* invalid_pairs,
                                           int64_t e_cap, int check_isolated, uint8_t* w_over, uint8_t* w_cap,
                                           int64_t* w_edges, int32_t* w_iso, float max_disp, double* stats,
                                           const int64_t* triplet_count, int64_t t_cap, int64_t* w_triplets) {
  bool flag = overflowed;
  if (check_isolated) flag = flag || iso > 0;
  const uint8_t wo = (w_over[0] != 0 || flag) ? 1 : 0;
  w_over[0] = wo;
  // a line-graph build (triplet_count given) overflows its pairs at edges == e_cap (no padding
  // pair left), and its triplets above t_cap
  const int64_t triplets = triplet_count ? triplet_count[0] : 0;
  const bool cap = (triplet_count ? edges >= e_cap : edges > e_cap) || (invalid_pairs && invalid_pairs[0] != 0) ||
                   (triplet_count && triplets > t_cap);
  int64_t wt = 0;
  if (w_triplets) {
    wt = triplets > w_triplets[0] ? triplets : w_triplets[0];
    w_triplets[0] = wt;
  }
  const uint8_t wc = (w_cap[0] != 0 || cap) ? 1 : 0;
  w_cap[0] = wc;
  const int64_t we = edges > w_edges[0] ? edges : w_edges[0];
  w_edges[0] = we;
  w_iso[0] = iso > w_iso[0] ? iso : w_iso[0];
  if (stats) {
    // the window's statistics after this build: (overflow, edges, triplets, max displacement,
    // capacity overflow, max edges, max isolated)
    stats[0] = (double)wo;
    stats[1] = (double)edges;
    stats[2] = (double)wt;
    stats[3] = (double)max_disp;
    stats[4] = (double)wc;
    stats[5] = (double)we;
    stats[6] = (double)w_iso[0];
  }
}

// Fused build of small systems in ONE workgroup (no inter-block dependency): prologue, counts,
// scan, materialization, padding and flags, with the wrapped coordinates in LDS.
__global__ void __launch_bounds__(kSmallThreads) nl_build_small_kernel(BuildArgs a) {
  __shared__ float s_pos[kSmallMaxAtoms * 3];
  __shared__ int32_t s_wd[kSmallMaxAtoms * 3];
  __shared__ int32_t s_cnt[kSmallMaxAtoms + 1];
  __shared__ float s_red[kSmallThreads / FMD_WAVE];
  __shared__ int32_t s_iso[kSmallThreads / FMD_WAVE];
  __shared__ int32_t s_scan[kSmallThreads];
  // the keys of the real rows for the reverse search (row < kSmallMaxEdges): centre, neighbour and
  // the image packed as three 10-bit fields of component + 512 (field order = lexicographic order)
  __shared__ int16_t s_rc[kSmallMaxEdges];
  __shared__ int32_t s_rn[kSmallMaxEdges];
  __shared__ uint32_t s_ri[kSmallMaxEdges];
  __shared__ int s_wide_image;  // some real row has an image component outside [-511, 511]
  const int t = threadIdx.x, T = blockDim.x;
  if (t == 0) s_wide_image = 0;
  const int lane = t & (FMD_WAVE - 1), wave = t / FMD_WAVE, nwaves = T / FMD_WAVE;
  const int n = (int)a.n;

  // (1) prologue
  float dmax = 0.f;
  for (int i = t; i < n; i += T) {
    float x, y, z, f[3], wr[3];
    int w[3];
    Mat3 inv, cm;
    atom_frame(a, i, inv, cm);
    load_position(a.positions, a.pos64, i, x, y, z);
    wrap_position(x, y, z, inv, cm, f, w, wr);
    int wd[3];
    const float moved = atom_motion(a, i, x, y, z, w, inv, cm, wd);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      a.frac[3 * i + k] = f[k];
      a.wrap_delta[3 * i + k] = wd[k];
      if (a.wrapped_out) a.wrapped_out[3 * i + k] = wr[k];
      s_pos[3 * i + k] = wr[k];
      s_wd[3 * i + k] = wd[k];
    }
    dmax = nan_max(dmax, moved);
  }
  dmax = wave_nan_max(dmax);
  if (lane == 0) s_red[wave] = dmax;
  __syncthreads();

  auto nbr_state = [&](int32_t j, float& xj, float& yj, float& zj, int wdj[3]) {
    xj = s_pos[3 * j];
    yj = s_pos[3 * j + 1];
    zj = s_pos[3 * j + 2];
    wdj[0] = s_wd[3 * j];
    wdj[1] = s_wd[3 * j + 1];
    wdj[2] = s_wd[3 * j + 2];
  };

  // The first 64 candidate slots of kSmallBatch atoms of a wave (atoms i0 + u nwaves) with their
  // loads issued together: one memory round trip per batch instead of one per atom. Slots past
  // the candidate count are loaded (in bounds: the matrix has bmax slots per atom) and ignored.
  struct SlotBatch {
    int cnt[kSmallBatch];
    int32_t j[kSmallBatch];
    int32_t sh[kSmallBatch][3];
  };
  auto load_batch = [&](int i0, SlotBatch& b) {
#pragma unroll
    for (int u = 0; u < kSmallBatch; ++u) {
      const int i = i0 + u * nwaves;
      b.cnt[u] = 0;
      b.j[u] = 0;
      b.sh[u][0] = b.sh[u][1] = b.sh[u][2] = 0;
      if (i < n) {
        const int c = a.num[i];
        b.cnt[u] = c < a.bmax ? c : a.bmax;
        if (lane < a.bmax) {
          const int64_t q = (int64_t)i * a.bmax + lane;
          b.j[u] = a.nbr[q];
          b.sh[u][0] = a.shifts[3 * q];
          b.sh[u][1] = a.shifts[3 * q + 1];
          b.sh[u][2] = a.shifts[3 * q + 2];
        }
      }
    }
  };

  // (2) counts, one wave per atom
  int iso = 0;
  for (int i0 = wave; i0 < n; i0 += nwaves * kSmallBatch) {
    SlotBatch b;
    load_batch(i0, b);
#pragma unroll
    for (int u = 0; u < kSmallBatch; ++u) {
      const int i = i0 + u * nwaves;
      if (i >= n) break;
      const float xi = s_pos[3 * i], yi = s_pos[3 * i + 1], zi = s_pos[3 * i + 2];
      const int wdi[3] = {s_wd[3 * i], s_wd[3 * i + 1], s_wd[3 * i + 2]};
      Mat3 inv, cm;
      atom_frame(a, i, inv, cm);
      const int cnt = b.cnt[u];
      int32_t j;
      int img[3];
      float d2;
      bool e = lane < cnt && slot_edge_of(a, cm, b.j[u], b.sh[u], xi, yi, zi, wdi, nbr_state, j, img, d2);
      int total = __popcll(__ballot(e));
      for (int base = FMD_WAVE; base < cnt; base += FMD_WAVE) {
        const int s = base + lane;
        e = s < cnt && slot_edge(a, cm, i, s, xi, yi, zi, wdi, nbr_state, j, img, d2);
        total += __popcll(__ballot(e));
      }
      if (lane == 0) {
        s_cnt[i] = total;
        a.edge_counts[i] = total;
        iso += (total == 0);
      }
    }
  }
  if (lane == 0) s_iso[wave] = iso;
  __syncthreads();

  // (3) exclusive scan of the counts (chunk per thread, then a block scan over the threads)
  {
    const int chunk = (n + T - 1) / T;
    const int lo = t * chunk, hi = lo + chunk < n ? lo + chunk : n;
    int s = 0;
    for (int k = lo; k < hi; ++k) s += s_cnt[k];
    int total = 0;
    const int mine = block_exclusive_scan<int>(s, s_scan, &total);
    if (t == 0) {
      const int run = total;
      s_cnt[kSmallMaxAtoms] = run;
      float m = s_red[0];
      int isol = s_iso[0];
      for (int k = 1; k < nwaves; ++k) {
        m = nan_max(m, s_red[k]);
        isol += s_iso[k];
      }
      const bool valid = (m * 2.0f <= a.skin_limit) && (a.capacity_valid[0] != 0);
      const bool over = (int64_t)run > a.e_cap || !valid;
      a.max_disp[0] = m;
      a.cand_valid[0] = valid ? 1 : 0;
      a.overflow[0] = over ? 1 : 0;
      a.isolated[0] = isol;
      a.edge_offsets[n] = run;
      if (a.w_over)
        window_fold(run, isol, over, nullptr, a.e_cap, a.w_check_iso, a.w_over, a.w_cap, a.w_edges, a.w_iso, m,
                    a.w_stats, nullptr, 0, nullptr);
    }
    __syncthreads();
    int run = mine;
    for (int k = lo; k < hi; ++k) {
      const int v = s_cnt[k];
      s_cnt[k] = run;  // now the offset
      a.edge_offsets[k] = run;
      run += v;
    }
  }
  __syncthreads();
  const int64_t total = s_cnt[kSmallMaxAtoms];

  // (4) materialize in candidate (= canonical) order
  for (int i0 = wave; i0 < n; i0 += nwaves * kSmallBatch) {
    SlotBatch b;
    load_batch(i0, b);
#pragma unroll
    for (int u = 0; u < kSmallBatch; ++u) {
      const int i = i0 + u * nwaves;
      if (i >= n) break;
      const float xi = s_pos[3 * i], yi = s_pos[3 * i + 1], zi = s_pos[3 * i + 2];
      const int wdi[3] = {s_wd[3 * i], s_wd[3 * i + 1], s_wd[3 * i + 2]};
      Mat3 inv, cm;
      atom_frame(a, i, inv, cm);
      const int cnt = b.cnt[u];
      int64_t row0 = s_cnt[i];
      for (int base = 0; base < cnt; base += FMD_WAVE) {
        const int s = base + lane;
        bool e = false;
        int32_t j = 0;
        int img[3] = {0, 0, 0};
        float d2 = 0.f;
        if (s < cnt) {
          e = base == 0 ? slot_edge_of(a, cm, b.j[u], b.sh[u], xi, yi, zi, wdi, nbr_state, j, img, d2)
                        : slot_edge(a, cm, i, s, xi, yi, zi, wdi, nbr_state, j, img, d2);
        }
        const uint64_t m = __ballot(e);
        const int64_t row = row0 + lane_prefix(m);
        if (e && row < a.e_cap) {
          write_row(a, row, (int32_t)i, j, img[0], img[1], img[2], d2, true);
          if (row < kSmallMaxEdges) {
            const bool narrow = img[0] > -kImageBias && img[0] < kImageBias && img[1] > -kImageBias &&
                                img[1] < kImageBias && img[2] > -kImageBias && img[2] < kImageBias;
            if (!narrow) s_wide_image = 1;
            s_rc[row] = (int16_t)i;
            s_rn[row] = j;
            s_ri[row] = ((uint32_t)(img[0] + kImageBias) << 20) | ((uint32_t)(img[1] + kImageBias) << 10) |
                        (uint32_t)(img[2] + kImageBias);
          }
        }
        row0 += __popcll(m);
      }
    }
  }
  // (5) padding rows
  pad_rows(a, total, t, T);
  // (6) reverse rows: the search of nl_reverse_kernel on the LDS keys, or (more rows than the
  // LDS holds, or a wide image) on the rows this workgroup has written (visible after the barrier)
  if (a.reverse) {
    __syncthreads();
    const int64_t ec = total < a.e_cap ? total : a.e_cap;
    auto off_of = [&](int64_t k) -> int64_t { return k < n ? s_cnt[k] : total; };
    if (ec > kSmallMaxEdges || s_wide_image) {
      reverse_rows(a, ec, off_of, t, T);
      return;
    }
    constexpr uint32_t kField = 2 * kImageBias, kMask = kField - 1;
    for (int64_t e = t; e < a.e_cap; e += T) {
      int32_t r = -1;
      if (e < ec) {
        const int32_t c = s_rc[e], j = s_rn[e];
        const uint32_t p = s_ri[e];
        // (c, -image): each field f = component + 512 in [1, 1023] becomes 1024 - f
        const uint32_t want = ((kField - (p >> 20)) << 20) | ((kField - ((p >> 10) & kMask)) << 10) |
                              (kField - (p & kMask));
        const int64_t o1 = off_of(j + 1);
        const int64_t end = o1 < ec ? o1 : ec;
        int64_t hi = end;
        const int64_t o0 = off_of(j);
        int64_t lo = o0 < hi ? o0 : hi;
        while (lo < hi) {
          const int64_t mid = (lo + hi) >> 1;
          const int32_t mj = s_rn[mid];
          if (mj < c || (mj == c && s_ri[mid] < want))
            lo = mid + 1;
          else
            hi = mid;
        }
        if (lo < end && s_rn[lo] == c && s_ri[lo] == want) r = (int32_t)lo;
      }
      a.reverse[e] = r;
    }
  }
}

// Multi-block path, kernel 1: prologue of atom i (own wrap) and its edge count; the
// neighbours' wrapped coordinates are recomputed from their positions with the same
// arithmetic (bitwise the values kernel 1 publishes for them).
__global__ void __launch_bounds__(kBlock) nl_count_kernel(BuildArgs a) {
  __shared__ float s_red[kBlock / FMD_WAVE];
  __shared__ int32_t s_iso[kBlock / FMD_WAVE];
  __shared__ int32_t s_cnt[kBlock / FMD_WAVE];
  const int lane = threadIdx.x & (FMD_WAVE - 1), wave = threadIdx.x / FMD_WAVE;
  const int64_t i = (int64_t)blockIdx.x * (kBlock / FMD_WAVE) + wave;
  float dmax = 0.f;
  int iso = 0;
  int ecount = 0;  // the atom's edge count (uniform over the wave)
  if (i < a.n) {
    Mat3 inv, cm;
    atom_frame(a, i, inv, cm);  // atom i's system's; its neighbours are of the same system
    float x, y, z, f[3], wr[3];
    int w[3], wdi[3];
    load_position(a.positions, a.pos64, i, x, y, z);
    wrap_position(x, y, z, inv, cm, f, w, wr);
    dmax = atom_motion(a, i, x, y, z, w, inv, cm, wdi);
    if (lane < 3) {
      a.frac[3 * i + lane] = f[lane];
      a.wrap_delta[3 * i + lane] = wdi[lane];
      if (a.wrapped_out) a.wrapped_out[3 * i + lane] = wr[lane];
    }
    auto nbr_state = [&](int32_t j, float& xj, float& yj, float& zj, int wdj[3]) {
      float px, py, pz, fj[3], wj[3];
      int ww[3];
      load_position(a.positions, a.pos64, j, px, py, pz);
      wrap_position(px, py, pz, inv, cm, fj, ww, wj);
      xj = wj[0];
      yj = wj[1];
      zj = wj[2];
      atom_motion(a, j, px, py, pz, ww, inv, cm, wdj);  // the wrap delta kernel 1 publishes for j
    };
    int cnt = a.num[i];
    cnt = cnt < a.bmax ? cnt : a.bmax;
    int total = 0;
    for (int base = 0; base < cnt; base += FMD_WAVE) {
      const int s = base + lane;
      bool e = false;
      if (s < cnt) {
        int32_t j;
        int img[3];
        float d2;
        e = slot_edge(a, cm, i, s, wr[0], wr[1], wr[2], wdi, nbr_state, j, img, d2);
      }
      total += __popcll(__ballot(e));
    }
    if (lane == 0) a.edge_counts[i] = total;
    iso = (total == 0);
    ecount = total;
  }
  if (lane == 0) {
    s_red[wave] = dmax;
    s_iso[wave] = iso;
    s_cnt[wave] = ecount;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = s_red[0];
    int isol = s_iso[0];
    for (int k = 1; k < kBlock / FMD_WAVE; ++k) {
      m = nan_max(m, s_red[k]);
      isol += s_iso[k];
    }
    const int64_t nb = gridDim.x;
    float* red = reinterpret_cast<float*>(a.work);
    red[blockIdx.x] = m;
    reinterpret_cast<int32_t*>(a.work + fmd_cdiv(nb, 2))[blockIdx.x] = isol;
    // the block's edge count, for the materialize kernel's row offsets
    int32_t sum = 0;
    for (int k = 0; k < kBlock / FMD_WAVE; ++k) sum += s_cnt[k];
    reinterpret_cast<int32_t*>(a.work + 2 * fmd_cdiv(nb, 2))[blockIdx.x] = sum;
  }
}

// Loads each thread keeps in flight when it sums the count kernel's per-workgroup partials.
constexpr int kScanLoads = 8;

// Kernel 2: the offsets and the materialization in one launch (one wave per atom, neighbours'
// state from kernel 1's output) and, in the trailing workgroups, the padding rows. An atom
// workgroup takes the atoms of the count kernel's workgroup of the same index (kBlock / 64
// each): its first row is the sum of that kernel's per-workgroup edge counts before it, read by
// every thread strided (16-byte loads, all of a thread's loads issued before any use), and its
// atoms follow in atom order. The first padding workgroup sums every count workgroup's edges (the
// total, edge_offsets[n]) and reduces the count kernel's partials (maximum displacement, isolated
// atoms) into the build's flags. Integer sums are exact: the offsets are those of any grouping.
__global__ void __launch_bounds__(kBlock) nl_materialize_kernel(BuildArgs a, int64_t atom_blocks) {
  __shared__ int64_t s_pre[kBlock / FMD_WAVE];
  __shared__ int32_t s_cnt[kBlock / FMD_WAVE];
  __shared__ float s_max[kBlock / FMD_WAVE];
  __shared__ int32_t s_iso[kBlock / FMD_WAVE];
  const int t = threadIdx.x, lane = t & (FMD_WAVE - 1), wave = t / FMD_WAVE;
  const bool pad = (int64_t)blockIdx.x >= atom_blocks, first_pad = (int64_t)blockIdx.x == atom_blocks;
  const int64_t before = pad ? atom_blocks : (int64_t)blockIdx.x;  // count workgroups before this one's rows
  const int32_t* bsum = reinterpret_cast<const int32_t*>(a.work + 2 * fmd_cdiv(atom_blocks, 2));
  const int4* bsum4 = reinterpret_cast<const int4*>(bsum);
  const int64_t before4 = before / 4;
  int64_t pre = 0;
  for (int64_t q0 = t; q0 < before4; q0 += (int64_t)kBlock * kScanLoads) {
    int4 v[kScanLoads];
#pragma unroll
    for (int u = 0; u < kScanLoads; ++u) {
      const int64_t q = q0 + (int64_t)u * kBlock;
      v[u] = q < before4 ? bsum4[q] : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kScanLoads; ++u) pre += (int64_t)v[u].x + v[u].y + v[u].z + v[u].w;
  }
  for (int64_t b = before4 * 4 + t; b < before; b += kBlock) pre += bsum[b];
  float m = 0.f;
  int32_t iso = 0;
  if (first_pad) {
    const float* red = reinterpret_cast<const float*>(a.work);
    const int32_t* isop = reinterpret_cast<const int32_t*>(a.work + fmd_cdiv(atom_blocks, 2));
    for (int64_t b0 = t; b0 < atom_blocks; b0 += (int64_t)kBlock * kScanLoads) {
      float r[kScanLoads];
      int32_t z[kScanLoads];
#pragma unroll
      for (int u = 0; u < kScanLoads; ++u) {
        const int64_t b = b0 + (int64_t)u * kBlock;
        r[u] = b < atom_blocks ? red[b] : 0.f;
        z[u] = b < atom_blocks ? isop[b] : 0;
      }
#pragma unroll
      for (int u = 0; u < kScanLoads; ++u) {
        m = nan_max(m, r[u]);
        iso += z[u];
      }
    }
  }
  const int64_t i = (int64_t)blockIdx.x * (kBlock / FMD_WAVE) + wave;  // this wave's atom (atom workgroups)
  pre = wave_sum(pre);
  if (first_pad) {
    m = wave_nan_max(m);
    iso = wave_sum(iso);
  }
  if (lane == 0) {
    s_pre[wave] = pre;
    s_max[wave] = m;
    s_iso[wave] = iso;
    s_cnt[wave] = !pad && i < a.n ? a.edge_counts[i] : 0;
  }
  __syncthreads();
  int64_t prefix = 0;
#pragma unroll
  for (int w = 0; w < kBlock / FMD_WAVE; ++w) prefix += s_pre[w];
  if (pad) {
    const int64_t total = prefix;
    if (first_pad && t == 0) {
      float mm = s_max[0];
      int32_t isol = s_iso[0];
      for (int w = 1; w < kBlock / FMD_WAVE; ++w) {
        mm = nan_max(mm, s_max[w]);
        isol += s_iso[w];
      }
      const bool valid = (mm * 2.0f <= a.skin_limit) && (a.capacity_valid[0] != 0);
      a.max_disp[0] = mm;
      a.cand_valid[0] = valid ? 1 : 0;
      a.overflow[0] = (total > a.e_cap || !valid) ? 1 : 0;
      a.isolated[0] = isol;
      a.edge_offsets[a.n] = total;
    }
    const int64_t pb = blockIdx.x - atom_blocks, npb = gridDim.x - atom_blocks;
    pad_rows(a, total, pb * kBlock + t, npb * kBlock);
    return;
  }
  if (i >= a.n) return;
  int64_t row0 = prefix;
  for (int w = 0; w < wave; ++w) row0 += s_cnt[w];
  if (lane == 0) a.edge_offsets[i] = row0;
  Mat3 inv, cm;
  atom_frame(a, i, inv, cm);
  // atom i's own wrapped position: recomputed (kernel 1 may not have published it)
  float x, y, z, f[3], wr[3];
  int w[3];
  load_position(a.positions, a.pos64, i, x, y, z);
  wrap_position(x, y, z, inv, cm, f, w, wr);
  const int wdi[3] = {a.wrap_delta[3 * i], a.wrap_delta[3 * i + 1], a.wrap_delta[3 * i + 2]};
  auto nbr_state = [&](int32_t j, float& xj, float& yj, float& zj, int wdj[3]) {
    float px, py, pz, fj[3], wj[3];
    int ww[3];
    load_position(a.positions, a.pos64, j, px, py, pz);
    wrap_position(px, py, pz, inv, cm, fj, ww, wj);
    xj = wj[0];
    yj = wj[1];
    zj = wj[2];
    wdj[0] = a.wrap_delta[3 * j];
    wdj[1] = a.wrap_delta[3 * j + 1];
    wdj[2] = a.wrap_delta[3 * j + 2];
  };
  int cnt = a.num[i];
  cnt = cnt < a.bmax ? cnt : a.bmax;
  for (int base = 0; base < cnt; base += FMD_WAVE) {
    const int s = base + lane;
    bool e = false;
    int32_t j = 0;
    int img[3] = {0, 0, 0};
    float d2 = 0.f;
    if (s < cnt) e = slot_edge(a, cm, i, s, wr[0], wr[1], wr[2], wdi, nbr_state, j, img, d2);
    const uint64_t m = __ballot(e);
    const int64_t row = row0 + lane_prefix(m);
    if (e && row < a.e_cap) write_row(a, row, (int32_t)i, j, img[0], img[1], img[2], d2, true);
    row0 += __popcll(m);
  }
}

// The window fold of a build whose reverse rows are formed: run by the first thread of the reverse
// kernel (its inputs, the count, the overflow and isolated flags and the maximum displacement, are
// final once materialize has run), so no launch of its own. w_over null: none.
struct RevWindow {
  const int64_t* edge_count;
  const uint8_t* overflow;
  const int32_t* isolated;
  int check_isolated;
  uint8_t* w_over;
  uint8_t* w_cap;
  int64_t* w_edges;
  int32_t* w_iso;
  const float* max_disp;
  double* stats;
};

__global__ void nl_reverse_kernel(const int32_t* center, const int32_t* neighbor, const int32_t* images,
                                  const int64_t* off, int64_t n, int64_t e_cap, int32_t* reverse, const RevWindow w) {
  if (w.w_over && blockIdx.x == 0 && threadIdx.x == 0)
    window_fold(w.edge_count[0], w.isolated[0], w.overflow[0] != 0, nullptr, e_cap, w.check_isolated, w.w_over,
                w.w_cap, w.w_edges, w.w_iso, w.max_disp ? w.max_disp[0] : 0.f, w.stats, nullptr, 0, nullptr);
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = off[n];
  const int64_t ec = total < e_cap ? total : e_cap;
  if (e >= e_cap) return;
  if (e >= ec) {
    reverse[e] = -1;
    return;
  }
  const int32_t c = center[e], j = neighbor[e];
  const int ix = -images[3 * e], iy = -images[3 * e + 1], iz = -images[3 * e + 2];
  int64_t lo = off[j], hi = off[j + 1];
  hi = hi < ec ? hi : ec;
  lo = lo < hi ? lo : hi;
  // first row of the block of j whose (neighbor, image) >= (c, -image)
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const int32_t mj = neighbor[mid];
    const int mx = images[3 * mid], my = images[3 * mid + 1], mz = images[3 * mid + 2];
    const bool less = (mj < c) || (mj == c && (mx < ix || (mx == ix && (my < iy || (my == iy && mz < iz)))));
    if (less)
      lo = mid + 1;
    else
      hi = mid;
  }
  int32_t r = -1;
  int64_t end = off[j + 1] < ec ? off[j + 1] : ec;
  if (lo < end && neighbor[lo] == c && images[3 * lo] == ix && images[3 * lo + 1] == iy && images[3 * lo + 2] == iz)
    r = (int32_t)lo;
  reverse[e] = r;
}

__global__ void nl_window_flags_kernel(const int64_t* edge_count, const uint8_t* invalid_pairs,
                                       const uint8_t* overflow, const int32_t* isolated, int64_t e_cap,
                                       int check_isolated, uint8_t* w_over, uint8_t* w_cap, int64_t* w_edges,
                                       int32_t* w_iso, const float* max_disp, double* stats,
                                       const int64_t* triplet_count, int64_t t_cap, int64_t* w_triplets) {
  if (threadIdx.x != 0) return;
  window_fold(edge_count[0], isolated[0], overflow[0] != 0, invalid_pairs, e_cap, check_isolated, w_over, w_cap,
              w_edges, w_iso, max_disp ? max_disp[0] : 0.f, stats, triplet_count, t_cap, w_triplets);
}

// The build's launches (small systems: one fused workgroup; otherwise count -> offsets and
// materialize (one launch) -> reverse rows with the window flags, with the count kernel's
// per-block partials in a.work).
int launch_build(const BuildArgs& a, hipStream_t stream) {
  FMD_REQUIRE(a.n > 0 && a.n < (int64_t(1) << 31) && a.e_cap > 0 && a.bmax > 0);
  FMD_REQUIRE(a.positions && a.inv_cell && a.cell && a.nbr && a.shifts && a.num);
  FMD_REQUIRE(a.ref_pos && a.ref_wraps && a.capacity_valid && a.work && a.frac && a.wrap_delta);
  FMD_REQUIRE(a.edge_counts && a.edge_offsets && a.center && a.neighbor && a.images && a.distances);
  FMD_REQUIRE(a.max_disp && a.cand_valid && a.overflow && a.isolated);
  FMD_REQUIRE(!a.system_of || a.pad_images);
  FMD_REQUIRE(a.n_dummy >= 0 && (a.n_dummy == 0 || !a.system_of) && a.n + a.n_dummy < (int64_t(1) << 31));
  if (a.n <= kSmallMaxAtoms && a.n <= 1024) {
    hipLaunchKernelGGL(nl_build_small_kernel, dim3(1), dim3(kSmallThreads), 0, stream, a);
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  const int64_t atom_blocks = fmd_cdiv(a.n, kBlock / FMD_WAVE);
  hipLaunchKernelGGL(nl_count_kernel, dim3((unsigned)atom_blocks), dim3(kBlock), 0, stream, a);
  FMD_CHECK_LAUNCH();
  int64_t pad_blocks = fmd_cdiv(a.e_cap, (int64_t)kBlock * 4);
  pad_blocks = pad_blocks < 1 ? 1 : (pad_blocks > 1024 ? 1024 : pad_blocks);
  hipLaunchKernelGGL(nl_materialize_kernel, dim3((unsigned)(atom_blocks + pad_blocks)), dim3(kBlock), 0, stream, a,
                     atom_blocks);
  FMD_CHECK_LAUNCH();
  if (a.reverse) {
    const RevWindow w = a.w_over ? RevWindow{a.edge_offsets + a.n, a.overflow, a.isolated, a.w_check_iso, a.w_over,
                                             a.w_cap, a.w_edges, a.w_iso, a.max_disp, a.w_stats}
                                 : RevWindow{};
    hipLaunchKernelGGL(nl_reverse_kernel, dim3((unsigned)fmd_cdiv(a.e_cap, 256)), dim3(256), 0, stream, a.center,
                       a.neighbor, a.images, a.edge_offsets, a.n, a.e_cap, a.reverse, w);
    FMD_CHECK_LAUNCH();
  } else if (a.w_over) {
    hipLaunchKernelGGL(nl_window_flags_kernel, dim3(1), dim3(64), 0, stream, a.edge_offsets + a.n,
                       (const uint8_t*)nullptr, (const uint8_t*)a.overflow, (const int32_t*)a.isolated, a.e_cap,
                       a.w_check_iso, a.w_over, a.w_cap, a.w_edges, a.w_iso, (const float*)a.max_disp, a.w_stats,
                       (const int64_t*)nullptr, (int64_t)0, (int64_t*)nullptr);
    FMD_CHECK_LAUNCH();
  }
  return FMD_OK;
}

// Scratch of fmd_nl_build_noalloc: the count kernel's per-block partials (max displacement,
// isolated atoms) for up to FMD_NL_BUILD_NOALLOC_MAX_ATOMS atoms. Every block writes its own
// slot before the materialize kernel reads it, so nothing in it has to start at zero. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for the symbol): its
// device address is looked up once per device and kept in scratch_ptr.
static __device__ __align__(256) int64_t scratch[FMD_NL_BUILD_NOALLOC_SCRATCH];

constexpr int kMaxDevices = 64;
std::mutex scratch_lock;
int64_t* scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (hipGetSymbolAddress on the first call per device).
int noalloc_scratch(int64_t** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return (int)err;
  if (device < 0 || device >= kMaxDevices) return FMD_EUNSUPPORTED;
  std::lock_guard<std::mutex> guard(scratch_lock);
  if (scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return (int)err;
    if (ptr == nullptr) return FMD_EUNSUPPORTED;
    scratch_ptr[device] = static_cast<int64_t*>(ptr);
  }
  *out = scratch_ptr[device];
  return FMD_OK;
}

}  // namespace

extern "C" {

int fmd_nl_wrap(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell,
                int64_t n_atoms, float* frac, int32_t* wraps, float* wrapped, float* reference_positions,
                int32_t* reference_wraps, int32_t* wrap_delta, hipStream_t stream) {
  FMD_REQUIRE(n_atoms >= 0 && positions && inv_cell && cell);
  if (n_atoms == 0) return FMD_OK;
  const int threads = 256;
  hipLaunchKernelGGL(nl_wrap_kernel, dim3((unsigned)fmd_cdiv(n_atoms, threads)), dim3(threads), 0, stream,
                     positions, pos_is_f64, inv_cell, cell, n_atoms, frac, wraps, wrapped, reference_positions,
                     reference_wraps, wrap_delta);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_nl_candidates(const float* wrapped, const float* frac, const float* cell, int64_t n_atoms, float cutoff2,
                      const int32_t* ncells, const int32_t* reach, int32_t bmax, int32_t* cell_count,
                      int32_t* cell_start, int32_t* cell_atoms, int32_t* neighbor_matrix, int32_t* neighbor_shifts,
                      int32_t* num_neighbors, uint8_t* capacity_valid, int64_t system_size, int64_t index_offset,
                      hipStream_t stream) {
  FMD_REQUIRE(n_atoms > 0 && bmax > 0 && ncells && reach);
  FMD_REQUIRE(index_offset >= 0 && n_atoms + index_offset < (int64_t(1) << 31));
  FMD_REQUIRE(system_size >= 0 && (system_size == 0 || n_atoms % system_size == 0));
  const int n0 = ncells[0], n1 = ncells[1], n2 = ncells[2];
  const int r0 = reach[0], r1 = reach[1], r2 = reach[2];
  FMD_REQUIRE(n0 > 0 && n1 > 0 && n2 > 0 && r0 >= 0 && r1 >= 0 && r2 >= 0);
  // image shifts are packed in 8 bits: |shift| <= reach / ncells + 1 must stay below 127
  FMD_REQUIRE(r0 / n0 + 2 < 127 && r1 / n1 + 2 < 127 && r2 / n2 + 2 < 127);
  FMD_REQUIRE(n_atoms < (int64_t(1) << 31));
  int lcap = 64;
  while (lcap < bmax) lcap <<= 1;
  if (lcap > 8192) return FMD_EUNSUPPORTED;
  const int64_t ncell = (int64_t)n0 * n1 * n2;
  const int threads = 256;
  hipLaunchKernelGGL(cells_reset_kernel, dim3((unsigned)fmd_cdiv(ncell, threads)), dim3(threads), 0, stream,
                     cell_count, ncell, capacity_valid);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(cells_count_kernel, dim3((unsigned)fmd_cdiv(n_atoms, threads)), dim3(threads), 0, stream, frac,
                     n_atoms, n0, n1, n2, cell_count);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(cells_scan_kernel, dim3(1), dim3(1024), 0, stream, cell_count, cell_start, ncell);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(cells_place_kernel, dim3((unsigned)fmd_cdiv(n_atoms, threads)), dim3(threads), 0, stream, frac,
                     n_atoms, n0, n1, n2, cell_count, cell_start, cell_atoms);
  FMD_CHECK_LAUNCH();
  hipLaunchKernelGGL(cells_query_kernel, dim3((unsigned)n_atoms), dim3(256), (size_t)lcap * sizeof(uint64_t), stream,
                     wrapped, frac, cell, n_atoms, cutoff2, n0, n1, n2, r0, r1, r2, bmax, lcap, cell_start, cell_atoms,
                     neighbor_matrix, neighbor_shifts, num_neighbors, capacity_valid, system_size, index_offset);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int64_t fmd_nl_build_work_size(int64_t n_atoms) {
  const int64_t nb = fmd_cdiv(n_atoms > 0 ? n_atoms : 1, kBlock / FMD_WAVE);
  return 3 * fmd_cdiv(nb, 2) + 2;  // per count block: maximum displacement, isolated atoms, edge count
}

int fmd_nl_build(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell, int64_t n_atoms,
                 const int32_t* neighbor_matrix, const int32_t* neighbor_shifts, const int32_t* num_neighbors,
                 int32_t bmax, const float* reference_positions, const int32_t* reference_wraps,
                 const uint8_t* capacity_valid, float rc2, float skin_limit, int32_t minimum_image, int32_t pad_ix,
                 int32_t pad_iy, int32_t pad_iz, int32_t n_dummy, const int32_t* system_of, const int32_t* pad_images, int64_t e_cap,
                 int64_t* work, float* frac, int32_t* wrap_delta, float* wrapped_out,
                 int64_t* edge_counts, int64_t* edge_offsets, int32_t* center, int32_t* neighbor, int32_t* images,
                 float* distances, int32_t* edge_index, float* edge_image, float* max_displacement,
                 uint8_t* candidate_valid, uint8_t* overflow, int32_t* isolated, float line2, uint8_t* short_flags,
                 int32_t* edge_reverse, uint8_t* window_overflow, uint8_t* window_capacity,
                 int64_t* window_max_edges, int32_t* window_max_isolated, double* window_stats,
                 int32_t window_check_isolated, hipStream_t stream) {
  FMD_REQUIRE(work && reinterpret_cast<uintptr_t>(work) % 16 == 0);  // its partials are read 16 bytes at a time
  FMD_REQUIRE(!window_overflow || (window_capacity && window_max_edges && window_max_isolated));
  BuildArgs a{positions, pos_is_f64, inv_cell, cell, n_atoms, neighbor_matrix, neighbor_shifts, num_neighbors, bmax,
              reference_positions, reference_wraps, capacity_valid, rc2, skin_limit, minimum_image, pad_ix, pad_iy, pad_iz,
              n_dummy, system_of, pad_images, e_cap, work, frac, wrap_delta, wrapped_out, edge_counts, edge_offsets, center, neighbor, images, distances,
              edge_index, edge_image, max_displacement, candidate_valid, overflow, isolated, line2, short_flags,
              edge_reverse, window_overflow, window_capacity, window_max_edges, window_max_isolated, window_stats,
              window_check_isolated};
  return launch_build(a, stream);
}

int fmd_nl_build_noalloc(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell,
                         int64_t n_atoms, const int32_t* neighbor_matrix, const int32_t* neighbor_shifts,
                         const int32_t* num_neighbors, int32_t bmax, const float* reference_positions,
                         const int32_t* reference_wraps, const uint8_t* capacity_valid, float rc2, float skin_limit,
                         int32_t minimum_image, int32_t pad_ix, int32_t pad_iy, int32_t pad_iz, int32_t n_dummy,
                         const int32_t* system_of, const int32_t* pad_images, int64_t e_cap, float* frac,
                         int32_t* wrap_delta, float* wrapped_out, int64_t* edge_counts, int64_t* edge_offsets,
                         int32_t* center, int32_t* neighbor, int32_t* images, float* distances, int32_t* edge_index,
                         float* edge_image, float* max_displacement, uint8_t* candidate_valid, uint8_t* overflow,
                         int32_t* isolated, float line2, uint8_t* short_flags, hipStream_t stream) {
  if (n_atoms > FMD_NL_BUILD_NOALLOC_MAX_ATOMS) return FMD_ETOOLARGE;
  FMD_REQUIRE(n_atoms > 0 && fmd_nl_build_work_size(n_atoms) <= FMD_NL_BUILD_NOALLOC_SCRATCH);
  int64_t* work = nullptr;
  const int status = noalloc_scratch(&work);
  if (status != FMD_OK) return status;
  BuildArgs a{positions, pos_is_f64, inv_cell, cell, n_atoms, neighbor_matrix, neighbor_shifts, num_neighbors, bmax,
              reference_positions, reference_wraps, capacity_valid, rc2, skin_limit, minimum_image, pad_ix, pad_iy, pad_iz,
              n_dummy, system_of, pad_images, e_cap, work, frac, wrap_delta, wrapped_out, edge_counts, edge_offsets, center, neighbor, images, distances,
              edge_index, edge_image, max_displacement, candidate_valid, overflow, isolated, line2, short_flags,
              nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0};
  return launch_build(a, stream);
}

// padded rows of a bucket workspace: rows [e_real, e_cap) become far self-loops of atom
// (row - e_real) mod n (the builder's own padding rule), with no reverse row
__global__ void nl_pad_rows_kernel(int32_t* edge_index, float* edge_image, int32_t* edge_reverse, int64_t e_real,
                                   int64_t e_cap, int64_t n, int32_t ix, int32_t iy, int32_t iz) {
  const int64_t row = e_real + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= e_cap) return;
  const int32_t atom = (int32_t)((row - e_real) % n);
  edge_index[2 * row] = atom;
  edge_index[2 * row + 1] = atom;
  edge_image[3 * row] = (float)ix;
  edge_image[3 * row + 1] = (float)iy;
  edge_image[3 * row + 2] = (float)iz;
  if (edge_reverse) edge_reverse[row] = -1;
}

int fmd_nl_pad_rows(int32_t* edge_index, float* edge_image, int32_t* edge_reverse, int64_t e_real, int64_t e_cap,
                    int64_t n_atoms, int32_t pad_ix, int32_t pad_iy, int32_t pad_iz, hipStream_t stream) {
  FMD_REQUIRE(e_real >= 0 && e_real <= e_cap && n_atoms > 0 && edge_index && edge_image);
  if (e_real == e_cap) return FMD_OK;
  hipLaunchKernelGGL(nl_pad_rows_kernel, dim3((unsigned)fmd_cdiv(e_cap - e_real, 256)), dim3(256), 0, stream,
                     edge_index, edge_image, edge_reverse, e_real, e_cap, n_atoms, pad_ix, pad_iy, pad_iz);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

// the edge-vector override of exact-cutoff padding (fixed_capacity_builder.py:357-361): the pad
// vector on rows [min(n_edges, e_cap), e_cap), zero on the real rows
__global__ void nl_pad_override_kernel(const int64_t* n_edges, int64_t e_cap, float vx, float vy, float vz,
                                       float* vec_override) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= e_cap) return;
  const int64_t total = n_edges[0];
  const bool pad = row >= (total < e_cap ? total : e_cap);
  vec_override[3 * row] = pad ? vx : 0.f;
  vec_override[3 * row + 1] = pad ? vy : 0.f;
  vec_override[3 * row + 2] = pad ? vz : 0.f;
}

int fmd_nl_pad_override(const int64_t* n_edges, int64_t e_cap, float vx, float vy, float vz, float* vec_override,
                        hipStream_t stream) {
  FMD_REQUIRE(n_edges && vec_override && e_cap > 0);
  hipLaunchKernelGGL(nl_pad_override_kernel, dim3((unsigned)fmd_cdiv(e_cap, 256)), dim3(256), 0, stream, n_edges,
                     e_cap, vx, vy, vz, vec_override);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_nl_reverse(const int32_t* center, const int32_t* neighbor, const int32_t* images, const int64_t* edge_offsets,
                   int64_t n_atoms, int64_t e_cap, int32_t* reverse, hipStream_t stream) {
  FMD_REQUIRE(n_atoms > 0 && e_cap > 0 && center && neighbor && images && edge_offsets && reverse);
  const int threads = 256;
  hipLaunchKernelGGL(nl_reverse_kernel, dim3((unsigned)fmd_cdiv(e_cap, threads)), dim3(threads), 0, stream, center,
                     neighbor, images, edge_offsets, n_atoms, e_cap, reverse, RevWindow{});
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_nl_window_flags(const int64_t* edge_count, const uint8_t* invalid_pairs, const uint8_t* overflow,
                        const int32_t* isolated, int64_t e_cap, int32_t check_isolated, uint8_t* window_overflow,
                        uint8_t* window_capacity_overflow, int64_t* window_max_edges, int32_t* window_max_isolated,
                        const float* max_displacement, double* stats, const int64_t* triplet_count, int64_t t_cap,
                        int64_t* window_max_triplets, hipStream_t stream) {
  FMD_REQUIRE(edge_count && overflow && isolated && window_overflow && window_capacity_overflow &&
              window_max_edges && window_max_isolated);
  FMD_REQUIRE(!triplet_count || t_cap > 0);
  hipLaunchKernelGGL(nl_window_flags_kernel, dim3(1), dim3(64), 0, stream, edge_count, invalid_pairs, overflow,
                     isolated, e_cap, check_isolated, window_overflow, window_capacity_overflow, window_max_edges,
                     window_max_isolated, max_displacement, stats, triplet_count, t_cap, window_max_triplets);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
