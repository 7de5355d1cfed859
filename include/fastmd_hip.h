/*
 * fastmd_hip.h - C ABI of the MI355X (gfx950) kernels of the GPU-resident MD step.
 *
 * Every entry point takes plain device pointers, sizes and the hipStream_t to launch on
 * (torch's current stream), never allocates or frees memory, never synchronizes the host
 * and returns 0 on success or a nonzero status (a hipError_t, or one of the FMD_E* codes
 * below) that fmd_error_string() describes. Argument validation happens in the Python
 * wrappers before the launch; the checks here only reject launches that could not be
 * in bounds (negative sizes, null buffers that a kernel would dereference).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   (a) fastmd/graph/fixed_capacity_builder.py, fastmd/graph/gpu_graph_builder.py
 *   (b) fastmd/models/matris/op/triton_gather_cat.py
 *   (c) fastmd/models/matris/op/triton_csr_segment_sum.py, fastmd/engine/kernels/segment.py
 *   (d) fastmd/engine/kernels/triton_wide_gemm.py
 *   (e) fastmd/execution/gpu_nhc.py
 * Line citations sit beside each declaration.
 */
#ifndef FASTMD_HIP_H
#define FASTMD_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMD_ABI_VERSION 1

/* Status codes beyond hipError_t (hipError_t values stay below 10000). */
#define FMD_OK 0
#define FMD_EINVAL 10001      /* a size or pointer argument no launch could honour */
#define FMD_EUNSUPPORTED 10002 /* a configuration this build does not implement */
#define FMD_ETOOLARGE 10003   /* a size beyond an allocation-free entry point's static scratch */

int fmd_abi_version(void);
const char* fmd_error_string(int status);

/* ----------------------------------------------------------------------------------------
 * (a) Neighbour list
 * -------------------------------------------------------------------------------------- */

/* Candidate refresh: the cell-list candidates of every atom within `cutoff` (the builder's
 * candidate cutoff = pair cutoff + skin), over all periodic images, from the WRAPPED float32
 * coordinates. Row i of `neighbor_matrix`/`neighbor_shifts` (row stride bmax) holds the first
 * bmax candidates of atom i in ascending (neighbour, sx, sy, sz) order; `num_neighbors[i]`
 * counts every candidate (a count above bmax means truncation; `capacity_valid[0]` = all
 * counts <= bmax). Unused slots keep neighbour n_atoms and shift 0.
 * ncells/reach: cells per lattice axis and the cell search reach per axis (host computed).
 * Replaces nvalchemiops batch_build_cell_list/batch_query_cell_list as called at
 * fastmd/graph/fixed_capacity_builder.py:1519-1554 (FixedCapacityGraphBuilder._build_candidates).
 * system_size > 0: the atoms are replicas of one system, [k S, (k+1) S) each, and pairs across
 * replicas are not candidates (the union graph of replica batching, replica_batch.py:126-180).
 * index_offset is added to every stored neighbour index (the pad value becomes
 * n_atoms + index_offset): a union of systems searches each system on its own slice of rows and
 * stores union indices. A row with more candidates than the LDS key buffer holds (at least
 * bmax) is stored empty, so every row's content is deterministic; it is flagged invalid. */
int fmd_nl_candidates(const float* wrapped, const float* frac, const float* cell, int64_t n_atoms,
                      float cutoff2, const int32_t* ncells, const int32_t* reach, int32_t bmax,
                      int32_t* cell_count, int32_t* cell_start, int32_t* cell_atoms,
                      int32_t* neighbor_matrix, int32_t* neighbor_shifts, int32_t* num_neighbors,
                      uint8_t* capacity_valid, int64_t system_size, int64_t index_offset,
                      hipStream_t stream);

/* Wrap (refresh flavour): float32 positions -> fractional coordinates in [0,1), integer
 * wraps and wrapped Cartesian coordinates; optionally resets the reference positions/wraps
 * and the wrap delta (refresh). `positions` are float32 (pos_is_f64 = 0) or float64 (1, cast
 * to float32 first). Replaces fixed_capacity_builder.py:1674-1685 (refresh_candidates). */
int fmd_nl_wrap(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell,
                int64_t n_atoms, float* frac, int32_t* wraps, float* wrapped,
                float* reference_positions, int32_t* reference_wraps, int32_t* wrap_delta,
                hipStream_t stream);

/* One exact re-filter build over the candidate list (the per-step path of a fixed-capacity,
 * edges-only builder): wrap + wrap delta + skin test, per-atom edge counts, exclusive scan,
 * materialization of the rows at edge_offsets[i] + rank (rows >= e_cap dropped), far
 * self-loop padding of rows [min(E, e_cap), e_cap), overflow flag and the published batch
 * buffers. The candidates are sorted per atom, so the rows come out in the canonical
 * (centre, neighbour, image) order of fixed_capacity_builder.py:1968-1999 without a sort.
 * Replaces FixedCapacityGraphBuilder.build(rebuild_candidates=False)
 * fixed_capacity_builder.py:2180-2298 with _count_neighbors_kernel :97-185,
 * _materialize_neighbors_kernel :188-288, _pad_self_loops_kernel :323-366, _sort_edges
 * :1968-1999 and the batch copies :2260-2282.
 *   positions      float32 or float64 [n,3] (pos_is_f64)
 *   inv_cell, cell float32 [3,3] (row = lattice vector)
 *   neighbor_matrix/neighbor_shifts/num_neighbors: the refresh's candidates (bmax stride)
 *   reference_positions [n,3] f32, reference_wraps [n,3] i32: state of the last refresh
 *   capacity_valid  uint8[1] from the refresh
 *   rc2             float32 square of the pair cutoff
 *   skin_limit      float32: the build is valid iff 2 * max displacement <= skin_limit
 *   system_of       null for one system; for a union of systems (system_batch.py:177-444) the
 *                   system of each row [n] i32: inv_cell and cell are then [systems, 3, 3]
 *                   tables, each row wraps with its system's cell, and pad_images [systems, 3]
 *                   i32 gives the far self-loop image of each system's padded rows (pad_i* unused)
 *   minimum_image   1: a lattice jump since the refresh (the caller wrapped an atom) is no
 *                   motion: the skin test takes the minimum-image displacement and the jump
 *                   leaves the wrap delta (fixed_capacity_builder.py:2233-2245); 0: plain
 *   pad_image       integer image of the padded self-loops
 *   n_dummy         0: far self-loop padding (pad_image); > 0: sink padding
 *                   (_pad_edges_kernel, fixed_capacity_builder.py:291-320): padded row r is a
 *                   self-loop of sink row n + p n_dummy / (e_cap / 2 - ec / 2), p = (r - ec) / 2,
 *                   ec = min(E, e_cap), image (3, 3, 3), distance 1e6 (one system only)
 *   work            int64 scratch of fmd_nl_build_work_size(n) elements, 16-byte aligned
 * Outputs: frac [n,3] f32, wrap_delta [n,3] i32, wrapped_out [n,3] f32 (published
 * positions, may be null), edge_counts [n] i64, edge_offsets [n+1] i64, center/neighbor
 * [e_cap] i32, images [e_cap,3] i32, distances [e_cap] f32, edge_index [e_cap,2] i32 and
 * edge_image [e_cap,3] f32 (published, may be null), status: max_displacement f32[1],
 * candidate_valid u8[1], overflow u8[1], isolated i32[1]; short_flags [e_cap] u8 (may be null:
 * a line-graph build's short-bond flag, real rows with the same d2 < line2, line2 the float32
 * square of the bond cutoff, fixed_capacity_builder.py:258-260; padding rows 0); edge_reverse
 * [e_cap] i32 (may be null: not formed) the reverse rows of fmd_nl_reverse on this build's rows,
 * formed in the same launch for small systems (one workgroup), else by one more launch.
 * window_* (window_overflow null: not folded; window_stats may be null): this build's status folded
 * into a whole-step window's flags as fmd_nl_window_flags does for an edges-only build (in the same
 * launch for small systems, else by one more launch). */
int64_t fmd_nl_build_work_size(int64_t n_atoms);
int fmd_nl_build(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell,
                 int64_t n_atoms, const int32_t* neighbor_matrix, const int32_t* neighbor_shifts,
                 const int32_t* num_neighbors, int32_t bmax, const float* reference_positions,
                 const int32_t* reference_wraps, const uint8_t* capacity_valid, float rc2,
                 float skin_limit, int32_t minimum_image, int32_t pad_ix, int32_t pad_iy, int32_t pad_iz,
                 int32_t n_dummy, const int32_t* system_of, const int32_t* pad_images, int64_t e_cap, int64_t* work,
                 float* frac, int32_t* wrap_delta, float* wrapped_out,
                 int64_t* edge_counts, int64_t* edge_offsets, int32_t* center, int32_t* neighbor,
                 int32_t* images, float* distances, int32_t* edge_index, float* edge_image,
                 float* max_displacement, uint8_t* candidate_valid, uint8_t* overflow,
                 int32_t* isolated, float line2, uint8_t* short_flags, int32_t* edge_reverse,
                 uint8_t* window_overflow, uint8_t* window_capacity, int64_t* window_max_edges,
                 int32_t* window_max_isolated, double* window_stats, int32_t window_check_isolated,
                 hipStream_t stream);

/* Allocation-free variant of fmd_nl_build. It has no counterpart in the reference: it is for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). Same arguments, kernels and results as fmd_nl_build,
 * without `work` (and without edge_reverse: fmd_nl_reverse forms it): the per-block partials go
 * to a static device array of
 * FMD_NL_BUILD_NOALLOC_SCRATCH int64 words (3 MiB) that each GPU the library runs on holds until
 * the process ends. n_atoms above FMD_NL_BUILD_NOALLOC_MAX_ATOMS returns FMD_ETOOLARGE with
 * nothing launched. Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents (nothing in it must start at zero: each block writes its slot before it is read).
 * It must not be called concurrently on one device: two calls whose kernels can overlap (on
 * streams the caller has not ordered, or from two host threads) overwrite each other's partials
 * and both return wrong edge offsets and flags, with no error reported. Calls on one stream, or
 * on streams ordered by events, are safe. */
#define FMD_NL_BUILD_NOALLOC_MAX_ATOMS (1 << 20)
#define FMD_NL_BUILD_NOALLOC_SCRATCH 393218 /* fmd_nl_build_work_size(FMD_NL_BUILD_NOALLOC_MAX_ATOMS) */
int fmd_nl_build_noalloc(const void* positions, int32_t pos_is_f64, const float* inv_cell, const float* cell,
                         int64_t n_atoms, const int32_t* neighbor_matrix, const int32_t* neighbor_shifts,
                         const int32_t* num_neighbors, int32_t bmax, const float* reference_positions,
                         const int32_t* reference_wraps, const uint8_t* capacity_valid, float rc2,
                         float skin_limit, int32_t minimum_image, int32_t pad_ix, int32_t pad_iy,
                         int32_t pad_iz, int32_t n_dummy, const int32_t* system_of, const int32_t* pad_images,
                         int64_t e_cap,
                         float* frac, int32_t* wrap_delta, float* wrapped_out, int64_t* edge_counts,
                         int64_t* edge_offsets, int32_t* center, int32_t* neighbor, int32_t* images,
                         float* distances, int32_t* edge_index, float* edge_image, float* max_displacement,
                         uint8_t* candidate_valid, uint8_t* overflow, int32_t* isolated, float line2,
                         uint8_t* short_flags, hipStream_t stream);

/* The three-body line graph over a build's rows (FixedCapacityGraphBuilder._materialize_pairs
 * / _materialize_line_graph / _line_graph_kernel, fixed_capacity_builder.py:2001-2161,680-753),
 * far self-loop padding: directed2undirected d2u [e_cap] i32 and undirected2directed u2d
 * [u_cap] i32 (e_cap = 2 u_cap), invalid_pairs u8[1], short_counts [n] i64, short_offsets and
 * pair_offsets [n+1] i64 (exclusive scans of s and s (s - 1)), short_edge_matrix [n, bmax] i32
 * (an atom's short rows in row order, then e_cap), overflow u8[1] (set to edges >= e_cap |
 * triplets > t_cap | invalid_pairs | !candidate_valid), line_graph [t_cap, 5] i32 rows
 * (atom, u1, row1, u2, row2), the all-loop topology on overflow. Inputs: edge_reverse from
 * fmd_nl_reverse, short_flags from fmd_nl_build, work of fmd_nl_line_graph_work_size int64.
 * Also the segment layouts of the angle -> bond -> atom sums: edge_triplet_offsets [e_cap + 1]
 * i64, a CSR over the directed rows whose run for row e holds the triplets with e as their first
 * bond (empty for other rows; clamped to t_cap), bond_rows [e_cap] i32, the short rows in
 * (atom, rank) order (then -1), the rows of the CSR short_offsets over the atoms, and second_perm
 * [t_cap] i32, the permutation that with edge_triplet_offsets lists for row e the triplets with e
 * as their second bond, by first bond (-1 past the real triplets and throughout an overflowed build).
 * n_dummy > 0 (sink padding): padding triplet t sits on sink n + (t - t_real) n_dummy /
 * (t_cap - t_real), and the overflow topology is all-sink (_line_graph_kernel without
 * LOOP_PADDING and _allocate_overflow_topology, fixed_capacity_builder.py:745-749,1474-1513). */
int64_t fmd_nl_line_graph_work_size(int64_t n_atoms, int64_t e_cap);
int fmd_nl_line_graph(const int32_t* center, const int32_t* edge_reverse, const uint8_t* short_flags,
                      const int64_t* edge_offsets, const uint8_t* candidate_valid, int64_t n_atoms, int64_t e_cap,
                      int64_t u_cap, int64_t t_cap, int32_t bmax, int64_t* work, int32_t* d2u, int32_t* u2d,
                      uint8_t* invalid_pairs, int64_t* short_counts, int64_t* short_offsets,
                      int32_t* short_edge_matrix, int64_t* pair_offsets, uint8_t* overflow, int32_t* line_graph,
                      int64_t* edge_triplet_offsets, int32_t* bond_rows, int32_t* second_perm, int32_t n_dummy,
                      hipStream_t stream);

/* The edge rows of an overflowed line-graph build, after fmd_nl_line_graph (overflow its flag):
 * row e becomes a loop of pair u = e / 2's atom, u mod n (far self-loops) or sink
 * n + u n_dummy / (e_cap / 2), image + or - the pad image ((3, 3, 3) for sinks) for even / odd e;
 * nothing is written without overflow. Replaces _substitute_overflow_topology with the edge part
 * of _allocate_overflow_topology (fixed_capacity_builder.py:2163-2177,1474-1496). edge_index
 * [e_cap, 2] i32 and edge_image [e_cap, 3] f32 (the published copies) may be null. */
int fmd_nl_overflow_rows(const uint8_t* overflow, int64_t n_atoms, int64_t e_cap, int32_t n_dummy, int32_t pad_ix,
                         int32_t pad_iy, int32_t pad_iz, int32_t* center, int32_t* neighbor, int32_t* images,
                         int32_t* edge_index, float* edge_image, hipStream_t stream);

/* The edge-vector override of exact-cutoff padding (PaddingRule("exact_rc_loops"),
 * fixed_capacity_builder.py:323-366 with HAS_OVERRIDE): vec_override [e_cap, 3] f32 holds
 * (vx, vy, vz) on the padded rows [min(*n_edges, e_cap), e_cap) and 0 on the real rows. */
int fmd_nl_pad_override(const int64_t* n_edges, int64_t e_cap, float vx, float vy, float vz, float* vec_override,
                        hipStream_t stream);

/* The three-body Fourier angle basis (threebody_fourier_basis, triton_threebody_fourier.py:45-80,
 * :230-260): out[t] = [1/sqrt(2), sin(theta f_k), cos(theta f_k)] / scale (1 + 2 n_freq columns),
 * theta = acos((u[target[t]] . u[source[t]]) (1 - 1e-6)), u rows of stride ld_unit. */
int fmd_threebody_fourier_f32(const float* unit_vec, int64_t ld_unit, const int32_t* target_index,
                              const int32_t* source_index, int64_t rows, const float* freqs, int32_t n_freq,
                              float scale, float* out, hipStream_t stream);
/* Its per-row VJP terms: contrib[t] = (g to u[target[t]], g to u[source[t]]) [rows, 6]; the caller
 * sums them per vector row in a fixed order (the reference's atomics, :121-127, are not used). */
int fmd_threebody_fourier_bwd_rows_f32(const float* gout, const float* unit_vec, int64_t ld_unit,
                                       const int32_t* target_index, const int32_t* source_index, int64_t rows,
                                       const float* freqs, int32_t n_freq, float scale, float* contrib,
                                       hipStream_t stream);
/* The basis over a line graph of fmd_nl_line_graph (target = first bond, source = second bond of
 * each triplet row; padding rows from line_graph) and its VJP over the real triplets,
 * deterministic: one wave per atom forms its bonds' gradients (grad_unit rows of the short bonds,
 * = or += with accumulate) from its triplets in triplet order. overflow (nullable) is the build's
 * flag: set, every row is read from line_graph and the VJP is zero. */
int fmd_threebody_fourier_line_f32(const float* unit_vec, int64_t ld_unit, const int64_t* pair_offsets,
                                   const int64_t* short_counts, const int32_t* short_edge_matrix, int32_t bmax,
                                   const int32_t* line_graph, const uint8_t* overflow, int64_t n_atoms, int64_t t_cap,
                                   const float* freqs, int32_t n_freq, float scale, float* out, hipStream_t stream);
int fmd_threebody_fourier_line_bwd_f32(const float* gout, const float* unit_vec, int64_t ld_unit,
                                       const int64_t* pair_offsets, const int64_t* short_counts,
                                       const int32_t* short_edge_matrix, int32_t bmax, const uint8_t* overflow,
                                       int64_t n_atoms, int64_t t_cap, const float* freqs, int32_t n_freq, float scale,
                                       float* grad_unit, int64_t ld_grad, int32_t accumulate, hipStream_t stream);

/* ---- three-body (CHGNet/MatRIS-style) model kernels. The reference runs CHGNet (upstream
 * chgnet, fastmd/models/chgnet.py:1-60) and MatRIS (fastmd/models/matris/interaction_block.py)
 * through their own modules; these are the pieces of this package's configs[4] model: the bond
 * envelope of the line graph, the gated segment sums of its angle -> bond and edge -> atom updates
 * (the reference's triplet gather + segment sums, fastmd/models/matris/op/
 * triton_weighted_segment_sum.py, triton_csr_segment_sum.py:433-479), the readout and the
 * geometry VJP. */

/* geo [e_cap, 8] rows (u, r, fc, dfc, s, ds) of fmd_edge_geometry_f32: writes s, ds, the polynomial
 * envelope 1 - 21x^5 + 35x^6 - 15x^7 (x = r / rb) of each real short row and its r-derivative (0
 * elsewhere). */
int fmd_tb_bond_envelope_f32(float* geo, const uint8_t* short_flags, const int64_t* n_edges, int64_t e_cap, float rb,
                             hipStream_t stream);
/* out[s] (+)= scale * sum_{r in [offsets[s], offsets[s+1]) and r < rows} silu(z[r]) * w(r),
 * w(r) = w[r], w[index1[r]] or w[index1[r]] * w[index2[r]] (index rows of stride ld_index, w of
 * stride ldw); one wave per segment, rows in order. channels <= 256. */
int fmd_tb_gated_sum_f32(const float* z, int64_t ldz, int64_t rows, int32_t channels, const float* w, int64_t ldw,
                         const int32_t* index1, const int32_t* index2, int64_t ld_index, const int64_t* offsets,
                         int64_t n_segments, float scale, float* out, int64_t ldo, int32_t accumulate,
                         hipStream_t stream);
/* Its VJP: gz[r] = scale gout[s] w(r) silu'(z[r]) for every row (0 past the last run); gsum[s] =
 * sum_r gz[r] (nullable); gw[r] (nullable) = sum_c scale gout[s] silu(z[r]), as (gw w2, gw w1) for
 * the two-index weight, stored or (accumulate_gw) added. */
int fmd_tb_gated_sum_bwd_f32(const float* gout, int64_t ldg, const float* z, int64_t ldz, int64_t rows,
                             int32_t channels, const float* w, int64_t ldw, const int32_t* index1,
                             const int32_t* index2, int64_t ld_index, const int64_t* offsets, int64_t n_segments,
                             float scale, float* gz, int64_t ldgz, float* gsum, int64_t ldgs, float* gw, int64_t ldgw,
                             int32_t accumulate_gw, hipStream_t stream);
/* The angle -> bond sums over a line graph of fmd_nl_line_graph (its segment layouts: the bonds
 * bond_rows[0, short_offsets[n]), a bond's triplets as first bond the run [eto[b], eto[b+1]), as
 * second bond the same run through second_perm), a fixed grid striding over the real bonds /
 * triplets, every sum in triplet order. The reference's triplet gather + segment sums
 * (fastmd/models/matris/op/triton_weighted_segment_sum.py, triton_csr_segment_sum.py:433-479).
 * Forward: eps[b] += scale * sum over b's triplets k of silu(z3[k]) s_b s_b2 (s = geo column 6). */
int fmd_tb_bond_sum_f32(const float* z3, int64_t ldz, int32_t channels, const float* geo, const int64_t* short_offsets,
                        const int32_t* bond_rows, const int64_t* edge_triplet_offsets, const int32_t* line_graph,
                        int64_t n_atoms, int64_t t_cap, float scale, float* eps, int64_t lde, hipStream_t stream);
/* VJP per triplet: gz3[k] = scale geps[b1] s_b1 s_b2 silu'(z3[k]) (0 past the real triplets) and
 * the envelope terms gsw [t_cap, 2] = (gw s_b2, gw s_b1), gw = sum_c scale geps[b1] silu(z3[k]). */
int fmd_tb_triplet_bwd_f32(const float* geps, int64_t ldg, const float* z3, int64_t ldz, int32_t channels,
                           const float* geo, const int32_t* line_graph, const int64_t* pair_offsets, int64_t n_atoms,
                           int64_t t_cap, float scale, float* gz3, int64_t ldgz, float* gsw, hipStream_t stream);
/* VJP per bond: geps[b] += sum over b's triplets as first bond of ga3[k, 0:C] + as second bond of
 * ga3[k, C:2C] (ga3 = gz3 [W_b1; W_b2]^T); gs[b] = (or += with accumulate_gs) the same sums of
 * gsw[k, 0] and gsw[k, 1]. Rows that are no bond are not written. */
int fmd_tb_bond_reduce_f32(const float* ga3, int64_t lda, int32_t channels, const float* gsw,
                           const int64_t* short_offsets, const int32_t* bond_rows, const int64_t* edge_triplet_offsets,
                           const int32_t* second_perm, int64_t n_atoms, int64_t t_cap, float* geps, int64_t ldg,
                           float* gs, int32_t accumulate_gs, hipStream_t stream);
/* energy[i] = e0[elem[i]] + h[i] . wr, and its VJP gh[i] = (gE ? gE[i] : sign) * wr. */
int fmd_tb_readout_f32(const float* h, int64_t ldh, int32_t channels, const float* wr, const int32_t* elem,
                       const float* e0, int64_t n, float* energy, hipStream_t stream);
int fmd_tb_readout_bwd_f32(const float* gE, float sign, const float* wr, int32_t channels, int64_t n, float* gh,
                           int64_t ldgh, hipStream_t stream);
/* gvec [e_cap, 3] = gr u + (gu - (gu . u) u) / r per real row (0 on padding), gr = sum_n gef def +
 * gfc dfc + gs ds (each term nullable); with bond_flags (nullable) gu and gs are read on the flagged
 * rows only (the bonds of a line graph, the rows the three-body VJP writes). */
int fmd_tb_geometry_bwd_f32(const float* geo, const float* def, int32_t nb, const float* gef, int64_t ldgef,
                            const float* gu, int64_t ldgu, const float* gfc, const float* gs, const uint8_t* bond_flags,
                            const int64_t* n_edges, int64_t e_cap, float* gvec, hipStream_t stream);

/* The padded rows of a model-graph bucket workspace (gpu_md.py model_graph, cuda_graph.py:209-293
 * _PaddedEdgesWorkspace.update): rows [e_real, e_cap) of a ragged build copied into a fixed
 * capacity become the builder's far self-loops of atom (row - e_real) mod n_atoms with the pad
 * image, edge_reverse -1 (nullable). */
int fmd_nl_pad_rows(int32_t* edge_index, float* edge_image, int32_t* edge_reverse, int64_t e_real, int64_t e_cap,
                    int64_t n_atoms, int32_t pad_ix, int32_t pad_iy, int32_t pad_iz, hipStream_t stream);

/* Reverse edge of every real row e < min(E, e_cap): the row of (neighbour, centre, -image),
 * or -1 when it is not stored (overflowed build). Gives the sender-side CSR of the sorted
 * edge list (perm = reverse, off = edge_offsets), used by the deterministic VJPs. No
 * counterpart in the reference, which scatters with atomics instead
 * (triton_gather_cat.py:58-72). */
int fmd_nl_reverse(const int32_t* center, const int32_t* neighbor, const int32_t* images,
                   const int64_t* edge_offsets, int64_t n_atoms, int64_t e_cap, int32_t* reverse,
                   hipStream_t stream);

/* Window flag fold of one build (fixed_capacity_builder.py:430-455, _window_flags_kernel); with
 * `stats` (float64 [7], may be null) also the window's statistics after this build: (overflow,
 * edges, max triplets, max displacement, capacity overflow, max edges, max isolated), the one
 * buffer the host reads per window (whole_step_cuda_graph.py:353-356). A line-graph build passes
 * its triplet count (pair_offsets[n]) and t_cap: capacity overflow is then edges >= e_cap (no
 * padding pair), invalid pairs or triplets > t_cap, and window_max_triplets (nullable) keeps the
 * window's largest triplet count. */
int fmd_nl_window_flags(const int64_t* edge_count, const uint8_t* invalid_pairs, const uint8_t* overflow,
                        const int32_t* isolated, int64_t e_cap, int32_t check_isolated,
                        uint8_t* window_overflow, uint8_t* window_capacity_overflow,
                        int64_t* window_max_edges, int32_t* window_max_isolated,
                        const float* max_displacement, double* stats, const int64_t* triplet_count, int64_t t_cap,
                        int64_t* window_max_triplets, hipStream_t stream);

/* ----------------------------------------------------------------------------------------
 * (b) Gather-cat
 * -------------------------------------------------------------------------------------- */

/* out[e] = cat(part_0[e'], ..., part_{n-1}[e']) over n_parts <= 4 column blocks, where part k
 * reads row index_k[e * index_stride_k] of src_k (gathered) or row e (index_k null, aligned),
 * width w_k, row stride ld_k; out row stride ld_out. Per-part arrays are host arrays
 * (index_strides may be null: 1). Replaces aligned_gather_cat3/4
 * (triton_gather_cat.py:29-43,181-199,202-232,353-374) and the north-star form
 * gather_cat(x, src, dst, rbf) = cat(x[src], x[dst], rbf). Index arrays are int32. */
int fmd_gather_cat_f32(int32_t n_parts, const float* const* srcs, const int32_t* const* indices,
                       const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t rows,
                       float* out, int64_t ld_out, hipStream_t stream);

/* ----------------------------------------------------------------------------------------
 * (c) Deterministic CSR segment sums
 * -------------------------------------------------------------------------------------- */

/* out[s, :] = sum over terms t of  scale_t * sum_{j in [off_t[s], off_t[s+1]) ∩ [0, rows_t)}
 *             [w_t[r]*] v_t[r, col_t + :]   with r = perm_t ? perm_t[j] : j (r < 0 skipped)
 * for up to 2 terms, width `dim`, fixed summation order (deterministic, no atomics); the
 * per-term arrays (values, ld_values, col_offsets, weights, scales, perms, offs, rows) are
 * host arrays of n_terms entries (weights, scales, perms may be null: none, 1, identity).
 * `skip_segment` >= 0 writes 0 to that segment. accumulate != 0 adds into out.
 * Replaces csr_segment_sum (triton_csr_segment_sum.py:70-120,433-479) and the gather-cat VJP
 * scatters (triton_gather_cat.py:58-72) by two CSRs. */
int fmd_segsum_csr_f32(int32_t n_terms, const float* const* values, const int64_t* ld_values,
                       const int64_t* col_offsets, const float* const* weights, const float* scales,
                       const int32_t* const* perms, const int64_t* const* offs,
                       const int64_t* rows, int64_t num_segment, int64_t dim, int64_t skip_segment,
                       int32_t accumulate, float* out, int64_t ld_out, hipStream_t stream);

/* Transpose (VJP) of one term: for j in the run of s, r = perm ? perm[j] : j,
 *   gvalue[r] = gout[s] (* weight[r]),  gweight[r] = gout[s] * value[r];
 * rows of [0, n_rows) in no run (padding) get 0. skip_segment's rows get 0.
 * Replaces _csr_segsum_bwd_runs / _csr_segsum_bwd_rows (triton_csr_segment_sum.py:123-230). */
int fmd_segsum_csr_t_f32(const float* gout, int64_t ld_gout, const float* value, const float* weight,
                         int64_t ld_value, const int32_t* perm, const int64_t* off, int64_t num_segment,
                         int64_t n_rows, int64_t dim, int64_t skip_segment, float* gvalue,
                         float* gweight, hipStream_t stream);

/* ----------------------------------------------------------------------------------------
 * (d) Edge GEMM on MFMA
 * -------------------------------------------------------------------------------------- */

/* C[M,N] (ldc) = A[M,K] (lda) * op(B) (+ bias[N]) (+ C if accumulate), fp32 in/out.
 * b_layout 0: B is [N,K] (ldb), op(B) = B^T (F.linear weight); 1: B is [K,N] (ldb), op(B) = B.
 * epilogue 0: none, 1: SiLU. Large b_layout-0 GEMMs with K % 4 == 0 and 16-byte aligned
 * operands run as three bf16 planes per operand on the bf16 matrix cores (fp32-accurate, the
 * counterpart of the reference's 3xTF32); everything else on fp32 MFMA
 * (v_mfma_f32_32x32x2_f32). Replaces linear / linear_into / matmul
 * (triton_wide_gemm.py:482-553), whose 3xTF32 kernels decline K % 16 != 0 (:235) and fall back
 * to F.linear. */
int fmd_gemm_f32(const float* a, int64_t lda, const float* b, int64_t ldb, int32_t b_layout,
                 const float* bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                 int32_t accumulate, int32_t epilogue, hipStream_t stream);

/* Up to four independent fmd_gemm_f32 problems of one b_layout in one launch (arrays of length
 * count, problem g: C_g = [A_g | A2_g] op(B_g) (+ bias_g) (+ C_g if accumulate_g)). A2_g (may be
 * null, or the a2 array itself null) supplies K columns [ksplit_g, K_g) with row stride lda2_g;
 * ksplit_g % 32 == 0. Every problem runs the 64 x 64 fp32 MFMA tiles of fmd_gemm_f32 (same K
 * order); large groups with pre-split weights go to fmd_gemm_group_x3_planes_f32. Replaces several linear / matmul calls on independent operands
 * (triton_wide_gemm.py:482-553) with one launch: the node side of an interaction layer, whose
 * per-layer GEMMs are each too small to fill the chip. bias and accumulate may be null. */
int fmd_gemm_group_f32(int32_t count, const float* const* a, const int64_t* lda, const float* const* a2,
                       const int64_t* lda2, const int64_t* ksplit, const float* const* b, const int64_t* ldb,
                       int32_t b_layout, const float* const* bias, float* const* c, const int64_t* ldc,
                       const int64_t* m, const int64_t* n, const int64_t* k, const int32_t* accumulate,
                       int32_t epilogue, hipStream_t stream);

/* fmd_gemm_group_f32 with b_layout 0 and each weight given as its bf16 planes (fmd_split3_f32 of
 * the [N_g, K_g] weight, row stride ldb_g = 48 ceil(K_g / 16)): the split-plane product of
 * fmd_gemm_f32 (bitwise the same C), without splitting the weights again in every workgroup.
 * Tiles of 64 x 128 while the group has fewer than 768 tiles of 128 x 128. Conditions: A_g, A2_g
 * and the planes 16-byte aligned, lda_g, lda2_g, ksplit_g and K_g - ksplit_g multiples of 4,
 * ksplit_g a multiple of 16 when A2_g is set; FMD_EUNSUPPORTED otherwise (nothing launched).
 * Replaces the same linear / matmul calls as fmd_gemm_group_f32 (triton_wide_gemm.py:482-553). */
int fmd_gemm_group_x3_planes_f32(int32_t count, const float* const* a, const int64_t* lda,
                                 const float* const* a2, const int64_t* lda2, const int64_t* ksplit,
                                 const uint16_t* const* b_planes, const int64_t* ldb,
                                 const float* const* bias, float* const* c, const int64_t* ldc,
                                 const int64_t* m, const int64_t* n, const int64_t* k,
                                 const int32_t* accumulate, int32_t epilogue, hipStream_t stream);
/* fmd_gemm_group_x3_planes_f32 with a gathered row added to each output row: for a problem with
 * row_add[g] non-null, C[r, :] = (A B)[r, :] + row_add[g][row_index[g][r] * row_ld[g] + (0 .. n)]
 * (+ the old C when accumulate, then bias and the activation): the sum a launch on a C prefilled
 * with those rows and accumulate = 1 gives, bitwise, without the prefill's write and read (the
 * model's per-element residual and next-layer tables, indexed by element). row_add, row_index,
 * row_ld may be null (no row added anywhere). No reference counterpart: a fused epilogue of this
 * build's node side (the reference adds those terms in PyTorch). */
int fmd_gemm_group_x3_planes_rows_f32(int32_t count, const float* const* a, const int64_t* lda,
                                      const float* const* a2, const int64_t* lda2, const int64_t* ksplit,
                                      const uint16_t* const* b_planes, const int64_t* ldb, const float* const* bias,
                                      float* const* c, const int64_t* ldc, const int64_t* m, const int64_t* n,
                                      const int64_t* k, const int32_t* accumulate, const float* const* row_add,
                                      const int32_t* const* row_index, const int64_t* row_ld, int32_t epilogue_kind,
                                      hipStream_t stream);

/* fmd_gemm_group_f32 with b_layout 0 (B_g [N_g, K_g] K-contiguous) for groups too small to fill
 * the chip (small systems' node side): 16 x 16 output tiles, one workgroup each, whose four
 * waves multiply a contiguous quarter of the K slices of 32 each with fp32 MFMAs and add their
 * partial tiles in wave order (deterministic; not fmd_gemm_f32's K order, so not its bits).
 * Conditions: A_g, A2_g and B_g 16-byte aligned, lda_g, lda2_g and ldb_g multiples of 4,
 * ksplit_g a multiple of 32 when A2_g is set; FMD_EUNSUPPORTED otherwise (nothing launched).
 * Replaces the same linear / matmul calls as fmd_gemm_group_f32 (triton_wide_gemm.py:482-553). */
int fmd_gemm_group_ks_f32(int32_t count, const float* const* a, const int64_t* lda, const float* const* a2,
                          const int64_t* lda2, const int64_t* ksplit, const float* const* b, const int64_t* ldb,
                          const float* const* bias, float* const* c, const int64_t* ldc, const int64_t* m,
                          const int64_t* n, const int64_t* k, const int32_t* accumulate, int32_t epilogue,
                          hipStream_t stream);

/* C = [A | A2] op(B) (+ bias) (+ C if accumulate) as fmd_gemm_f32, with K cut into `splits` equal
 * slices (multiples of 32, none straddling ksplit, the width of A; A2 may be null) multiplied by
 * separate workgroups into workspace [splits, M, N] and then summed in slice order
 * (deterministic): the tall-K node GEMMs (K = 8C) that fmd_gemm_f32's tiles would leave to a few
 * hundred long-running workgroups. Replaces the reference's matmul (triton_wide_gemm.py:542-553)
 * for that shape. */
int fmd_gemm_splitk_f32(const float* a, int64_t lda, const float* a2, int64_t lda2, int64_t ksplit, const float* b,
                        int64_t ldb, int32_t b_layout, const float* bias, float* c, int64_t ldc, int64_t m, int64_t n,
                        int64_t k, int32_t accumulate, int32_t splits, float* workspace, hipStream_t stream);

/* The same K-split product in the split-plane form: B given as its bf16 planes (fmd_split3_f32
 * of the [N, K] weight, ldb = 48 ceil(K / 16)); split s (splits <= 4, K / splits a multiple of
 * 16 that does not straddle [a | a2]) multiplies its K slice as problem s of one grouped
 * split-plane launch into workspace [splits, M, N], then the slices are summed in order (+ bias)
 * (+ C). fp32-accurate (six bf16 plane products), deterministic. 16-byte aligned A rows with
 * lda % 4 == 0. Replaces the reference's matmul (triton_wide_gemm.py:542-553) for the tall-K node
 * GEMM of the MACE-like VJP. */
int fmd_gemm_splitk_x3_planes_f32(const float* a, int64_t lda, const float* a2, int64_t lda2, int64_t ksplit,
                                  const uint16_t* b_planes, int64_t ldb, const float* bias, float* c, int64_t ldc,
                                  int64_t m, int64_t n, int64_t k, int32_t accumulate, int32_t splits,
                                  float* workspace, hipStream_t stream);

/* C[M,N] = A[M,K] B[N,K]^T (+ bias) (+ C) with the gather-cat fused into the operand load:
 * A = cat(part_0, ..., part_{n-1}) over n_parts <= 3 column blocks, part p reading row
 * indices_p[r * index_strides_p] of srcs_p (or row r when indices_p is null), width widths_p,
 * row stride lds_p; K = sum of the widths; B [N, ldb] K-contiguous (b_layout 0 of fmd_gemm_f32).
 * Replaces the reference's edge-row pair aligned_gather_cat3 -> linear
 * (triton_gather_cat.py:181-199 feeding triton_wide_gemm.py:482-515): same C as
 * fmd_gather_cat_f32 followed by fmd_gemm_f32, without the [M, K] row matrix in memory.
 * fp32-accurate (three bf16 planes per operand, six MFMA products). row_add (optional, ld
 * ld_row_add >= N) adds row row_add_index[r * row_add_index_stride] (or row r) of row_add to
 * output row r before bias/accumulate/epilogue: a block of the gather-cat that depends only on
 * an index (the receiver's features) multiplied once per node instead of once per edge. Needs
 * 16-byte aligned sources with lds_p % 4 == 0, widths % 4 == 0 and every width but the last
 * % 16 == 0, b aligned with ldb % 4 == 0: otherwise FMD_EUNSUPPORTED (the caller gathers, then
 * multiplies). */
int fmd_gemm_gather_f32(int32_t n_parts, const float* const* srcs, const int32_t* const* indices,
                        const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                        const float* b, int64_t ldb, const float* row_add, const int32_t* row_add_index,
                        int64_t row_add_index_stride, int64_t ld_row_add, const float* bias, float* c,
                        int64_t ldc, int64_t n, int32_t accumulate, int32_t epilogue, hipStream_t stream);

/* The three bf16 planes of a float32 matrix src [rows, width] (row stride ld), slice-interleaved:
 * planes [rows][S][3][16] (bf16 as uint16, S = ceil(width / 16), 16-byte aligned), plane p of
 * columns [16 s, 16 s + 16) of row r at (r S + s) 48 + 16 p, with x = p0 + p1 + p2 exactly
 * (p0 = bf16(x), p1 = bf16(x - p0), p2 = bf16(x - p0 - p1), round to nearest even) and zeros past
 * the width. The operand format of fmd_gemm_x3_planes_f32. Counterpart of the reference's
 * once-per-weight-version operand split (_split_kernel / _split, triton_wide_gemm.py:12-15,
 * 131-199: hi/lo TF32 pairs there, three bf16 planes here). */
int fmd_split3_f32(const float* src, int64_t ld, int64_t rows, int32_t width, uint16_t* planes, hipStream_t stream);
/* fmd_gemm_gather_f32 with pre-split operands: B [N, K] as planes (fmd_split3_f32, ldb =
 * 48 ceil(K / 16)), and with a_planes the parts as planes too (srcs_p planes of width widths_p,
 * lds_p = 48 ceil(widths_p / 16); widths multiples of 8, all but the last of 16); a_planes 0: the
 * parts are fp32 as in fmd_gemm_gather_f32. Bitwise the same C as fmd_gemm_gather_f32 on the
 * unsplit operands (same planes, products and order), without the splitting arithmetic in the
 * GEMM: a weight is split once, a per-atom feature once per evaluation instead of once per output
 * tile, and a row's 16-k slice is one contiguous 96-byte read. Replaces the same reference calls
 * as fmd_gemm_gather_f32 (triton_gather_cat.py:181-199 feeding triton_wide_gemm.py:482-515).
 * FMD_EUNSUPPORTED when a layout condition fails. */
int fmd_gemm_x3_planes_f32(int32_t a_planes, int32_t n_parts, const void* const* srcs, const int32_t* const* indices,
                           const int64_t* index_strides, const int64_t* lds, const int32_t* widths, int64_t m,
                           const uint16_t* b_planes, int64_t ldb, int64_t k, const float* row_add,
                           const int32_t* row_add_index, int64_t row_add_index_stride, int64_t ld_row_add,
                           const float* bias, float* c, int64_t ldc, int64_t n, int32_t accumulate,
                           int32_t epilogue, hipStream_t stream);

/* As fmd_gemm_f32 with bf16 operands (uint16 storage), fp32 accumulate and fp32 output, on
 * v_mfma_f32_32x32x16_bf16. Not in the reference (which has no bf16 GEMM on this path). */
int fmd_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int32_t b_layout,
                  const float* bias, float* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                  int32_t accumulate, int32_t epilogue, hipStream_t stream);

/* ----------------------------------------------------------------------------------------
 * (e) Nose-Hoover chain velocity Verlet (ASE NoseHooverChainNVT), float64 state
 * -------------------------------------------------------------------------------------- */

/* consts layout (float64): [dt, dt/2, kT, 3N*kT, 3 x (delta, delta/2, -(delta/4), -delta),
 * Q[tchain], 1/Q[tchain]] (gpu_nhc.py:113-133,273-275). Up to 4096 atoms one workgroup runs a
 * half step with every ke2 = sum(p^2/m) recomputed (ASE's order); beyond, see fmd_nhc_work_size.
 * pre: NHC(dt/2); p += dt/2 * F (cached forces, float64; f32_kick: the float32 product of
 * NumPy NEP 50); q += dt * p / m. Replaces _nhc_pre_force_kernel (gpu_nhc.py:359-391). */
int fmd_nhc_pre_force(double* q, double* p, const double* f, const double* masses, double* eta,
                      double* p_eta, const double* consts, int64_t n_atoms, int32_t tchain,
                      int32_t tloop, int32_t f32_kick, double* work, hipStream_t stream);

/* post: p += dt/2 * F_in; NHC(dt/2); cache F_in as float64 in f_cache; copy the energy.
 * f_in_is_f64 selects float32/float64 forces, e_kind 0: no energy, 1: float32, 2: float64.
 * Replaces _nhc_post_force_kernel (gpu_nhc.py:393-425). */
int fmd_nhc_post_force(double* p, const void* f_in, int32_t f_in_is_f64, double* f_cache,
                       const double* masses, double* eta, double* p_eta, const double* consts,
                       const void* e_in, int32_t e_kind, double* e_out, int64_t n_atoms,
                       int32_t tchain, int32_t tloop, int32_t f32_kick, double* work, hipStream_t stream);

/* fmd_nhc_post_force of step n then fmd_nhc_pre_force of step n + 1 (the pre half's kick with the
 * forces just cached in f_cache), as one launch (multi-block: three instead of four); the same
 * state, bit for bit. Consecutive steps of a window (whole_step_cuda_graph.py:56-736 runs
 * _nhc_post_force_kernel and _nhc_pre_force_kernel back to back there, gpu_nhc.py:359-425). */
int fmd_nhc_post_pre(double* q, double* p, const void* f_in, int32_t f_in_is_f64, double* f_cache,
                     const double* masses, double* eta, double* p_eta, const double* consts, const void* e_in,
                     int32_t e_kind, double* e_out, int64_t n_atoms, int32_t tchain, int32_t tloop, int32_t f32_kick,
                     double* work, hipStream_t stream);

/* float64 elements of the `work` buffer the NHC entry points need for n_atoms (systems of more
 * than 4096 atoms run the multi-block path: per-block partial sums with the chain half step run
 * by the last workgroup to finish (a completion counter in the last slot of `work`, which must be
 * zero when the buffer is first used and is left at zero by every call), then an elementwise
 * pass: two launches per half step; after each momentum scaling ke2 is updated as ke2 * s^2,
 * the reference's "scaled" update of gpu_nhc.py:520-706, instead of a fresh reduction). May be
 * null below. */
int64_t fmd_nhc_work_size(int64_t n_atoms);

/* ----------------------------------------------------------------------------------------
 * Small deterministic reductions used around the step
 * -------------------------------------------------------------------------------------- */

/* out[0] = sum_{i<n} (double)x[i] in a fixed order (x float32 if x_is_f64 == 0). The FP64
 * energy sum of EnergyDerivative (fastmd/engine/energy_derivative.py:131-133). */
int fmd_sum_f64(const void* x, int32_t x_is_f64, int64_t n, double* out, hipStream_t stream);

/* ----------------------------------------------------------------------------------------
 * Model kernels (the MACE-like interaction and the Morse pair potential of the benchmark
 * configurations). Edge rows are the real rows [0, min(*n_edges, e_cap)) of the builder's
 * sorted list (n_edges read on the device); node sums walk the centre CSR (edge_offsets),
 * sender sums the reverse-edge CSR. The reference's model arithmetic is third-party
 * (mace-torch, wrapped by fastmd/models/mace.py:356-388); these kernels implement this
 * build's own MACE-like model, specified in fastmd_amd/models/mace_like.py.
 * -------------------------------------------------------------------------------------- */

/* geo[e] = (u, r, fcut, dfcut, 0, 0) [E,8]; ef[e,n] = Bessel_n(r) fcut(r), def = d ef / dr [E,nb].  * system_of (null: one cell): the system of each atom for a union of systems, cell then a
 * [systems, 3, 3] table and each edge's image taken in its centre's cell. */
int fmd_edge_geometry_f32(const float* positions, const float* cell, const int32_t* system_of,
                          const int32_t* edge_index, const float* edge_image, const int64_t* n_edges, int64_t e_cap,
                          float rc, int32_t nb, float* geo, float* ef, float* def, hipStream_t stream);
/* gvec[e] = dE/dvec from dE/def (up to two sources, row strides ld0/ld1) and dE/d(u, fcut) (ggeo [E,4]). */
int fmd_edge_geometry_bwd_f32(const float* geo, const float* def, int32_t nb, const float* gef0, int64_t ld0,
                              const float* gef1, int64_t ld1, const float* ggeo, const int64_t* n_edges,
                              int64_t e_cap, float* gvec, hipStream_t stream);
/* A0[i], A1[i] = inv_avg * sum over the rows of centre i of the messages. z [E, W] holds the
 * edge pre-activation blocks a | b | c | d (W = 4C) when h1 is given; with h1 null (zero vector
 * features, where c and d meet only zeros) z holds a | b only (W = 2C). The pre-activations are
 * z[e] + zq[i] when zq ([N, W], the receiver block of the edge GEMM formed once per atom) is
 * given, else z[e]. z, zq, h0, h1, A0, A1 start on 16-byte boundaries (8 for C = 64), geo on 16.
 * Every row of a centre is taken by a half-wave (C / 32 channels per lane).
 * order (may be null): a permutation of the atoms, the order in which the waves take them (each
 * atom's results are the same in any order; a spatial order keeps the neighbours' rows a wave
 * gathers in the L2 of its XCD).
 * z_per_node = 1 (node-factored pre-activation): z is P = h0 W1[:C] per atom ([N, W]) and zq is
 * Q = h0 W1[C:2C] ([N, W], required); row e of centre i and sender j takes
 * (P[j] + sum_n ef[e, n] w1ef[n, :W]) + Q[i], with ef [E, nb] the radial basis rows (16-byte
 * aligned) and w1ef [nb, 4C] the radial rows of W1 (nb <= 16): no [E, W] array exists.
 * waves_per_atom (1 or 4): the rows of an atom are taken by one wave, or split over four waves
 * whose per-atom sums are added in wave order (for small systems; a different association of
 * the sums, so the choice belongs to the system size, not to the call). */
int fmd_mace_message_f32(const float* z, const float* zq, const float* geo, const int32_t* edge_index,
                         const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap, int64_t n_atoms,
                         const int32_t* order, int32_t channels, const float* h0, const float* h1, float inv_avg,
                         float* A0, float* A1, int32_t z_per_node, const float* ef, const float* w1ef, int32_t nb,
                         int32_t waves_per_atom, hipStream_t stream);
/* VJP of fmd_mace_message_f32 (z, zq and the width W as there): gz [E,W] (may be null), gzsum
 * [N,W] (may be null: the sum of gz over each centre's rows, in row order), gzsum_src [N,W] (may
 * be null: the sum of gz over the rows whose sender is the node, over the reverse CSR, without gz
 * in memory), ggeo [E,4] (= or +=), with w1ef ([nb, 4C], the radial rows of the edge GEMM weight;
 * its first W columns enter) also gef[e] = gz[e] @ w1ef[:, :W]^T [E,nb], and if gh0: the
 * sender-side gh0/gh1 over the reverse CSR (accumulate_h bit 0: gh0 +=, bit 1: gh1 +=; otherwise
 * =). The gather-cat row gradient's node blocks are then gzsum_src @ W1[:C]^T (sender) and
 * gzsum @ W1[C:2C]^T (receiver), node GEMMs (by linearity the same sums as gz @ W1^T summed per
 * sender / receiver). Alignment as there (gA0, gA1, gz, gzsum, gzsum_src, gh0, gh1 like h0; ggeo
 * on 16 bytes). z_per_node = 1: z, zq as in the node-factored forward (P, Q), with its ef; w1ef
 * is then required and gz must be null. accumulate_h bit 2 (4): launch the sender-side kernel
 * only (its arguments as in the full call; the edge side having run in an earlier call), so
 * that each side can be timed on its own. waves_per_atom as in the forward. */
int fmd_mace_message_bwd_f32(const float* z, const float* zq, const float* geo, const int32_t* edge_index,
                             const int32_t* reverse,
                             const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap, int64_t n_atoms,
                             const int32_t* order, int32_t channels, const float* h0, const float* h1,
                             const float* gA0, const float* gA1, float inv_avg, float* gz, float* gzsum,
                             float* gzsum_src, float* ggeo,
                             int32_t accumulate_geo, float* gh0, float* gh1, int32_t accumulate_h, const float* w1ef,
                             int32_t nb, float* gef, int32_t z_per_node, const float* ef, int32_t waves_per_atom,
                             hipStream_t stream);
/* The node side of one interaction layer fused per 32-atom tile (one launch instead of six),
 * fp32-accurate on the bf16 matrix cores: P0 = A0 Wm0, P1_x = A1_x Wm1, the symmetric
 * contraction (B0, B1: workspace, [N,C] and [N,3,C]), h0n = B0 Wo0 + h0 Wsc0, h1n_x = B1_x Wo1
 * (h1n null: last layer, no vector output). Weights laid out [columns, K] K-contiguous:
 * wm0t = Wm0^T, wm1t = Wm1^T [C, C]; wout0 = [Wo0; Wsc0]^T, wout1 = [Wo1; 0]^T [C, 2C]. Same
 * results as fmd_gemm_f32 + fmd_mace_symcon_f32 chains to fp32 rounding. No reference
 * counterpart: it replaces the model's node-side chain (mace.py:386 runs mace-torch there). */
int fmd_mace_node_fwd_f32(const float* A0, const float* A1, const float* h0, const int32_t* elem, const float* wm0t,
                          const float* wm1t, const float* Wc, const float* Wd, const float* wout0, const float* wout1,
                          int64_t n_atoms, int32_t channels, float* P0, float* P1, float* B0, float* B1, float* h0n,
                          float* h1n, hipStream_t stream);
/* VJP of fmd_mace_node_fwd_f32 per 32-atom tile: gB0 = g0 Wo0^T, gB1_x = g1_x Wo1^T (g1 null: no
 * vector input gradient), g_in0 (=, or += when accumulate_in0; null: not formed) = g0 Wsc0^T,
 * the contraction VJP (gP0, gP1), gA0 = gP0 Wm0^T, gA1_x = gP1_x Wm1^T. wo0st = [Wo0; Wsc0]
 * [2C, C], wo1st = [Wo1; 0] [2C, C], wm0 = Wm0, wm1 = Wm1 [C, C] (row-major [in, out] as stored). */
int fmd_mace_node_bwd_f32(const float* g0, const float* g1, const float* P0, const float* P1, const int32_t* elem,
                          const float* wo0st, const float* wo1st, const float* Wc, const float* Wd, const float* wm0,
                          const float* wm1, int64_t n_atoms, int32_t channels, float* gB0, float* gB1, float* gin0,
                          int32_t accumulate_in0, float* gP0, float* gP1, float* gA0, float* gA1, hipStream_t stream);
/* The first half of a layer's node side for small systems, one launch: P0 = A0 Wm0, P1_x = A1_x
 * Wm1 (A1 [N,3,C]) and the symmetric contraction B0, B1 (B1 null: last layer, no vector output)
 * of every (atom, channel), P0 and P1 written too (the VJP reads them). A workgroup takes 16 atoms
 * x 16 channels: one wave per row kind (the scalar row, the vector rows x, y, z) over all of K =
 * C with fp32 MFMAs, the contraction from the four tiles in LDS. wm0t = Wm0^T, wm1t = Wm1^T [C, C]
 * (K-contiguous), 16-byte aligned like A0, A1; channels a multiple of 32. Same results as
 * fmd_gemm_group_ks_f32 + fmd_mace_symcon_f32 up to the K order of the products. No reference
 * counterpart: it replaces two launches of the model's node-side chain (mace.py:386 runs
 * mace-torch there). */
int fmd_mace_mix_symcon_f32(const float* A0, const float* A1, const float* wm0t, const float* wm1t,
                            const int32_t* elem, const float* Wc, const float* Wd, int64_t n_atoms, int32_t channels,
                            float* P0, float* P1, float* B0, float* B1, hipStream_t stream);
/* The VJP's matching half, one launch: gB0 = g0 wb0^T (g0 [N, k0], wb0 [C, k0]; k0 = C with
 * wb0 = Wo0, or the readout width with the merged last layer's weight), gB1_x = g1_x wb1^T (g1
 * [N,3,C], wb1 = Wo1 [C, C]; g1 null: no vector output gradient) and the contraction's VJP from
 * them -> gP0 [N,C], gP1 [N,3,C] (gB0 and gB1 are never written). Layout and conditions as
 * fmd_mace_mix_symcon_f32, k0 a multiple of 4. No reference counterpart (see there). */
int fmd_mace_mix_symcon_bwd_f32(const float* g0, int64_t k0, const float* wb0, const float* g1, const float* wb1,
                                const float* P0, const float* P1, const int32_t* elem, const float* Wc,
                                const float* Wd, int64_t n_atoms, int32_t channels, float* gP0, float* gP1,
                                hipStream_t stream);
/* Symmetric contraction (correlation 3, L <= 1) and its VJP. */
int fmd_mace_symcon_f32(const float* P0, const float* P1, const int32_t* elem, const float* Wc, const float* Wd,
                        int64_t n_atoms, int32_t channels, float* B0, float* B1, hipStream_t stream);
int fmd_mace_symcon_bwd_f32(const float* P0, const float* P1, const int32_t* elem, const float* Wc, const float* Wd,
                            const float* gB0, const float* gB1, int64_t n_atoms, int32_t channels, float* gP0,
                            float* gP1, hipStream_t stream);
/* Node energies E_i = E0[elem] + scale (ha . wr1 + sum_k silu(y_k) wr2b_k) + shift, and the VJP
 * (gE null: dE/dE_i = 1 for every row). */
int fmd_mace_energy_f32(const float* ha, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                        int32_t hidden, const int32_t* elem, const float* e0, float scale, float shift,
                        int64_t n_atoms, float* energy, hipStream_t stream);
int fmd_mace_energy_bwd_f32(const float* gE, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                            int32_t hidden, float scale, int64_t n_atoms, float* gha, float* gy, hipStream_t stream);
/* fmd_mace_energy_f32 together with fmd_mace_energy_bwd_f32's gha and gy for a null gE, in one
 * launch (the explicit force path of EnergyDerivative, energy_derivative.py:110-140, whose seed is
 * dE/dE_i = 1). total (may be null) [1] f64: also the sum of the n_atoms energies, bitwise
 * fmd_sum_f64's, formed by the last workgroup to finish; counter: a uint32 that is zero before
 * the first call and that the call leaves at zero (calls sharing one counter must not overlap). */
int fmd_mace_energy_grad_f32(const float* ha, const float* wr1, const float* y, const float* wr2b, int32_t channels,
                             int32_t hidden, const int32_t* elem, const float* e0, float scale, float shift,
                             int64_t n_atoms, float* energy, float* gha, float* gy, double* total,
                             uint32_t* counter, hipStream_t stream);
/* h0[i] = table[elem[i]]. */
int fmd_embed_f32(const int32_t* elem, const float* table, int64_t n_atoms, int32_t channels, float* h0,
                  hipStream_t stream);
/* Up to eight per-element tables gathered in one launch: outs[g][i, :] = tables[g][elem[i], :]
 * ([n_atoms, widths[g]] each; widths a multiple of 4, every pointer 16-byte aligned): the first
 * layer's per-element rows (embedding, node-factored pre-activation blocks, residual tables). */
int fmd_embed_rows_f32(const int32_t* elem, int64_t n_atoms, int32_t count, const float* const* tables,
                       const int32_t* widths, float* const* outs, hipStream_t stream);
/* fmd_edge_geometry_f32 and fmd_embed_rows_f32 (the same arguments, the same results) in one
 * launch: the two independent passes that open a force evaluation. No reference counterpart: it
 * saves a launch where a step is launch-bound (small systems). */
int fmd_edge_geometry_embed_f32(const float* positions, const float* cell, const int32_t* system_of,
                                const int32_t* edge_index, const float* edge_image, const int64_t* n_edges,
                                int64_t e_cap, float rc, int32_t nb, float* geo, float* ef, float* def,
                                const int32_t* elem, int64_t n_atoms, int32_t count, const float* const* tables,
                                const int32_t* widths, float* const* outs, hipStream_t stream);
/* Morse pair potential (shifted to 0 at rc): E_i = 1/2 sum V(r_e) over the rows of centre i,
 * dvdr[e] = V'(r_e); VJP gvec[e] = 1/2 gE[centre] V'(r) u. */
int fmd_morse_f32(const float* geo, const int64_t* edge_offsets, const int64_t* n_edges, int64_t e_cap,
                  int64_t n_atoms, float D, float a, float r0, float rc, float vshift, float* energy, float* dvdr,
                  hipStream_t stream);
int fmd_morse_bwd_f32(const float* geo, const float* dvdr, const int32_t* edge_index, const float* gE,
                      const int64_t* n_edges, int64_t e_cap, float* gvec, hipStream_t stream);

/* Stress of the engine-owned derivative (fastmd/engine/energy_derivative.py:110-140: a symmetric
 * strain of positions and cell, stress = dE/d(strain) / |det cell|) from the edge-vector
 * gradient a model's VJP forms: strain moves every edge vector as v -> v (I + S), so
 * dE/dS = sum_e v_e (x) gvec_e over the real rows (v = u r from the geometry rows geo [e_cap, 8]),
 * symmetrised. stress [3, 3] float32, row-major; cell [3, 3] float32 (the unstrained cell);
 * work: fmd_edge_virial_work_size() float64 elements. Float64 sums in a fixed order. */
int64_t fmd_edge_virial_work_size(void);
int fmd_edge_stress_f32(const float* geo, const float* gvec, const int64_t* n_edges, int64_t e_cap, const float* cell,
                        double* work, float* stress, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTMD_HIP_H */
