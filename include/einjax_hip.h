/*
 * einjax_hip.h -- C ABI of the MI355X (gfx950) tensor-relational sparse-einsum path.
 *
 * The reference runs this path as host NumPy plus one jnp.einsum call
 * (execution/sparse_dispatch.py:226-297).  This library replaces its phases
 * with HIP kernels behind plain C entry points:
 *
 *   tiling        ej_bucket_dense_count / ej_bucket_dense_fill,
 *                 ej_bucket_coo_count / ej_bucket_coo_fill
 *                 (replace SparseTensor.to_relation, tensor/sparse.py:160-219)
 *   COO ingest    ej_extract_coo_count / ej_extract_coo_fill
 *                 (replaces _extract_coo for dense input, tensor/sparse.py:234-270)
 *   statistics    ej_scheme_stats_dense / ej_scheme_stats_coo
 *                 (replace SparseTensor._compute_sparsity_metrics,
 *                  tensor/sparse.py:124-158, over BaseTensor's tile shapes,
 *                  tensor/base.py:39-49)
 *   join          ej_join_count / ej_join_fill
 *                 (replaces coordinate_join, execution/sparse_dispatch.py:29-82;
 *                  coordinate_join_hash / coordinate_join_sorted,
 *                  kernels/pallas_gather.py:19-76 / :79-174)
 *   output coords ej_output_coords
 *                 (replaces _compute_output_coords, execution/sparse_dispatch.py:174-223)
 *   segment plan  ej_segment_count / ej_segment_fill
 *                 (the grouping half of segment_sum, execution/sparse_dispatch.py:155-162)
 *   gather        ej_gather_tiles
 *                 (replaces lhs_values[lhs_indices], execution/sparse_dispatch.py:118-119)
 *   tile einsum   ej_einsum_describe / ej_pair_einsum / ej_segment_einsum
 *                 (replaces jnp.einsum(_add_batch_dim(kernel_string)),
 *                  execution/sparse_dispatch.py:121-126)
 *   queued step   ej_join_count_async / ej_segment_count_async /
 *                 ej_pair_plan_async (both counts in one call) /
 *                 ej_segment_fill_async / ej_segment_einsum_async
 *                 (+ ej_segment_einsum_group for the plan's run order)
 *                 (the same phases with the counts kept on the device, so a
 *                  caller can queue a whole execute_sparse,
 *                  execution/sparse_dispatch.py:226-297, without waiting)
 *   segment sum   ej_segment_sum
 *                 (the accumulation half of segment_sum, execution/sparse_dispatch.py:164-171)
 *   backward      ej_index_plan / ej_pair_einsum_vjp
 *                 (replace sparse_einsum_raw's backward, autodiff/custom_vjp.py:254-275)
 *
 * Conventions
 *   - Every pointer argument named *coords, *values, *_idx, *keys, perm,
 *     seg_*, out*, dense, indices, tiles, idx, offsets, grad_* and workspace
 *     is a DEVICE pointer.
 *     Small descriptor arrays (dims, radices, shapes, tile_shapes, agg_*),
 *     the scalar outputs n_pairs, n_segments, n_tiles, nnz and the
 *     statistics num_tuples / value_count are HOST pointers; `counts` of the
 *     *_async functions is PINNED host memory (hipHostMalloc).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 *     Functions whose name ends in _count, and the ej_scheme_stats_*
 *     functions, synchronize `stream` because they return data-dependent
 *     values to the host; every other function,
 *     including the *_count_async forms, is asynchronous.
 *   - A *_count call leaves its state in the caller's workspace; the matching
 *     *_fill call must receive the same workspace, unmodified.
 *   - Return value: EJ_OK (0) or a negative EJ_E_* status.  ej_last_error()
 *     returns a thread-local message for the last failing call.
 *   - No global mutable state: calls on different streams with different
 *     workspaces may run concurrently.
 *   - Coordinates are int32, row-major [n, ncols].  Pair indices are int64,
 *     as the reference returns them.  Values are EJ_F32 or EJ_BF16.  Tile
 *     einsums accumulate in fp32 and write fp32, or bf16 when the operands
 *     are bf16 and the descriptor's out_dtype asks for it: the reference's
 *     jnp.einsum returns the operands' dtype (sparse_dispatch.py:125) and its
 *     segment sum keeps it (:165); here a bf16 result is rounded once, from
 *     the finished fp32 sum.
 */
#ifndef EINJAX_HIP_H
#define EINJAX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EJ_ABI_VERSION 14

#define EJ_OK 0
#define EJ_E_INVAL (-1)       /* bad argument (shape, null pointer, bad string) */
#define EJ_E_CAPACITY (-2)    /* output buffer smaller than the counted size */
#define EJ_E_HIP (-3)         /* HIP runtime error */
#define EJ_E_UNSUPPORTED (-4) /* valid request this build does not implement */
#define EJ_E_RANGE (-5)       /* a coordinate lies outside its declared grid */

#define EJ_F32 0
#define EJ_BF16 1
#define EJ_F64 2 /* tiling, COO ingest, to_dense and ej_segment_sum */
#define EJ_I32 3 /* integer tile einsums (ej_pair_einsum, ej_segment_einsum) and ej_segment_sum */
#define EJ_I64 4 /* ej_segment_sum */
#define EJ_F16 5 /* ej_segment_sum */

/* Pair orders of the join.  With n_keys == 0 both give the cross product in
 * lhs-major order (sparse_dispatch.py:53-59, pallas_gather.py:50-54). */
#define EJ_ORDER_PROBE 0  /* hash join order: rhs index ascending, then lhs
                             index ascending (sparse_dispatch.py:65-80) */
#define EJ_ORDER_SORTED 1 /* sort-merge order: key ascending, then lhs-major
                             nested product of the stably sorted key groups
                             (pallas_gather.py:130-172) */

#define EJ_MAX_DIMS 8   /* tile / coordinate rank limit */
#define EJ_MAX_KEYS 8   /* join keys and output dims */
#define EJ_MAX_LABELS 8 /* distinct labels per group in a tile einsum */

typedef void *ej_stream_t; /* hipStream_t */

/* Canonical form of a binary tile einsum "lhs,rhs->out" (both operands, one
 * output; the reference passes exactly two operands, sparse_dispatch.py:125).
 * Produced by ej_einsum_describe; treat it as opaque input to the einsum
 * entry points.  Strides are in elements of a row-major tile. */
typedef struct ej_einsum_desc {
  int32_t n_out;                    /* output labels (output tile rank) */
  int32_t n_red;                    /* contracted labels */
  int64_t out_ext[EJ_MAX_LABELS];   /* extent of each output label */
  int64_t out_a[EJ_MAX_LABELS];     /* lhs stride of each output label (0 if absent) */
  int64_t out_b[EJ_MAX_LABELS];     /* rhs stride of each output label (0 if absent) */
  int64_t red_ext[EJ_MAX_LABELS];   /* extent of each contracted label */
  int64_t red_a[EJ_MAX_LABELS];     /* lhs stride of each contracted label (0 if absent) */
  int64_t red_b[EJ_MAX_LABELS];     /* rhs stride of each contracted label (0 if absent) */
  int64_t a_elems, b_elems, c_elems; /* elements per lhs / rhs / output tile */
  /* GEMM form (valid when is_gemm == 1): C[b][m][n] = sum_k A[b][m][k] B[b][k][n] */
  int32_t is_gemm;
  /* Scheduling hint set by the caller (ej_einsum_describe writes 0): the
   * output segments come in aligned runs of this many consecutive segments
   * that contract the same lhs tiles in the same order, as an lhs row does
   * against a dense rhs.  The segment einsum then computes up to that many
   * segments per workgroup, reading each lhs tile once for all of them.  A
   * wrong hint costs speed, never correctness: each workgroup checks its
   * segments and falls back to pair-by-pair accumulation. */
  int32_t seg_group;
  int64_t batch, m, n, k;
  int64_t a_sb, a_sm, a_sk;
  int64_t b_sb, b_sk, b_sn;
  int64_t c_sb, c_sm, c_sn;
  /* Output dtype, set by the caller (ej_einsum_describe writes EJ_F32):
   * EJ_F32, or EJ_BF16 with bf16 operands (fp32 sums rounded once), or
   * EJ_I32 with (and only with) EJ_I32 operands. */
  int32_t out_dtype;
  int32_t reserved;
} ej_einsum_desc;

/* ---- diagnostics ------------------------------------------------------- */
int ej_version(void);
const char *ej_last_error(void);

/* ---- tile einsum description ------------------------------------------- */
/* Parses `kernel_string` (e.g. "ij,jk->ik") against the two tile shapes.
 * Label extents come from the tile shapes; a label whose extent differs
 * between the operands, an output label absent from both inputs, a repeated
 * output label, a missing "->" or a third operand give EJ_E_INVAL
 * (reference: _add_batch_dim raises without "->", sparse_dispatch.py:494-495;
 * _infer_output_tile_shape raises KeyError for an unknown output label, :544). */
int ej_einsum_describe(const char *kernel_string, const int64_t *lhs_tile, int32_t lhs_ndim,
                       const int64_t *rhs_tile, int32_t rhs_ndim, ej_einsum_desc *desc);

/* ---- join (reference: coordinate_join, sparse_dispatch.py:29-82) -------- */
/* radices[i] bounds key column i on both sides: 0 <= coord < radices[i].
 * A coordinate outside that range gives EJ_E_RANGE. */
int ej_join_workspace_size(int64_t n_lhs, int64_t n_rhs, int32_t order, size_t *bytes);
int ej_join_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                  const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols, int32_t n_keys,
                  const int32_t *lhs_dims, const int32_t *rhs_dims, const int64_t *radices,
                  int32_t order, void *workspace, size_t workspace_bytes, int64_t *n_pairs,
                  ej_stream_t stream);
/* Writes the n_pairs matched pairs counted by ej_join_count.  capacity is
 * the length of lhs_idx / rhs_idx; capacity < n_pairs gives EJ_E_CAPACITY.
 * Writes are clipped to the count stored in the workspace. */
int ej_join_fill(int64_t n_lhs, int64_t n_rhs, int32_t n_keys, int32_t order,
                 const void *workspace, size_t workspace_bytes, int64_t n_pairs,
                 int64_t *lhs_idx, int64_t *rhs_idx, int64_t capacity, ej_stream_t stream);

/* Asynchronous form of ej_join_count.  No counterpart in the reference, whose
 * join runs on the host inside execute_sparse (sparse_dispatch.py:226-297);
 * it lets a caller queue the whole sparse einsum without waiting for the
 * pair count.  Enqueues the count on `stream` and copies, in stream order,
 * counts[0] = P and counts[1] = a range flag (nonzero: a join-key coordinate
 * lies outside [0, radix), what ej_join_count reports as EJ_E_RANGE) to
 * `counts`, host memory allocated pinned, valid once the stream has passed
 * this call.  P also stays on the device as the first int64 of the
 * workspace: ej_join_fill called with n_pairs = capacity = any bound clips
 * its writes to it, and ej_segment_count_async takes it as n_pairs_dev. */
int ej_join_count_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                        const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                        int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                        const int64_t *radices, int32_t order, void *workspace,
                        size_t workspace_bytes, int64_t *counts, ej_stream_t stream);

/* ---- output coordinates (reference: _compute_output_coords, :174-223) --- */
/* out[p][d] = (agg_src[d] == 0 ? lhs : rhs).coords[idx[p]][agg_dim[d]];
 * a pair whose index lies outside [0, n_lhs) or [0, n_rhs) gets -1 in every
 * column. */
int ej_output_coords(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                     const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                     const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                     int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim, int32_t *out,
                     ej_stream_t stream);

/* ---- coordinate ranges -------------------------------------------------- */
/* Per-column minimum and maximum of int32 coordinates [n, ncols]:
 * lo_hi[2c] = min, lo_hi[2c+1] = max (HOST output; synchronizes `stream`).
 * n == 0 gives min 0, max -1.  workspace: device, >= 8 * ncols bytes.
 * Used to size key radices for bare coordinate arrays, which the reference
 * accepts without grid metadata (segment_sum, sparse_dispatch.py:129-132;
 * coordinate_join_hash / _sorted, pallas_gather.py:19-23, :79-83). */
int ej_coords_range(const int32_t *coords, int64_t n, int32_t ncols, int32_t *lo_hi,
                    void *workspace, size_t workspace_bytes, ej_stream_t stream);

/* ---- segment plan (reference: segment_sum grouping, :155-162) ----------- */
/* Groups the pairs by output coordinate.  Segment u is the u-th distinct
 * output coordinate in ascending lexicographic order (the reference's
 * sorted(coord_keys)); its pairs are perm[seg_offsets[u] .. seg_offsets[u+1])
 * in ascending pair index (the reference's accumulation order).
 * radices[d] bounds output dimension d.  Requires n_pairs < 2^31.  A pair
 * index outside [0, n_lhs) / [0, n_rhs) or an output coordinate outside its
 * radix gives EJ_E_RANGE. */
int ej_segment_workspace_size(int64_t n_pairs, size_t *bytes);
int ej_segment_count(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                     const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                     const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                     int32_t n_out, const int32_t *agg_src, const int32_t *agg_dim,
                     const int64_t *radices, void *workspace, size_t workspace_bytes,
                     int64_t *n_segments, ej_stream_t stream);
/* out_coords int32 [n_segments, n_out]; seg_offsets int32 [n_segments + 1];
 * perm int32 [n_pairs]; seg_ids int32 [n_pairs] (may be NULL): the segment of
 * each pair in pair order.  capacity bounds n_segments.  n_pairs and
 * n_segments must be the values of the matching ej_segment_count; writes are
 * clipped to both. */
int ej_segment_fill(int64_t n_pairs, int64_t n_segments, int32_t n_out, const int64_t *radices,
                    const void *workspace, size_t workspace_bytes, int32_t *out_coords,
                    int32_t *seg_offsets, int32_t *perm, int32_t *seg_ids, int64_t capacity,
                    ej_stream_t stream);

/* Asynchronous forms of the segment plan (no counterpart in the reference,
 * whose grouping runs on the host; see ej_join_count_async).
 * ej_segment_count_async: n_pairs bounds lhs_idx / rhs_idx (and sizes the
 * workspace); n_pairs_dev (may be NULL) is the live pair count on the
 * device, e.g. the first int64 of a join workspace after
 * ej_join_count_async.  counts[0] = U and counts[1] = a range flag are
 * copied in stream order to pinned host memory; U also stays on the device
 * as the first int64 of the workspace.
 * ej_segment_fill_async: ej_segment_fill on those device-side counts;
 * capacity bounds out_coords [capacity, n_out] and seg_offsets
 * [capacity + 1]; if U exceeds it nothing is written (the caller sees U in
 * counts[0]). */
int ej_segment_count_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                           const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                           const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs,
                           const int64_t *n_pairs_dev, int32_t n_out, const int32_t *agg_src,
                           const int32_t *agg_dim, const int64_t *radices, void *workspace,
                           size_t workspace_bytes, int64_t *counts, ej_stream_t stream);
int ej_segment_fill_async(int64_t n_pairs, int32_t n_out, const int64_t *radices,
                          const void *workspace, size_t workspace_bytes, int32_t *out_coords,
                          int32_t *seg_offsets, int32_t *perm, int32_t *seg_ids,
                          int64_t capacity, ej_stream_t stream);

/* ej_join_count_async (EJ_ORDER_PROBE), ej_join_fill, ej_segment_count_async
 * and ej_segment_fill_async in one call, with fewer launches: the pair fill
 * also forms the output keys, the plan's counters are cleared inside the join
 * count, the segment fill runs inside the flag scan, and one copy returns
 * every count.  No counterpart in the reference (see ej_join_count_async); it
 * queues the phases of execute_sparse (sparse_dispatch.py:226-297) up to the
 * einsum.  Needs n_keys >= 1 and non-empty relations.  join_workspace: sized
 * by ej_join_workspace_size(n_lhs, n_rhs, EJ_ORDER_PROBE); seg_workspace: by
 * ej_segment_workspace_size(pair_capacity); its first int64 (U) is then the
 * n_segments_dev of ej_segment_einsum_async.  lhs_idx / rhs_idx / perm hold
 * pair_capacity entries, out_coords [seg_capacity, n_out] and seg_offsets
 * [seg_capacity + 1]; writes are clipped to min(P, pair_capacity) pairs and
 * seg_capacity segments.  counts (pinned host memory, 6 int64) receives, in
 * stream order: counts[0] = U, [1] = plan range flag, [2] = pairs planned
 * min(P, pair_capacity), [4] = P, [5] = join range flag; P > pair_capacity
 * or U > seg_capacity means the plan is incomplete.  counts_direct > 0
 * declares counts coherent host memory from ej_host_alloc, of 8 int64: a plan
 * kernel may then store the counts there itself instead of a copy following
 * it, and counts[6] = counts_direct (a caller's ticket) is stored after them
 * in stream order, so that a host may wait for the ticket instead of an
 * event.  run_order (may be NULL, 1 + ceil(seg_capacity / group) int32): for
 * an einsum that will run groups of `group` consecutive segments per
 * workgroup (group from ej_segment_einsum_group for the einsum's descriptor),
 * the plan may write the order in which the workgroups should take the
 * ngroups = ceil(min(U, seg_capacity) / group) live groups (heaviest first
 * within each XCD's share of the live workgroups): run_order[0] = ngroups,
 * run_order[1 .. ngroups] a permutation of 0 .. ngroups - 1;
 * *run_order_written (host, set before the call returns) says whether it
 * will, and only then should the order be passed to the einsum.  Scheduling
 * only: the results do not depend on it. */
int ej_pair_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                       const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                       int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                       const int64_t *join_radices, int32_t n_out, const int32_t *agg_src,
                       const int32_t *agg_dim, const int64_t *agg_radices,
                       int64_t pair_capacity, void *join_workspace, size_t join_workspace_bytes,
                       void *seg_workspace, size_t seg_workspace_bytes, int64_t *lhs_idx,
                       int64_t *rhs_idx, int32_t *out_coords, int32_t *seg_offsets,
                       int32_t *perm, int64_t seg_capacity, int32_t group, int32_t *run_order,
                       int32_t *run_order_written, int64_t *counts, int32_t counts_direct,
                       ej_stream_t stream);

/* ej_pair_plan_async without workspace arguments: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * join and segment workspaces come from a static device scratch of 64 MiB
 * that the library holds on every GPU it runs on until the process ends (it
 * fits, e.g., 15,488 x 131,072 tiles with 991,232 pairs); a call that needs
 * more returns EJ_E_CAPACITY.  The call allocates nothing (no hipMalloc, no
 * hipFree) and clears what must start at zero itself.  Every call on one GPU
 * shares that GPU's scratch: calls that overlap on one GPU (other streams or
 * threads, before the previous call's kernels finished reading the scratch
 * through its einsum) race.  Arguments and results as ej_pair_plan_async,
 * except that the device-side segment count stays in the scratch: U is
 * returned in counts[0] (with counts_direct, the device address of counts,
 * from hipHostGetDevicePointer, can serve as the n_segments_dev of
 * ej_segment_einsum_async). */
int ej_pair_plan_async_noalloc(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                               const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                               int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                               const int64_t *join_radices, int32_t n_out, const int32_t *agg_src,
                               const int32_t *agg_dim, const int64_t *agg_radices,
                               int64_t pair_capacity, int64_t *lhs_idx, int64_t *rhs_idx,
                               int32_t *out_coords, int32_t *seg_offsets, int32_t *perm,
                               int64_t seg_capacity, int32_t group, int32_t *run_order,
                               int32_t *run_order_written, int64_t *counts, int32_t counts_direct,
                               ej_stream_t stream);

/* Join and segment plan in one launch for a join against a dense rhs (no
 * counterpart in the reference, whose join and grouping run on the host,
 * sparse_dispatch.py:29-82, :129-171; the results are the same).  Applies
 * when the rhs holds every tile of its grid rhs_grid in lexicographic order,
 * its join dims are rhs dims 0 .. n_keys-1 (each joined once, their lhs dims
 * increasing in that order), the output dims are lhs dims 0 .. nlo-1 followed
 * by rhs dims n_keys .. rhs_ncols-1, every other lhs dim is a join dim, and
 * the lhs coordinates are strictly increasing in lexicographic order and
 * inside lhs_grid; 1 <= n_lhs <= 16384, the rhs grid under 2^31 tiles and
 * n_lhs * NK under 2^30 pairs.  Then every lhs tile meets one rhs
 * tile per value of the rhs dims after the join dims (NK of them), P = n_lhs
 * * NK, and the lhs tiles sharing their first nlo coordinates form a run: the
 * plan writes the pairs in segment order (perm = identity: pass perm = NULL
 * to the einsum), segment u = (run u / NK, k = u % NK) holding the run's
 * tiles in lhs order (the reference's accumulation order),
 * seg_offsets[0 .. U], out_coords [U, n_out] (ascending, as the reference
 * sorts them) and, given run_order and group, a run order in the layout of
 * ej_pair_plan_async's: when NK is a multiple of group and the einsum's
 * eight equal shares of consecutive groups would leave one share's pair
 * total more than 5% above the mean, the runs ranked longest first and
 * dealt to the XCDs in snake order (0-7, 7-0, ...), each run's groups kept
 * together; otherwise a header of 0, which the einsum ignores (groups in
 * plan order).  Structure that does not match gives
 * EJ_E_UNSUPPORTED (take the general plan).  Properties that fail on the
 * device (rhs not the full grid in order, lhs not increasing or outside its
 * grid, more than 8192 runs, U > seg_capacity) give counts[1] = 1 and a
 * segment count of 0 on the device, so that an einsum queued behind does no
 * work; the caller then takes the general plan.  Capacities: pair_capacity
 * >= n_lhs * NK; seg_capacity bounds U.  dev_counts: device int64[8] whose
 * entry [7] is zero at the call (the plan returns it to zero, so a caller
 * zeroes the buffer once and reuses it on its stream); afterwards
 * dev_counts[0 .. 5] hold the six counts (U, the not-applicable flag, P, 0,
 * P, 0), dev_counts[0] = U being the n_segments_dev of
 * ej_segment_einsum_async.  counts (pinned host memory): with counts_direct
 * == 0 the six counts are copied there in stream order; counts_direct > 0
 * (a ticket below 2^30) declares counts coherent host memory from
 * ej_host_alloc, and the plan stores the single word counts[6] = ticket << 33
 * | flag << 32 | U instead (P = n_lhs * NK is known to the caller), so that a
 * host waiting for the ticket reads every count from one store, without the
 * plan having to order several.  Asynchronous. */
int ej_dense_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                        const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                        int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                        const int64_t *lhs_grid, const int64_t *rhs_grid, int32_t n_out,
                        const int32_t *agg_src, const int32_t *agg_dim, int64_t *lhs_idx,
                        int64_t *rhs_idx, int64_t pair_capacity, int32_t *out_coords,
                        int32_t *seg_offsets, int64_t seg_capacity, int32_t group,
                        int32_t *run_order, int32_t *run_order_written, int64_t *dev_counts,
                        int64_t *counts, int32_t counts_direct, ej_stream_t stream);

/* Join and segment plan, in three launches and without sorting, for a join
 * of two sorted sparse relations with the structure of ej_dense_plan_async
 * (no counterpart in the reference, whose join and grouping run on the host,
 * sparse_dispatch.py:29-82, :129-171; the results are the same): the join
 * covers rhs dims 0 .. n_keys-1 once each, their lhs dims increasing; the
 * output is lhs dims 0 .. nlo-1 followed by rhs dims n_keys .. rhs_ncols-1;
 * every other lhs dim is a join dim; both relations' coordinates strictly
 * increasing in lexicographic order and inside their grids.  The rhs need
 * not hold every tile.  Then the lhs tiles sharing their first nlo
 * coordinates form a run, lhs tile t meets the rhs tiles with its join key
 * (a contiguous "row" of the rhs, in rhs order), the run's segments are the
 * distinct values F of the rhs dims after the join dims among the rows its
 * tiles meet (ascending: the reference's sorted output coordinates), and
 * segment (run, F) holds one pair per run tile whose row holds F, in lhs
 * order (the reference's accumulation order).  The plan writes the pairs in
 * segment order (perm = identity: pass perm = NULL to the einsum),
 * seg_offsets[0 .. U] and out_coords [U, n_out].  Limits (else
 * EJ_E_UNSUPPORTED, take the general plan): 1 <= n_lhs <= 16384, n_rhs >= 1,
 * at most 65536 join keys (the product of rhs_grid over the join dims), 8192
 * values of F (the product over the rhs dims after them) and 8192 runs
 * (min(n_lhs, product of lhs_grid over dims 0 .. nlo-1)).  workspace: at
 * least ej_row_plan_workspace_size(n_lhs, n_rhs, join keys) bytes.  Data that fails
 * a check on the device (order, grids) gives flag bit 0; P > pair_capacity,
 * U > seg_capacity, or P or U at or above 2^21 gives flag bit 1; either way
 * nothing is written and the device-side segment count is 0, so that an
 * einsum queued behind does no work (bit 0: take the general plan; bit 1:
 * retry with capacities for P, when P < 2^21).  dev_counts: device int64[8]
 * whose entries [6] and [7] are zero at the call (the plan returns them to
 * zero; the buffer of ej_dense_plan_async on the same stream serves);
 * afterwards dev_counts[0 .. 5] = (U, or 0 after a failure; flag; min(P,
 * pair_capacity); 0; P; 0), dev_counts[0] being the n_segments_dev of
 * ej_segment_einsum_async.  counts (pinned host memory): with counts_direct
 * == 0 those six counts are copied there in stream order; counts_direct > 0
 * (a ticket below 2^20) declares counts coherent host memory from
 * ej_host_alloc, and the plan stores the single word counts[6] = ticket << 44
 * | flag << 42 | min(P, 2^21 - 1) << 21 | min(U, 2^21 - 1) instead.
 * Asynchronous. */
int ej_row_plan_async(const int32_t *lhs_coords, int64_t n_lhs, int32_t lhs_ncols,
                      const int32_t *rhs_coords, int64_t n_rhs, int32_t rhs_ncols,
                      int32_t n_keys, const int32_t *lhs_dims, const int32_t *rhs_dims,
                      const int64_t *lhs_grid, const int64_t *rhs_grid, int32_t n_out,
                      const int32_t *agg_src, const int32_t *agg_dim, int64_t *lhs_idx,
                      int64_t *rhs_idx, int64_t pair_capacity, int32_t *out_coords,
                      int32_t *seg_offsets, int64_t seg_capacity, void *workspace,
                      size_t workspace_bytes, int64_t *dev_counts, int64_t *counts,
                      int32_t counts_direct, ej_stream_t stream);

/* Workspace bytes of ej_row_plan_async for n_lhs lhs tiles (1 .. 16384),
 * n_rhs rhs tiles and n_join rhs join keys (1 .. 65536). */
int ej_row_plan_workspace_size(int64_t n_lhs, int64_t n_rhs, int64_t n_join, size_t *bytes);

/* Coherent, device-mapped host memory (hipHostMalloc, mapped | coherent) for
 * counts that kernels store directly (ej_pair_plan_async, counts_direct). */
int ej_host_alloc(size_t bytes, void **host_ptr);
int ej_host_free(void *host_ptr);

/* ---- gather (reference: values[indices], sparse_dispatch.py:118-119) ---- */
/* out[i] = values[idx[i]] for whole tiles of tile_bytes each.  Indices
 * outside [0, n_tiles) produce a zero tile. */
int ej_gather_tiles(const void *values, int64_t n_tiles, int64_t tile_bytes, const int64_t *idx,
                    int64_t n, void *out, ej_stream_t stream);

/* ---- tile einsum (reference: kernel_einsum, sparse_dispatch.py:85-126) -- */
/* GEMM-shaped descriptors (is_gemm == 1) with 32-multiple M and N, a K that
 * is a multiple of 32 (bf16) or 16 (fp32) and 16-byte aligned operand rows
 * run on the MFMA kernel; every other descriptor, or one whose is_gemm the
 * caller cleared, runs on the generic strided kernel.  A pair whose tile
 * index lies outside [0, n_*_tiles) contributes nothing.
 * dtype EJ_I32 (int32 tiles, the reference's jnp arrays of integer values
 * with 64-bit types off) runs on the generic kernel with products and sums
 * in two's-complement int32, wrapping as an integer dot in XLA does; the
 * descriptor's out_dtype must then be EJ_I32.
 * Per-pair mode: out[p] = einsum(lhs_values[lhs_idx[p]], rhs_values[rhs_idx[p]])
 * for p < n_pairs, [n_pairs, c_elems] of desc->out_dtype.  lhs_idx / rhs_idx
 * may be NULL, meaning pair p reads tile p (a gathered panel). */
int ej_pair_einsum(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                   const void *rhs_values, int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                   const int64_t *lhs_idx, const int64_t *rhs_idx, int64_t n_pairs, void *out,
                   ej_stream_t stream);
/* Fused mode (gather + einsum + segment sum): out[u] = sum over the pairs
 * of segment u, in plan order, of the per-pair einsum, formed in fp32;
 * [n_segments, c_elems] of desc->out_dtype, each output tile written once,
 * no atomics. */
int ej_segment_einsum(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                      const void *rhs_values, int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                      const int64_t *lhs_idx, const int64_t *rhs_idx, const int32_t *perm,
                      const int32_t *seg_offsets, int64_t n_segments, void *out,
                      ej_stream_t stream);

/* ej_segment_einsum with the segment count read on the device from
 * *n_segments_dev (e.g. the first int64 of a segment workspace after
 * ej_segment_count_async): the grid covers max_segments, seg_offsets holds
 * at least min(U, max_segments) + 1 entries and out max_segments tiles, of
 * which the first U are written; the workgroups of the first U segments are
 * the ones spread over the XCDs.  run_order (may be NULL): a run order from
 * ej_pair_plan_async made for groups of run_order_group segments; the einsum
 * follows it only when it runs groups of that size and the order's header
 * (run_order[0]) equals its number of live groups, ceil(min(U,
 * max_segments) / group); otherwise it ignores the whole order.  The
 * results do not depend on the order.  No counterpart in the reference (see
 * ej_join_count_async). */
int ej_segment_einsum_async(const ej_einsum_desc *desc, int32_t dtype, const void *lhs_values,
                            const void *rhs_values, int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                            const int64_t *lhs_idx, const int64_t *rhs_idx, const int32_t *perm,
                            const int32_t *seg_offsets, int64_t max_segments,
                            const int64_t *n_segments_dev, const int32_t *run_order,
                            int32_t run_order_group, void *out, ej_stream_t stream);

/* Segments per workgroup of the fused einsum for this descriptor and dtype
 * (grouped by the seg_group hint; 16-byte aligned operands assumed): the
 * group size to pass to ej_pair_plan_async for a run order.  1 means the
 * einsum does not run grouped.  No counterpart in the reference. */
int ej_segment_einsum_group(const ej_einsum_desc *desc, int32_t dtype, int32_t *group);

/* ---- segment sum (reference: segment_sum accumulation, :164-171) -------- */
/* out[u] = sum_{q in [seg_offsets[u], seg_offsets[u+1])} pair_values[perm[q]],
 * added sequentially in q order (the reference's order).  pair_values and out
 * are both of dtype, the reference keeping the values' dtype (:165): EJ_F32
 * or EJ_BF16 (sums formed in fp32, a bf16 output rounded once), EJ_F64 (sums
 * in float64, each element's exactly as the reference's sequential numpy
 * additions form it), EJ_F16 (each addition formed in fp32 and rounded to
 * float16, as numpy adds float16) or EJ_I32 / EJ_I64 (two's-complement,
 * wrapping as numpy's integer additions do). */
int ej_segment_sum(const void *pair_values, int32_t dtype, int64_t tile_elems,
                   const int32_t *perm, const int32_t *seg_offsets, int64_t n_segments,
                   void *out, ej_stream_t stream);

/* ---- tiling (reference: SparseTensor.to_relation, tensor/sparse.py:160-219) */
/* Dense row-major input of rank ndim.  A tile is kept iff it holds an element
 * that compares != 0 (NaN counts as nonzero, -0.0 does not, as the
 * reference's `values != 0` filter); kept tiles appear in ascending
 * lexicographic coordinate order; inside a kept tile every element that
 * compares == 0 is written as +0.0.  tile_shape must divide shape
 * (EJ_E_INVAL otherwise, as the reference raises ValueError).
 * The tiles keep the input's dtype: EJ_F64 (the reference's dtype for
 * relation values, sparse.py:191, :210), EJ_F32 or EJ_BF16. */
int ej_bucket_workspace_size(int32_t ndim, const int64_t *shape, const int64_t *tile_shape,
                             size_t *bytes);
int ej_bucket_dense_count(const void *dense, int32_t dtype, int32_t ndim, const int64_t *shape,
                          const int64_t *tile_shape, void *workspace, size_t workspace_bytes,
                          int64_t *n_tiles, ej_stream_t stream);
/* coords int32 [n_tiles, ndim]; values [n_tiles, *tile_shape] of `dtype`. */
int ej_bucket_dense_fill(const void *dense, int32_t dtype, int32_t ndim, const int64_t *shape,
                         const int64_t *tile_shape, const void *workspace,
                         size_t workspace_bytes, int64_t n_tiles, int32_t *coords, void *values,
                         int64_t capacity, ej_stream_t stream);

/* ---- COO ingest (reference: _extract_coo, tensor/sparse.py:234-270) ----- */
/* Dense row-major input (EJ_F32, EJ_BF16 or EJ_F64) to COO: the elements that
 * compare != 0 (NaN included, -0.0 excluded) in row-major order, the order of
 * np.nonzero; indices int32 [nnz, ndim], values float64 [nnz] (the
 * reference's dtype, :246-260; the conversion is exact).  Extents must be
 * below 2^31. */
int ej_extract_coo_workspace_size(int32_t ndim, const int64_t *shape, int32_t dtype,
                                  size_t *bytes);
int ej_extract_coo_count(const void *dense, int32_t dtype, int32_t ndim, const int64_t *shape,
                         void *workspace, size_t workspace_bytes, int64_t *nnz,
                         ej_stream_t stream);
int ej_extract_coo_fill(const void *dense, int32_t dtype, int32_t ndim, const int64_t *shape,
                        const void *workspace, size_t workspace_bytes, int64_t nnz,
                        int32_t *indices, double *values, int64_t capacity, ej_stream_t stream);

/* ---- COO tiling (reference: SparseTensor.to_relation, tensor/sparse.py:160-219) */
/* COO input: indices int32 [nnz, ndim] (device), values [nnz] of EJ_F64,
 * EJ_F32 or EJ_BF16 (device), nnz < 2^31, in any order, repeats allowed.
 * Entries whose value compares == 0 are dropped (:184-187); the tiles holding
 * the others appear in ascending lexicographic coordinate order (:204-206);
 * every other element of a kept tile is +0.0 (:210-212); an element listed
 * more than once takes the value of its last nonzero entry, as the
 * reference's fancy assignment leaves it.  A nonzero entry whose index lies
 * outside shape gives EJ_E_RANGE; tile_shape must divide shape (EJ_E_INVAL).
 * Tiles have the values' dtype (float64 for EJ_F64, as the reference's
 * float64 tiles, sparse.py:210). */
int ej_bucket_coo_workspace_size(int64_t nnz, int32_t dtype, int32_t ndim, const int64_t *shape,
                                 const int64_t *tile_shape, size_t *bytes);
int ej_bucket_coo_count(const int32_t *indices, const void *values, int32_t dtype, int64_t nnz,
                        int32_t ndim, const int64_t *shape, const int64_t *tile_shape,
                        void *workspace, size_t workspace_bytes, int64_t *n_tiles,
                        ej_stream_t stream);
/* coords int32 [n_tiles, ndim]; tiles [n_tiles, *tile_shape]; indices and
 * values as given to ej_bucket_coo_count. */
int ej_bucket_coo_fill(const int32_t *indices, const void *values, int32_t dtype, int64_t nnz,
                       int32_t ndim, const int64_t *shape, const int64_t *tile_shape,
                       const void *workspace, size_t workspace_bytes, int64_t n_tiles,
                       int32_t *coords, void *tiles, int64_t capacity, ej_stream_t stream);

/* ---- statistics (reference: _compute_sparsity_metrics, tensor/sparse.py:124-158) */
/* For each of n_schemes tile shapes (tile_shapes: HOST int64
 * [n_schemes, ndim], each extent dividing shape), over the elements that
 * compare != 0:
 *   num_tuples[s]            = number of distinct tile coordinates idx // t_s;
 *   value_count[s * ndim + l] = number of distinct idx[l] // t_s[l];
 * all zero when no element is nonzero (:141-145).  num_tuples and
 * value_count are HOST arrays; the calls synchronize `stream`.  Extents must
 * lie in [1, 2^31).
 * Dense input: nnz = -1 in the workspace query.  The workspace holds
 * occupancy maps of about twice the tensor's element count in bytes.
 * COO input (indices int32 [nnz, ndim], values [nnz], as ej_bucket_coo_*):
 * tile shapes whose grid has more than bitmap_cap tiles (<= 0: 2^32) are
 * counted by sorting the entries' tile keys instead of an occupancy map.  A
 * nonzero entry outside shape gives EJ_E_RANGE. */
int ej_scheme_stats_workspace_size(int32_t ndim, const int64_t *shape, int64_t n_schemes,
                                   const int64_t *tile_shapes, int64_t nnz, int64_t bitmap_cap,
                                   size_t *bytes);
int ej_scheme_stats_dense(const void *dense, int32_t dtype, int32_t ndim, const int64_t *shape,
                          int64_t n_schemes, const int64_t *tile_shapes, void *workspace,
                          size_t workspace_bytes, int64_t *num_tuples, int64_t *value_count,
                          ej_stream_t stream);
int ej_scheme_stats_coo(const int32_t *indices, const void *values, int32_t dtype, int64_t nnz,
                        int32_t ndim, const int64_t *shape, int64_t n_schemes,
                        const int64_t *tile_shapes, int64_t bitmap_cap, void *workspace,
                        size_t workspace_bytes, int64_t *num_tuples, int64_t *value_count,
                        ej_stream_t stream);

/* ---- backward (reference: sparse_einsum_raw._bwd, autodiff/custom_vjp.py:254-275) */
/* Groups positions 0 .. n-1 by target idx[p] in [0, n_targets): perm int32
 * [n] lists them target by target, ascending position within a target;
 * offsets int32 [n_targets + 1] delimits the targets; positions whose target
 * lies outside the range come last in perm, beyond offsets[n_targets].
 * n < 2^31.  Asynchronous.  This is the grouping of the reference's
 * .at[indices].add scatter (:271-272), made deterministic. */
int ej_index_plan_workspace_size(int64_t n, size_t *bytes);
int ej_index_plan(const int64_t *idx, int64_t n, int64_t n_targets, int32_t *perm,
                  int32_t *offsets, void *workspace, size_t workspace_bytes, ej_stream_t stream);

/* Gradients of out[p] = einsum(kernel_string, lhs_values[lhs_idx[p]],
 * rhs_values[rhs_idx[p]]) for the cotangent grad_out [n_pairs, *out_tile]:
 *   grad_lhs[l] = sum_{p: lhs_idx[p] == l} einsum("C,B->A", grad_out[p], rhs_values[rhs_idx[p]])
 *   grad_rhs[r] = sum_{p: rhs_idx[p] == r} einsum("A,C->B", lhs_values[lhs_idx[p]], grad_out[p])
 * for kernel_string "A,B->C" (the reference's reversed strings,
 * custom_vjp.py:31-62).  grad_lhs [n_lhs_tiles, *lhs_tile] and grad_rhs
 * [n_rhs_tiles, *rhs_tile] are fully written (zeros where no pair
 * contributes); either may be NULL to skip it.  Each gradient tile is summed
 * in fp32 in ascending pair order, without atomics, so results are
 * reproducible.  A pair whose index lies outside its operand's tile count
 * contributes nothing.  A reversed string that is not a valid einsum of its
 * operands (a label of A found in neither C nor B) gives EJ_E_INVAL, as the
 * reference's jnp.einsum raises.  dtype (EJ_F32 / EJ_BF16) is the dtype of
 * the operand values; grad_dtype that of grad_out, grad_lhs and grad_rhs:
 * EJ_F32 (with bf16 operands each fp32 value is then split into three
 * bf16 terms that sum to it exactly and the einsums run bf16 MFMAs with fp32
 * sums, the precision of fp32 products; layouts the split kernels do not
 * cover widen the operands to fp32 in the workspace), or
 * EJ_BF16 with bf16 operands (the reference's dtype for bf16 values: the
 * einsums run on bf16 operands and each gradient is rounded once).
 * Asynchronous on `stream`.  With both gradients requested, part of the work
 * (the lhs gradient's grouping) runs on a second stream that the library
 * keeps per host thread and device: it starts after the work already queued
 * on `stream`, and `stream` waits for it before the lhs gradient's einsum,
 * so the call is ordered on `stream` as a whole (the fork and join are
 * event records and waits). */
int ej_pair_einsum_vjp_workspace_size(int64_t n_pairs, int64_t n_lhs_tiles, int64_t n_rhs_tiles,
                                      int64_t lhs_elems, int64_t rhs_elems, int32_t dtype,
                                      int32_t grad_dtype, size_t *bytes);
int ej_pair_einsum_vjp(const char *kernel_string, const int64_t *lhs_tile, int32_t lhs_ndim,
                       const int64_t *rhs_tile, int32_t rhs_ndim, int32_t dtype,
                       const void *lhs_values, int64_t n_lhs_tiles, const void *rhs_values,
                       int64_t n_rhs_tiles, const int64_t *lhs_idx, const int64_t *rhs_idx,
                       int64_t n_pairs, int32_t grad_dtype, const void *grad_out,
                       void *grad_lhs, void *grad_rhs, void *workspace, size_t workspace_bytes,
                       ej_stream_t stream);

/* ---- relation to dense (reference: SparseTensorRelation.to_dense, :75-90) */
/* Writes every tile of the relation into `dense` (row-major `shape`, of the
 * values' dtype: EJ_F32, EJ_BF16 or EJ_F64).  Elements not covered by a tile
 * are set to zero. */
int ej_relation_to_dense(const int32_t *coords, const void *values, int64_t n_tiles,
                         int32_t dtype, int32_t ndim, const int64_t *shape,
                         const int64_t *tile_shape, void *dense, ej_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EINJAX_HIP_H */
