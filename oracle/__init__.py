"""CPU oracle of einjax's tensor-relational sparse-einsum path.

TEST INFRASTRUCTURE ONLY.  This package is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only to compute expected results or the CPU baseline.  The
product path (``einjax_amd``) never imports it and has no CPU fallback.

Modules
  reference_path  NumPy restatement of the reference algorithm, each function
                  citing the reference file:line it follows.
  generators      seeded synthetic relations for the benchmark configurations.
  workload        algorithmic FLOP / byte counts per einsum.

Pinning (what checks each function; see tests/test_oracle.py):
  extract_coo, to_relation, relation_to_dense
      reference known answers (tests/test_sparse.py:216-291, :318-355),
      closed form (round trip to_dense(to_relation(x)) == x), brute force on
      tiny inputs (row-major nonzero order; a COO list with repeats equals a
      sequential write of its nonzero entries).
  divisors, all_tile_shapes, sparsity_metrics
      reference known answers (tests/test_sparse.py:135-214,
      tests/test_dense.py:41, :77-112, tests/test_rigorous.py:367-400) and
      brute force: the occupancy of every tile shape by reducing the dense
      blocks, value_count by projecting that occupancy.
  coordinate_join, coordinate_join_hash, coordinate_join_sorted
      match sets by brute force; counts from the reference tests
      (tests/test_sparse_dispatch.py:46-129, tests/test_pallas.py:235-338);
      pair ORDER by golden vectors written by tests/golden/make_golden.py
      from the reference's own kernels/pallas_gather.py, plus the closed forms
      (probe order == sort by (rhs, lhs); sorted order == (key, lhs rank,
      rhs rank)).
  kernel_einsum, add_batch_dim, infer_output_tile_shape
      reference known answers (tests/test_sparse_dispatch.py:137-196,
      :434-470) and numpy.einsum / matmul in float64 on random inputs.
  compute_output_coords
      reference known answers (tests/test_sparse_dispatch.py:474-521).
  segment_sum, segment_plan
      reference known answers (tests/test_sparse_dispatch.py:204-252) and the
      closed form (sorted unique coordinates, per-segment sums), brute force.
  reverse_einsum_string, pair_einsum_vjp
      reference known answers (tests/test_autodiff.py:42-72 for the strings;
      the gradients of :160-400 in closed form) and central finite
      differences in float64 of the forward kernel_einsum, exact for this
      bilinear map up to rounding.
  execute_sparse, block_sparse_matmul_generic, block_sparse_matmul
      to_dense(result) == einsum of the dense operands (the reference's own
      end-to-end tests, tests/test_sparse_dispatch.py:263-426,
      tests/test_pallas.py:53-224).
"""
