"""einjax_amd: einjax's tensor-relational sparse-einsum path on MI355X (gfx950).

The public names mirror the reference package's sparse-path exports
(reference: __init__.py:9-86 and kernels/__init__.py): einsum / analyze,
relations, dense and sparse tensor metadata and tile-shape selection, the
three-phase execute_sparse, the execution engine over chains of sparse
steps, the kernel registry, the block-sparse matmul
and the coordinate joins.  All computation runs in
libejhip.so (HIP kernels behind a C ABI, include/einjax_hip.h).
"""

from .autodiff import sparse_einsum, sparse_einsum_raw, sparse_einsum_raw_vjp
from .execution.engine import ExecutionEngine, build_dependency_graph, topological_sort
from .execution.sparse_dispatch import (
    coordinate_join,
    execute_sharded_sparse,
    execute_sparse,
    kernel_einsum,
    segment_sum,
)
from .kernels import (
    KernelInfo,
    KernelRegistry,
    block_sparse_matmul,
    block_sparse_matmul_generic,
    coordinate_join_hash,
    coordinate_join_sorted,
)
from .tensor import (
    CaseAssignment,
    DenseTensor,
    SparseTensor,
    SparseTensorRelation,
    TilingScheme,
    compute_relation_memory,
    compute_tile_memory,
    filter_schemes_by_device_count,
    filter_schemes_by_sharding,
    find_all_factors,
    get_sparse_partition_spec,
    prepare_sparse_tiling,
    prune_infeasible_schemes,
    rank_schemes_by_sparsity,
    select_best_sparse_tiling,
    sparsity_ratio,
    tile_shape_to_partition_spec,
)
from .api import (
    AnalysisResult,
    analyze,
    einsum,
    get_label_dimensions,
    normalize_notation,
    validate_inputs,
)

__version__ = "0.1.0"

__all__ = [
    "einsum", "analyze", "AnalysisResult", "normalize_notation", "validate_inputs",
    "get_label_dimensions", "find_all_factors", "CaseAssignment", "DenseTensor",
    "SparseTensor", "SparseTensorRelation", "TilingScheme", "sparsity_ratio",
    "prune_infeasible_schemes", "rank_schemes_by_sparsity", "select_best_sparse_tiling",
    "get_sparse_partition_spec", "compute_tile_memory", "compute_relation_memory",
    "filter_schemes_by_sharding", "filter_schemes_by_device_count", "prepare_sparse_tiling",
    "tile_shape_to_partition_spec", "coordinate_join",
    "kernel_einsum", "segment_sum", "execute_sparse", "execute_sharded_sparse", "KernelRegistry",
    "KernelInfo", "block_sparse_matmul", "block_sparse_matmul_generic", "coordinate_join_hash",
    "coordinate_join_sorted", "sparse_einsum", "sparse_einsum_raw", "sparse_einsum_raw_vjp",
    "ExecutionEngine", "build_dependency_graph", "topological_sort",
]
