"""Tensor-relational containers and tile-shape selection."""

from .dense import DenseTensor
from .sparse import SparseTensor, SparseTensorRelation
from .tiling import (
    CaseAssignment,
    TilingScheme,
    compute_relation_memory,
    compute_tile_memory,
    enumerate_tile_shapes,
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

__all__ = [
    "DenseTensor", "SparseTensor", "SparseTensorRelation", "CaseAssignment", "TilingScheme",
    "compute_relation_memory", "compute_tile_memory", "enumerate_tile_shapes",
    "filter_schemes_by_device_count", "filter_schemes_by_sharding", "find_all_factors",
    "get_sparse_partition_spec", "prepare_sparse_tiling", "prune_infeasible_schemes",
    "rank_schemes_by_sparsity", "select_best_sparse_tiling", "sparsity_ratio",
    "tile_shape_to_partition_spec",
]
