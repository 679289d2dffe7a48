"""The sparse execution path."""

from .engine import ExecutionEngine, build_dependency_graph, topological_sort
from .sparse_dispatch import (
    coordinate_join,
    execute_sharded_sparse,
    execute_sparse,
    kernel_einsum,
    segment_sum,
)

__all__ = ["coordinate_join", "kernel_einsum", "segment_sum", "execute_sparse",
           "execute_sharded_sparse", "ExecutionEngine", "build_dependency_graph",
           "topological_sort"]
