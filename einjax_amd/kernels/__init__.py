"""Kernel registry, block-sparse matmul and the coordinate joins."""

from .block_sparse import block_sparse_matmul, block_sparse_matmul_generic
from .join import coordinate_join_hash, coordinate_join_sorted
from .registry import KernelInfo, KernelRegistry

__all__ = [
    "KernelRegistry", "KernelInfo", "block_sparse_matmul", "block_sparse_matmul_generic",
    "coordinate_join_sorted", "coordinate_join_hash",
]
