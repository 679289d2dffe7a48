"""einjax_amd: einjax's tensor-relational sparse-einsum path on MI355X (gfx950).

The public names mirror the reference package's sparse-path exports
(reference: __init__.py:68-78 and kernels/__init__.py): relations and
tiling, the three-phase execute_sparse, the kernel registry, the
block-sparse matmul and the coordinate joins.  All computation runs in
libejhip.so (HIP kernels behind a C ABI, include/einjax_hip.h).
"""

from .autodiff import sparse_einsum, sparse_einsum_raw, sparse_einsum_raw_vjp
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
    SparseTensor,
    SparseTensorRelation,
    TilingScheme,
    prepare_sparse_tiling,
    rank_schemes_by_sparsity,
    select_best_sparse_tiling,
)

__version__ = "0.1.0"

__all__ = [
    "SparseTensor", "SparseTensorRelation", "TilingScheme", "prepare_sparse_tiling",
    "rank_schemes_by_sparsity", "select_best_sparse_tiling", "coordinate_join",
    "kernel_einsum", "segment_sum", "execute_sparse", "execute_sharded_sparse", "KernelRegistry",
    "KernelInfo", "block_sparse_matmul", "block_sparse_matmul_generic", "coordinate_join_hash",
    "coordinate_join_sorted", "sparse_einsum", "sparse_einsum_raw", "sparse_einsum_raw_vjp",
]
