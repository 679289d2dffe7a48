"""Block-sparse matrix multiply (reference: kernels/pallas_matmul.py).

``block_sparse_matmul_generic`` is the registry's entry for "ij,jk->ik":
join on the inner tile coordinate, then the fused MFMA tile GEMM with the
segment sum, on the GPU.
"""

from __future__ import annotations

import numpy as np

from ..execution.sparse_dispatch import _empty_result, _on_host, execute_sparse
from ..tensor.sparse import SparseTensorRelation


def block_sparse_matmul_generic(lhs: SparseTensorRelation, rhs: SparseTensorRelation,
                                block_shape=None) -> SparseTensorRelation:
    """C = A @ B for 2-D tile relations (reference: pallas_matmul.py:33-113).

    Raises ValueError for operands that are not 2-D (:55-59) or whose inner
    tile extents differ (:68-73).  ``block_shape=(m, k, n)`` sets the output
    tile shape reported for an empty result, as in the reference (:61-66,
    :79-86)."""
    if lhs.ndim != 2 or rhs.ndim != 2:
        raise ValueError(f"block_sparse_matmul requires 2D tensors, got {lhs.ndim}D and "
                         f"{rhs.ndim}D")
    if block_shape is not None:
        m_tile, _, n_tile = block_shape
    else:
        m_tile, n_tile = lhs.tile_shape[0], rhs.tile_shape[1]
    if lhs.tile_shape[1] != rhs.tile_shape[0]:
        raise ValueError(f"Inner tile dimensions must match: lhs.tile_shape[1]="
                         f"{lhs.tile_shape[1]} != rhs.tile_shape[0]={rhs.tile_shape[0]}")
    out_shape = (lhs.shape[0], rhs.shape[1])
    res = execute_sparse(lhs, rhs, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)],
                         output_shape=out_shape,
                         output_tile_shape=(lhs.tile_shape[0], rhs.tile_shape[1]))
    if res.num_tuples == 0:
        host = _on_host(lhs, rhs)
        empty = _empty_result(lhs, 2, (m_tile, n_tile), out_shape, host)
        if host:  # the reference's empty matmul result is float64 (:80-86)
            empty.values = np.zeros((0, m_tile, n_tile), dtype=np.float64)
        return empty
    return res


def block_sparse_matmul(lhs_coords, lhs_values, rhs_coords, rhs_values, block_shape, lhs_shape,
                        rhs_shape) -> SparseTensorRelation:
    """Raw-array form (reference: pallas_matmul.py:116-158): wraps the arrays as
    relations with tiles (m, k) and (k, n) and multiplies."""
    m_tile, k_tile, n_tile = block_shape
    lhs = SparseTensorRelation(lhs_coords, lhs_values, tuple(lhs_shape), (m_tile, k_tile))
    rhs = SparseTensorRelation(rhs_coords, rhs_values, tuple(rhs_shape), (k_tile, n_tile))
    return block_sparse_matmul_generic(lhs, rhs, block_shape)
