"""Restatement of the reference's host-side selection rules: tile-shape
selection (tensor/tiling.py:31-125, :296-324, with tensor/stats.py:113-134)
and kernel lookup (kernels/registry.py:67-140, :178-275).

Test infrastructure only (see ``oracle/__init__.py``).  Schemes are plain
``(tile_shape, num_tuples)`` records here, listed in the reference's
enumeration order (itertools.product of the ascending divisor lists,
tensor/base.py:43-49), so the oracle shares no code with the product.
"""

from __future__ import annotations

from math import prod
from typing import NamedTuple


class Scheme(NamedTuple):
    tile_shape: tuple
    num_tuples: int

    @property
    def tile_size(self) -> int:
        return prod(self.tile_shape)


def schemes_from_metrics(metrics: dict) -> list:
    """Scheme records, in enumeration order, from reference_path.sparsity_metrics
    output ({tile_shape: (num_tuples, value_count)}, itself in that order)."""
    return [Scheme(tuple(ts), int(v[0])) for ts, v in metrics.items()]


def sparsity_ratio(num_tuples: int, shape: tuple, tile_shape: tuple) -> float:
    """tensor/stats.py:113-134: num_tuples over the tile count of the grid;
    0.0 for an empty grid."""
    total = prod(s // t for s, t in zip(shape, tile_shape))
    if total == 0:
        return 0.0
    return num_tuples / total


def prune_infeasible_schemes(schemes: list, num_devices: int = 1, max_tile_bytes=None,
                             dtype_size: int = 4) -> list:
    """tensor/tiling.py:31-65: the device-count test keeps every scheme
    (:55-58); a scheme whose tile_size * dtype_size exceeds max_tile_bytes
    is dropped (:60-63)."""
    kept = []
    for s in schemes:
        if max_tile_bytes is not None and s.tile_size * dtype_size > max_tile_bytes:
            continue
        kept.append(s)
    return kept


def rank_schemes_by_sparsity(schemes: list, shape: tuple) -> list:
    """tensor/tiling.py:68-93: a stable sort on (sparsity ratio ascending,
    tile_size descending), ties kept in enumeration order."""
    return sorted(schemes,
                  key=lambda s: (sparsity_ratio(s.num_tuples, shape, s.tile_shape), -s.tile_size))


def select_best_sparse_tiling(schemes: list, shape: tuple, num_devices: int = 1,
                              max_tile_bytes=None, dtype_size: int = 4):
    """tensor/tiling.py:96-125 (and prepare_sparse_tiling, :296-324): prune,
    then the first of the ranking; None when nothing is left."""
    feasible = prune_infeasible_schemes(schemes, num_devices, max_tile_bytes, dtype_size)
    if not feasible:
        return None
    return rank_schemes_by_sparsity(feasible, shape)[0]


# ---------------------------------------------------------------------------
# Kernel registry lookup.

class Entry(NamedTuple):
    name: str
    pattern: str
    backend: str
    sparsity: str
    priority: int


# The reference's builtins, in registration order (registry.py:67-97).
BUILTINS = [
    Entry("generic_sparse_matmul", "ij,jk->ik", "generic", "sparse", 0),
    Entry("generic_sparse_einsum", "*", "generic", "sparse", -1),
    Entry("generic_dense_einsum", "*", "generic", "dense", 0),
]


def pattern_matches(registered: str, query: str) -> bool:
    """registry.py:245-252."""
    return registered == "*" or registered == query


def backend_matches(registered: str, query: str) -> bool:
    """registry.py:255-266: generic matches any backend; "gpu" also matches
    "gpu:<variant>"."""
    return registered == "generic" or registered == query or query.startswith(registered + ":")


def sparsity_matches(registered: str, query: str) -> bool:
    """registry.py:269-273."""
    return registered == "any" or registered == query


def lookup(entries: list, pattern: str, backend: str, sparsity: str = "dense"):
    """registry.py:107-140: candidates in registration order (:207-223),
    stable sort by priority descending, the first wins; None where the
    reference raises ValueError."""
    cands = [e for e in entries if pattern_matches(e.pattern, pattern)
             and backend_matches(e.backend, backend) and sparsity_matches(e.sparsity, sparsity)]
    if not cands:
        return None
    cands.sort(key=lambda e: e.priority, reverse=True)
    return cands[0]


def list_kernels(entries: list, pattern=None, backend=None, sparsity=None) -> list:
    """registry.py:178-205: filters applied in turn; the pattern filter keeps
    exact matches and "*" entries, the sparsity filter exact and "any"."""
    out = list(entries)
    if pattern is not None:
        out = [e for e in out if e.pattern == pattern or e.pattern == "*"]
    if backend is not None:
        out = [e for e in out if backend_matches(e.backend, backend)]
    if sparsity is not None:
        out = [e for e in out if e.sparsity == sparsity or e.sparsity == "any"]
    return out
