"""Tile-shape selection for sparse tensors (reference: tensor/tiling.py).

Host-side and O(number of tile shapes); the statistics it ranks on
(``TilingScheme.num_tuples``) come from ``SparseTensor.schemes``.  Function
names, arguments and results follow the reference so callers switch
without changes.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from enum import Enum
from math import prod
from typing import Any


class CaseAssignment(Enum):
    """Upper case = tiled (tile < extent), lower case = whole extent in the
    kernel (reference: core/types.py:68-76)."""

    UPPER = "upper"
    LOWER = "lower"


@dataclass(eq=False)
class TilingScheme:
    """One tiling of a tensor (reference: core/types.py:83-139).  Before the
    statistics are filled in, num_tuples is the size of the tile grid."""

    node: Any
    shape: tuple
    tile_shape: tuple
    tile_size: int = field(init=False)
    value_count: tuple = field(init=False)
    num_tuples: int = field(init=False)
    cost: float = 0.0
    comm: float = 0.0
    flops: float = 0.0
    accumulated_cost: float = 0.0
    accumulated_comm: float = 0.0
    accumulated_flops: float = 0.0
    # dependency tracking: the schemes this one is computed from (the
    # execution engine walks them)
    source: tuple = field(default_factory=tuple)
    dependencies: set = field(default_factory=set)
    partition_spec: Any = None
    mesh_axes: Any = None

    def __post_init__(self):
        self.shape = tuple(self.shape)
        self.tile_shape = tuple(self.tile_shape)
        self.tile_size = prod(self.tile_shape)
        self.value_count = tuple(s // t for s, t in zip(self.shape, self.tile_shape))
        self.num_tuples = prod(self.value_count)

    def __hash__(self):
        return hash((id(self.node), self.tile_shape))

    def get_case_assignments(self) -> list:
        return [CaseAssignment.LOWER if t == s else CaseAssignment.UPPER
                for s, t in zip(self.shape, self.tile_shape)]


def find_all_factors(n: int) -> list:
    """Divisors of n, ascending (reference: core/notation.py:27-44)."""
    if n <= 0:
        raise ValueError(f"n must be positive, got {n}")
    f = set()
    i = 1
    while i * i <= n:
        if n % i == 0:
            f.add(i)
            f.add(n // i)
        i += 1
    return sorted(f)


def enumerate_tile_shapes(shape: tuple) -> list:
    """Every tile shape whose extents divide the tensor's (reference:
    tensor/base.py:43-45); zero extents admit no tiling."""
    if any(s <= 0 for s in shape):
        return []
    return list(itertools.product(*[find_all_factors(s) for s in shape]))


def sparsity_ratio(num_tuples: int, shape: tuple, tile_shape: tuple) -> float:
    """T(U) / number of tiles in the grid (reference: tensor/stats.py:113-134)."""
    max_tuples = prod(s // t for s, t in zip(shape, tile_shape))
    return 0.0 if max_tuples == 0 else num_tuples / max_tuples


def prune_infeasible_schemes(schemes: dict, num_devices: int = 1, max_tile_bytes=None,
                             dtype_size: int = 4) -> dict:
    """Drops schemes whose tile exceeds max_tile_bytes (reference:
    tensor/tiling.py:31-65; the device-count branch keeps every scheme)."""
    out = {}
    for ts, sch in schemes.items():
        if max_tile_bytes is not None and sch.tile_size * dtype_size > max_tile_bytes:
            continue
        out[ts] = sch
    return out


def rank_schemes_by_sparsity(schemes: dict, shape: tuple) -> list:
    """Sparsest first (T(U)/max), ties to the larger tile (reference:
    tensor/tiling.py:68-93)."""
    return sorted(schemes.values(),
                  key=lambda s: (sparsity_ratio(s.num_tuples, shape, s.tile_shape), -s.tile_size))


def select_best_sparse_tiling(schemes: dict, shape: tuple, num_devices: int = 1,
                              max_tile_bytes=None, dtype_size: int = 4):
    """Prune then rank; the best scheme or None (reference: tensor/tiling.py:96-125)."""
    feasible = prune_infeasible_schemes(schemes, num_devices, max_tile_bytes, dtype_size)
    if not feasible:
        return None
    ranked = rank_schemes_by_sparsity(feasible, shape)
    return ranked[0] if ranked else None


def tile_shape_to_partition_spec(shape: tuple, tile_shape: tuple,
                                 mesh_axis_names=("x", "y", "z", "w")) -> tuple:
    """Mesh axis name for every upper-case dim, None for lower-case ones
    (reference: sharding/partition.py:17-92)."""
    if len(shape) != len(tile_shape):
        raise ValueError(f"shape ({len(shape)}D) and tile_shape ({len(tile_shape)}D) "
                         "must have the same number of dimensions")
    for d, (s, t) in enumerate(zip(shape, tile_shape)):
        if t > s:
            raise ValueError(f"tile_shape[{d}]={t} exceeds shape[{d}]={s}")
        if t <= 0:
            raise ValueError(f"tile_shape[{d}]={t} must be positive")
        if s % t != 0:
            raise ValueError(f"shape[{d}]={s} is not evenly divisible by tile_shape[{d}]={t}")
    upper = [t != s for s, t in zip(shape, tile_shape)]
    if sum(upper) > len(mesh_axis_names):
        raise ValueError(f"Need {sum(upper)} mesh axes for sharded dimensions but only "
                         f"{len(mesh_axis_names)} axis names available: {mesh_axis_names}")
    spec, a = [], 0
    for u in upper:
        if u:
            spec.append(mesh_axis_names[a])
            a += 1
        else:
            spec.append(None)
    return tuple(spec)


def get_sparse_partition_spec(scheme: TilingScheme, mesh_axis_names=("x", "y", "z", "w")) -> tuple:
    """reference: tensor/tiling.py:128-152."""
    return tile_shape_to_partition_spec(scheme.shape, scheme.tile_shape, mesh_axis_names)


def compute_tile_memory(tile_shape: tuple, dtype_size: int = 4, include_coords: bool = True) -> int:
    """Bytes of one tile (+ its int32 coordinates) (reference: tensor/tiling.py:155-173)."""
    return prod(tile_shape) * dtype_size + (len(tile_shape) * 4 if include_coords else 0)


def compute_relation_memory(scheme: TilingScheme, dtype_size: int = 4) -> int:
    """Bytes of the relation under a scheme (reference: tensor/tiling.py:176-194)."""
    return scheme.num_tuples * len(scheme.shape) * 4 + scheme.num_tuples * scheme.tile_size * dtype_size


def filter_schemes_by_sharding(schemes: dict, num_devices: int, min_sharded_dims: int = 0,
                               max_sharded_dims=None) -> dict:
    """Bounds the number of upper-case dims; with several devices, the shard
    count must not exceed them (reference: tensor/tiling.py:197-241)."""
    out = {}
    for ts, sch in schemes.items():
        cases = sch.get_case_assignments()
        n_up = sum(1 for c in cases if c == CaseAssignment.UPPER)
        if n_up < min_sharded_dims:
            continue
        if max_sharded_dims is not None and n_up > max_sharded_dims:
            continue
        if num_devices > 1 and n_up > 0:
            shards = prod(s // t for s, t, c in zip(sch.shape, sch.tile_shape, cases)
                          if c == CaseAssignment.UPPER)
            if shards > num_devices:
                continue
        out[ts] = sch
    return out


def filter_schemes_by_device_count(schemes: dict, num_devices: int,
                                   min_tiles_per_device: int = 1) -> dict:
    """With several devices keeps fully local schemes and those whose
    upper-case tile count is divisible by, and at least min_tiles_per_device
    times, the device count (reference: tensor/tiling.py:244-293)."""
    if num_devices <= 1:
        return dict(schemes)
    need = num_devices * min_tiles_per_device
    out = {}
    for ts, sch in schemes.items():
        cases = sch.get_case_assignments()
        if not any(c == CaseAssignment.UPPER for c in cases):
            out[ts] = sch
            continue
        n = prod(s // t for s, t, c in zip(sch.shape, sch.tile_shape, cases)
                 if c == CaseAssignment.UPPER)
        if n >= need and n % num_devices == 0:
            out[ts] = sch
    return out


def prepare_sparse_tiling(tensor, num_devices: int = 1, max_tile_bytes=None, dtype_size: int = 4):
    """Best scheme for a SparseTensor (reference: tensor/tiling.py:296-324)."""
    return select_best_sparse_tiling(tensor.schemes, tensor.shape, num_devices=num_devices,
                                     max_tile_bytes=max_tile_bytes, dtype_size=dtype_size)
