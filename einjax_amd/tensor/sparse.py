"""Tensor-relational containers (reference: tensor/sparse.py).

``SparseTensorRelation`` keeps the reference's fields and properties
(tensor/sparse.py:27-90).  Its arrays are either host NumPy arrays, as in the
reference, or torch tensors resident on the GPU; every operation of the
sparse path accepts both and answers in the residency it was given, so host
callers see the reference's types while chained device calls never leave
HBM.

``SparseTensor`` (tensor/sparse.py:93-231) buckets its data on the GPU in
``to_relation``.  Its per-scheme statistics (``schemes``, the reference's
``_compute_sparsity_metrics``, :124-158) are computed lazily on first access
rather than in the constructor, so building a relation does not pay for
them.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import prod
from typing import Any

import numpy as np

from .tiling import TilingScheme, enumerate_tile_shapes


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


@dataclass
class SparseTensorRelation:
    """Tile coordinates (int32 [T, ndim]) plus dense tiles ([T, *tile_shape]).

    Reference: tensor/sparse.py:27-90.  ``coords`` / ``values`` are NumPy
    arrays (host) or torch tensors on the GPU (device)."""

    coords: Any
    values: Any
    shape: tuple
    tile_shape: tuple

    def __post_init__(self):
        self.shape = tuple(int(s) for s in self.shape)
        self.tile_shape = tuple(int(t) for t in self.tile_shape)

    @property
    def num_tuples(self) -> int:
        """Number of non-empty tiles (sparse.py:49-52)."""
        return int(self.coords.shape[0])

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def tile_size(self) -> int:
        return prod(self.tile_shape)

    @property
    def nnz(self) -> int:
        """Nonzero elements across all tiles (sparse.py:64-67)."""
        if self.is_device:
            import torch

            return int(torch.count_nonzero(self.values).item())
        return int(np.count_nonzero(self.values))

    @property
    def density(self) -> float:
        total = prod(self.shape)
        return self.nnz / total if total > 0 else 0.0

    @property
    def is_device(self) -> bool:
        return _is_torch(self.values) and self.values.is_cuda

    def to_device(self, dtype=None) -> "SparseTensorRelation":
        """Copy to the GPU: int32 coords, float32 values (or bfloat16 when
        requested or already bfloat16).  float64 values become float32, the
        precision the reference's einsum computes in (jnp.array of a
        float64 array under JAX's default x64=False)."""
        import torch

        from .._device import require_gpu

        dev = require_gpu()
        if _is_torch(self.values):
            vals = self.values
        else:
            vals = torch.from_numpy(np.ascontiguousarray(self.values))
        if dtype is None:
            dtype = torch.bfloat16 if vals.dtype == torch.bfloat16 else torch.float32
        vals = vals.to(device=dev, dtype=dtype).contiguous()
        if _is_torch(self.coords):
            coords = self.coords
        else:
            coords = torch.from_numpy(np.ascontiguousarray(self.coords, dtype=np.int32))
        coords = coords.to(device=dev, dtype=torch.int32).reshape(self.num_tuples,
                                                                  -1 if self.num_tuples else
                                                                  len(self.shape)).contiguous()
        return SparseTensorRelation(coords, vals, self.shape, self.tile_shape)

    def to_host(self) -> "SparseTensorRelation":
        """Copy to host NumPy (bfloat16 values become float32)."""
        if not _is_torch(self.values) and not _is_torch(self.coords):
            return self
        coords = self.coords.cpu().numpy() if _is_torch(self.coords) else self.coords
        vals = self.values
        if _is_torch(vals):
            import torch

            if vals.dtype == torch.bfloat16:
                vals = vals.float()
            vals = vals.cpu().numpy()
        return SparseTensorRelation(coords.astype(np.int32, copy=False), vals, self.shape,
                                    self.tile_shape)

    def to_dense(self):
        """Dense tensor from the tiles (sparse.py:75-90).  Host relations give
        a NumPy array; device relations are scattered on the GPU and give a
        torch tensor."""
        if self.is_device and self.ndim > 0:
            from .._device import relation_to_dense

            return relation_to_dense(self.coords, self.values, self.shape, self.tile_shape)
        rel = self.to_host()
        out = np.zeros(rel.shape, dtype=rel.values.dtype)
        for t in range(rel.num_tuples):
            c = rel.coords[t]
            sl = tuple(slice(int(c[d]) * rel.tile_shape[d], (int(c[d]) + 1) * rel.tile_shape[d])
                       for d in range(rel.ndim))
            out[sl] = rel.values[t]
        return out


def _extract_coo(data: Any) -> tuple[np.ndarray, np.ndarray, tuple]:
    """COO indices (int32 [nnz, nd]) and float64 values of host data
    (sparse.py:234-270)."""
    try:
        import scipy.sparse as sp

        if sp.issparse(data):
            coo = sp.coo_matrix(data) if data.ndim == 2 else data.tocoo()
            idx = np.stack([coo.row, coo.col], axis=1).astype(np.int32)
            return idx, np.asarray(coo.data, dtype=np.float64), tuple(coo.shape)
    except ImportError:  # pragma: no cover
        pass
    arr = np.asarray(data, dtype=np.float64)
    nz = np.nonzero(arr)
    if len(nz[0]) == 0:
        return np.zeros((0, arr.ndim), np.int32), np.zeros((0,), np.float64), tuple(arr.shape)
    return np.stack(nz, axis=1).astype(np.int32), arr[nz], tuple(arr.shape)


class SparseTensor:
    """Sparse tensor over dense or scipy-sparse data (sparse.py:93-231).

    ``data`` may be a NumPy array, a scipy sparse matrix, or a torch tensor
    (CPU or GPU).  ``to_relation`` buckets on the GPU."""

    def __init__(self, name: str, data: Any):
        self.name = name
        self.data = data
        if _is_torch(data):
            self.shape = tuple(int(s) for s in data.shape)
        elif hasattr(data, "shape") and not isinstance(data, np.ndarray) and _is_scipy(data):
            self.shape = tuple(int(s) for s in data.shape)
        else:
            self.data = np.asarray(data, dtype=np.float64)
            self.shape = tuple(self.data.shape)
        self.tile_shapes = enumerate_tile_shapes(self.shape)
        self._schemes: dict | None = None
        self._coo: tuple | None = None

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def _host_coo(self):
        if self._coo is None:
            data = self.data.cpu().numpy() if _is_torch(self.data) else self.data
            if _is_torch(self.data) and data.dtype != np.float64:
                data = data.astype(np.float64)
            self._coo = _extract_coo(data)
        return self._coo

    @property
    def nnz(self) -> int:
        return len(self._host_coo()[1])

    @property
    def schemes(self) -> dict:
        """tile_shape -> TilingScheme with num_tuples (non-empty tiles) and
        value_count (distinct tile coordinates per dimension), the reference's
        per-scheme statistics (sparse.py:124-158), computed on first access."""
        if self._schemes is None:
            idx, vals, _ = self._host_coo()
            nz = idx[vals != 0]
            schemes = {}
            for ts in self.tile_shapes:
                sch = TilingScheme(self, self.shape, ts)
                if len(nz) == 0:
                    sch.num_tuples = 0
                    sch.value_count = tuple(0 for _ in self.shape)
                else:
                    tc = nz // np.array(ts, dtype=np.int32)
                    sch.value_count = tuple(len(np.unique(tc[:, d])) for d in range(self.ndim))
                    sch.num_tuples = len(np.unique(tc, axis=0))
                schemes[ts] = sch
            self._schemes = schemes
        return self._schemes

    def to_relation(self, tile_shape: tuple) -> SparseTensorRelation:
        """Coordinate-to-tile bucketing on the GPU (reference: sparse.py:160-219).

        Tiles holding any element != 0 are kept, in lexicographic coordinate
        order, with the other elements of a kept tile set to +0.0.  Host data
        gives a host relation (int32 coords, float32 tiles: occupancy is
        decided on the float64 values, tiles hold them rounded to float32);
        GPU float32 / bfloat16 data gives a device relation of that dtype.
        Raises ValueError when a tile extent does not divide the shape."""
        tile_shape = tuple(int(t) for t in tile_shape)
        if len(tile_shape) != self.ndim:
            raise ValueError(f"tile_shape {tile_shape} has rank {len(tile_shape)}, "
                             f"tensor has rank {self.ndim}")
        for d in range(self.ndim):
            if self.shape[d] % tile_shape[d] != 0:
                raise ValueError(f"tile_shape[{d}]={tile_shape[d]} does not evenly divide "
                                 f"shape[{d}]={self.shape[d]}")
        import torch

        from .._device import bucket_dense, require_gpu

        dev = require_gpu()
        on_device = _is_torch(self.data) and self.data.is_cuda
        if _is_torch(self.data):
            dense = self.data
            if dense.dtype not in (torch.float32, torch.bfloat16, torch.float64):
                dense = dense.to(torch.float64 if not on_device else torch.float32)
            dense = dense.to(dev)
        elif _is_scipy(self.data):
            dense = torch.from_numpy(np.asarray(self.data.toarray(), dtype=np.float64)).to(dev)
        else:
            dense = torch.from_numpy(np.ascontiguousarray(self.data)).to(dev)
        if prod(self.shape) == 0:
            coords = torch.zeros((0, self.ndim), dtype=torch.int32, device=dev)
            vals = torch.zeros((0, *tile_shape), dtype=torch.float32, device=dev)
        else:
            coords, vals = bucket_dense(dense, tile_shape)
        rel = SparseTensorRelation(coords, vals, self.shape, tile_shape)
        return rel if on_device else rel.to_host()

    def to_dense_array(self) -> np.ndarray:
        """Dense float64 array of the data (sparse.py:221-231)."""
        if _is_torch(self.data):
            return self.data.float().cpu().numpy().astype(np.float64)
        if _is_scipy(self.data):
            return np.asarray(self.data.toarray(), dtype=np.float64)
        return np.array(self.data, dtype=np.float64)


def _is_scipy(x) -> bool:
    try:
        import scipy.sparse as sp

        return sp.issparse(x)
    except ImportError:  # pragma: no cover
        return False
