"""Tensor-relational containers (reference: tensor/sparse.py).

``SparseTensorRelation`` keeps the reference's fields and properties
(tensor/sparse.py:27-90).  Its arrays are either host NumPy arrays, as in the
reference, or torch tensors resident on the GPU; every operation of the
sparse path accepts both and answers in the residency it was given, so host
callers see the reference's types while chained device calls never leave
HBM.

``SparseTensor`` (tensor/sparse.py:93-231) counts, buckets and measures its
data on the GPU.  Its per-scheme statistics (``schemes``, the reference's
``_compute_sparsity_metrics``, :124-158) are computed on first access rather
than in the constructor, so building a relation does not pay for them.
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

    @classmethod
    def _from_parts(cls, coords, values, shape: tuple, tile_shape: tuple):
        """A relation from parts already in normal form (shape and tile_shape
        tuples of ints), without the constructor's conversions."""
        rel = object.__new__(cls)
        rel.coords, rel.values, rel.shape, rel.tile_shape = coords, values, shape, tile_shape
        return rel

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


def _extract_coo(data: Any):
    """COO indices (int32 [nnz, nd]) and float64 values of the data, with
    its shape (reference: _extract_coo, tensor/sparse.py:234-270).

    A scipy sparse matrix gives its stored entries (scipy's own COO
    conversion, explicit zeros and repeats included).  A dense array gives
    its elements != 0 in row-major order, found on the GPU; host input
    answers in NumPy, GPU input in torch tensors on the GPU."""
    if _is_scipy(data):
        coo = data.tocoo()
        idx = np.stack([coo.row, coo.col], axis=1).astype(np.int32)
        return idx, np.asarray(coo.data, dtype=np.float64), tuple(int(s) for s in coo.shape)
    from .._device import extract_coo

    dense, on_device = _dense_on_gpu(data)
    shape = tuple(int(s) for s in dense.shape)
    if dense.numel() == 0 or dense.dim() == 0:
        import torch

        flat = dense.reshape(-1)
        keep = flat != 0
        if on_device:  # a 0-d tensor: one element, no kernel needed
            return (torch.zeros((int(keep.sum()), dense.dim()), dtype=torch.int32,
                                device=dense.device), flat[keep].double(), shape)
        return (np.zeros((int(keep.sum()), dense.dim()), np.int32),
                flat[keep].double().cpu().numpy(), shape)
    idx, vals = extract_coo(dense)
    if on_device:
        return idx, vals, shape
    return idx.cpu().numpy(), vals.cpu().numpy(), shape


def _dense_on_gpu(data):
    """(dense torch tensor on the GPU, whether the input already was there).
    float32 / bfloat16 / float64 stay as they are; other dtypes become
    float64 on the host side (the reference's np.asarray(..., float64)) and
    float32 on the GPU."""
    import torch

    from .._device import require_gpu

    dev = require_gpu()
    if _is_torch(data):
        on_device = data.is_cuda
        t = data
        if t.dtype not in (torch.float32, torch.bfloat16, torch.float64):
            t = t.to(torch.float32 if on_device else torch.float64)
        return t.to(dev).contiguous(), on_device
    arr = np.ascontiguousarray(np.asarray(data, dtype=np.float64))
    return torch.from_numpy(arr).to(dev), False


class SparseTensor:
    """Sparse tensor over dense or scipy-sparse data (sparse.py:93-231).

    ``data`` may be a NumPy array, a scipy sparse matrix, or a torch tensor
    (CPU or GPU).  Nonzero counting, the per-tile-shape statistics and
    ``to_relation`` run on the GPU; the data is copied there once, on first
    use, and kept (dense data as a dense tensor, scipy data as COO entries)."""

    def __init__(self, name: str, data: Any):
        self.name = name
        self.data = data
        if _is_torch(data) or _is_scipy(data):
            self.shape = tuple(int(s) for s in data.shape)
        else:
            self.data = np.asarray(data, dtype=np.float64)
            self.shape = tuple(self.data.shape)
        self.tile_shapes = enumerate_tile_shapes(self.shape)
        self._schemes: dict | None = None
        self._gpu: tuple | None = None
        self._nnz: int | None = None
        self._coo_host: tuple | None = None

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def _gpu_form(self) -> tuple:
        """("dense", tensor) or ("coo", indices int32 [n, nd], values float64 [n]),
        resident on the GPU."""
        if self._gpu is None:
            if _is_scipy(self.data):
                import torch

                from .._device import require_gpu

                dev = require_gpu()
                idx, vals, _ = _extract_coo(self.data)
                self._gpu = ("coo", torch.from_numpy(idx).to(dev), torch.from_numpy(vals).to(dev))
            else:
                self._gpu = ("dense", _dense_on_gpu(self.data)[0])
        return self._gpu

    @property
    def nnz(self) -> int:
        """Stored entries: elements != 0 of dense data, stored entries of a
        scipy matrix (sparse.py:119-122 over :234-270)."""
        if self._nnz is None:
            form = self._gpu_form()
            if form[0] == "coo":
                self._nnz = int(form[2].numel())
            else:
                from .._device import count_nonzero

                self._nnz = count_nonzero(form[1]) if form[1].numel() else 0
        return self._nnz

    @property
    def _indices(self) -> np.ndarray:
        """Host COO indices int32 [nnz, nd] (the reference's attribute)."""
        return self._host_coo()[0]

    @property
    def _values(self) -> np.ndarray:
        """Host COO values float64 [nnz] (the reference's attribute)."""
        return self._host_coo()[1]

    def _host_coo(self):
        if self._coo_host is None:
            idx, vals, _ = _extract_coo(self.data)
            if _is_torch(idx):
                idx, vals = idx.cpu().numpy(), vals.cpu().numpy()
            self._coo_host = (idx, vals)
        return self._coo_host

    @property
    def schemes(self) -> dict:
        """tile_shape -> TilingScheme with num_tuples (non-empty tiles) and
        value_count (distinct tile coordinates per dimension), the reference's
        per-scheme statistics (sparse.py:124-158), computed on the GPU for
        every tile shape at once on first access."""
        if self._schemes is None:
            self._schemes = _measured_schemes(self, self._gpu_form)
        return self._schemes

    def to_relation(self, tile_shape: tuple) -> SparseTensorRelation:
        """Coordinate-to-tile bucketing on the GPU (reference: sparse.py:160-219).

        Tiles holding any element != 0 are kept, in lexicographic coordinate
        order, with the other elements of a kept tile set to +0.0.  Host data
        gives a host relation with int32 coords and float64 tiles, as the
        reference's (sparse.py:191, :210); GPU float64 / float32 / bfloat16
        data gives a device relation of that dtype.
        scipy data is bucketed from its COO entries (a repeated entry keeps
        its last nonzero value) without forming the dense matrix.
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

        from .._device import bucket_coo, bucket_dense

        on_device = _is_torch(self.data) and self.data.is_cuda
        form = self._gpu_form()
        dev = form[1].device
        if prod(self.shape) == 0:
            coords = torch.zeros((0, self.ndim), dtype=torch.int32, device=dev)
            vals = torch.zeros((0, *tile_shape), dtype=form[-1].dtype if form[0] == "coo"
                               else form[1].dtype, device=dev)
        elif form[0] == "coo":
            coords, vals = bucket_coo(form[1], form[2], self.shape, tile_shape)
        else:
            coords, vals = bucket_dense(form[1], tile_shape)
        rel = SparseTensorRelation(coords, vals, self.shape, tile_shape)
        return rel if on_device else rel.to_host()

    def to_dense_array(self) -> np.ndarray:
        """Dense float64 array of the data (sparse.py:221-231); stored entries
        of a scipy matrix are written in order, so a repeated entry keeps the
        last value."""
        if _is_torch(self.data):
            return self.data.double().cpu().numpy()
        if _is_scipy(self.data):
            idx, vals, _ = _extract_coo(self.data)
            out = np.zeros(self.shape, dtype=np.float64)
            if len(vals):
                out[tuple(idx[:, d] for d in range(self.ndim))] = vals
            return out
        return np.array(self.data, dtype=np.float64)


def _measured_schemes(tensor, gpu_form) -> dict:
    """tile_shape -> TilingScheme of `tensor` (shape, tile_shapes, ndim),
    with num_tuples and value_count counted on the GPU over the elements
    != 0 of gpu_form() for every tile shape in one call (the reference's
    _compute_sparsity_metrics, sparse.py:124-158 and dense.py:44-66)."""
    schemes = {ts: TilingScheme(tensor, tensor.shape, ts) for ts in tensor.tile_shapes}
    form = gpu_form()
    if tensor.ndim == 0:
        if form[0] == "coo":
            n = 1 if int(form[2].numel()) else 0
        else:
            n = 1 if bool((form[1] != 0).any()) else 0
        for sch in schemes.values():
            sch.num_tuples, sch.value_count = n, ()
        return schemes
    from .._device import scheme_stats

    if form[0] == "coo":
        nt, vc = scheme_stats(tensor.tile_shapes, tensor.shape, indices=form[1], values=form[2])
    else:
        nt, vc = scheme_stats(tensor.tile_shapes, tensor.shape, dense=form[1])
    for ts, n, v in zip(tensor.tile_shapes, nt, vc):
        schemes[ts].num_tuples = n
        schemes[ts].value_count = v
    return schemes


def _is_scipy(x) -> bool:
    try:
        import scipy.sparse as sp

        return sp.issparse(x)
    except ImportError:  # pragma: no cover
        return False
