"""Dense tensor metadata for tile-shape selection (reference: tensor/dense.py).

The reference's DenseTensor holds an array and the per-tile-shape
statistics of its nonzero elements (dense.py:19-99), which the tiling
surface ranks (tensor/tiling.py).  Here the statistics are counted on the
GPU on first access of ``schemes``, by the same kernels as SparseTensor's.
Dense einsum execution is not part of this library.
"""

from __future__ import annotations

from typing import Any

import numpy as np

from .sparse import _dense_on_gpu, _is_torch, _measured_schemes
from .tiling import enumerate_tile_shapes


class DenseTensor:
    """A dense array and its tiling schemes (reference: tensor/dense.py:19-66).

    ``data`` may be a NumPy array or a torch tensor (CPU or GPU); it is kept
    as given.  ``schemes`` maps every tile shape to a TilingScheme whose
    num_tuples / value_count count the tiles holding an element != 0."""

    def __init__(self, name: str, data: Any):
        self.name = name
        self.data = data
        if _is_torch(data):
            self.shape = tuple(int(s) for s in data.shape)
        else:
            self.shape = tuple(np.asarray(data).shape)
        self.tile_shapes = enumerate_tile_shapes(self.shape)
        self._schemes: dict | None = None
        self._gpu = None

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def _gpu_form(self) -> tuple:
        if self._gpu is None:
            self._gpu = ("dense", _dense_on_gpu(self.data)[0])
        return self._gpu

    @property
    def schemes(self) -> dict:
        if self._schemes is None:
            self._schemes = _measured_schemes(self, self._gpu_form)
        return self._schemes
