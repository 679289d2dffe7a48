"""Coordinate joins on bare coordinate arrays (reference: kernels/pallas_gather.py).

Both run on the GPU join kernels; they differ only in the pair order they
return, which matches the corresponding reference function exactly.
"""

from __future__ import annotations

import numpy as np

from .. import _device, _lib
from ..execution.sparse_dispatch import (_column_shifts, _dev_coords, _host, _on_host,
                                         _shift_columns)


def _norm(join_dims) -> list:
    if join_dims and isinstance(join_dims[0], (int, np.integer)):
        return [(int(d), int(d)) for d in join_dims]
    return [tuple(int(x) for x in k) for k in join_dims]


def _join(lhs_coords, rhs_coords, join_dims, order):
    import torch

    host = _on_host(lhs_coords, rhs_coords)
    keys = _norm(join_dims)
    n_l, n_r = int(lhs_coords.shape[0]), int(rhs_coords.shape[0])
    if n_l == 0 or n_r == 0:
        e = np.array([], dtype=np.int64)
        if host:
            return e, e.copy()
        dev = _device.require_gpu()
        return (torch.zeros(0, dtype=torch.int64, device=dev),
                torch.zeros(0, dtype=torch.int64, device=dev))
    lc = _dev_coords(lhs_coords, lhs_coords.shape[1] if lhs_coords.ndim > 1 else 1)
    rc = _dev_coords(rhs_coords, rhs_coords.shape[1] if rhs_coords.ndim > 1 else 1)
    radices = []
    if keys:
        llo, lhi = _device.coords_range(lc)
        rlo, rhi = _device.coords_range(rc)
        if any(llo[a] < 0 or rlo[b] < 0 for a, b in keys):
            # negative key columns: joined columns shifted by one common
            # minimum, which keeps the match set and both pair orders
            sl, sr = _column_shifts(lc, rc, keys, [])
            lc, rc = _shift_columns(lc, sl), _shift_columns(rc, sr)
            llo, lhi = _device.coords_range(lc)
            rlo, rhi = _device.coords_range(rc)
        for a, b in keys:
            radices.append(max(lhi[a], rhi[b]) + 1)
    li, ri = _device.join(lc, rc, keys, radices, order)
    return (_host(li), _host(ri)) if host else (li, ri)


def coordinate_join_hash(lhs_coords, rhs_coords, join_dims):
    """Hash-join pair order: rhs index ascending, then lhs index ascending;
    ints in join_dims mean the same dim on both sides; an empty side gives
    empty int64 arrays; no keys gives the lhs-major cross product
    (reference: pallas_gather.py:19-76)."""
    return _join(lhs_coords, rhs_coords, join_dims, _lib.EJ_ORDER_PROBE)


def coordinate_join_sorted(lhs_coords, rhs_coords, join_dims):
    """Sort-merge pair order: key tuple ascending, then the lhs-major product
    of the stably sorted equal-key runs (reference: pallas_gather.py:79-174)."""
    return _join(lhs_coords, rhs_coords, join_dims, _lib.EJ_ORDER_SORTED)
