"""Seeded synthetic relations for the five benchmark workloads.

Test infrastructure only (see ``oracle/__init__.py``).  Relations are built
directly in tensor-relational form: the chosen tile coordinates are sorted
lexicographically (the order to_relation produces, tensor/sparse.py:204-206)
and every element of a chosen tile is nonzero, so each relation equals
to_relation of the dense tensor it describes.  Generation protocol:
``numpy.random.default_rng(seed)``; nonzero tiles are
``rng.choice(n_tiles, k=round(density * n_tiles), replace=False)`` then
sorted; bf16 means round-to-nearest-even from float32.

With values=False only coordinates are generated (value arrays are empty);
the coordinates are the same as with values=True (every coordinate draw
precedes the value draws it could disturb).  Each workload returns a dict
with lhs / rhs (``Rel`` with float32 values that
are bf16-representable when dtype == "bf16"), join_keys, agg_keys,
kernel_string and dtype.
"""

from __future__ import annotations

import numpy as np

from .reference_path import Rel, bf16_round


def _choose_tiles(rng, grid: tuple, density: float) -> np.ndarray:
    n = int(np.prod(grid))
    k = int(round(density * n))
    flat = np.sort(rng.choice(n, size=k, replace=False))
    return np.stack(np.unravel_index(flat, grid), axis=1).astype(np.int32)


def _all_tiles(grid: tuple) -> np.ndarray:
    n = int(np.prod(grid))
    return np.stack(np.unravel_index(np.arange(n), grid), axis=1).astype(np.int32)


def _normal(rng, shape, scale=1.0, dtype="fp32", values=True):
    if not values:
        return np.zeros((0, *shape[1:]), np.float32)
    v = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(scale)
    return bf16_round(v) if dtype == "bf16" else v


def workload_blocksparse_1k(seed: int = 0, n: int = 1024, tile: int = 32, density: float = 0.10, values: bool = True):
    """'ij,jk->ik': A n x n fp32, tile x tile tiles, `density` of tiles nonzero,
    N(0,1); B dense n x n fp32 N(0,1) as a tile relation."""
    rng = np.random.default_rng(seed)
    g = (n // tile, n // tile)
    ac = _choose_tiles(rng, g, density)
    av = _normal(rng, (len(ac), tile, tile), values=values)
    bc = _all_tiles(g)
    bv = _normal(rng, (len(bc), tile, tile), values=values)
    return dict(
        name=f"blocksparse_{n}_t{tile}_d{density:g}_fp32",
        lhs=Rel(ac, av, (n, n), (tile, tile)), rhs=Rel(bc, bv, (n, n), (tile, tile)),
        join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)], kernel_string="ij,jk->ik", dtype="fp32")


def workload_blocksparse_16k(seed: int = 0, m: int = 16384, n: int = 4096, tile: int = 128,
                             density: float = 0.05, values: bool = True):
    """'ij,jk->ik': A m x m bf16, tile^2 tiles, 5% tile density uniform, N(0,1);
    B dense m x n bf16 N(0, 1/sqrt(m)); fp32 accumulate."""
    rng = np.random.default_rng(seed)
    ga = (m // tile, m // tile)
    ac = _choose_tiles(rng, ga, density)
    av = _normal(rng, (len(ac), tile, tile), dtype="bf16", values=values)
    gb = (m // tile, n // tile)
    bc = _all_tiles(gb)
    bv = _normal(rng, (len(bc), tile, tile), scale=1.0 / np.sqrt(m), dtype="bf16",
                 values=values)
    return dict(
        name=f"blocksparse_{m}x{m}_x_dense_{m}x{n}_t{tile}_d{density:g}_bf16",
        lhs=Rel(ac, av, (m, m), (tile, tile)), rhs=Rel(bc, bv, (m, n), (tile, tile)),
        join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)], kernel_string="ij,jk->ik", dtype="bf16")


def _zipf_tiles(rng, grid_rows: int, grid_cols: int, k: int, s: float) -> np.ndarray:
    p = (np.arange(grid_rows) + 1.0) ** (-s)
    p /= p.sum()
    chosen: set = set()
    out = []
    while len(out) < k:
        need = k - len(out)
        rows = rng.choice(grid_rows, size=2 * need, p=p)
        cols = rng.integers(0, grid_cols, size=2 * need)
        for r, c in zip(rows.tolist(), cols.tolist()):
            if (r, c) not in chosen:
                chosen.add((r, c))
                out.append((r, c))
                if len(out) == k:
                    break
    arr = np.array(sorted(out), dtype=np.int32)
    return arr


def workload_sparse_sparse_zipf(seed: int = 0, n: int = 32768, tile: int = 64,
                                density: float = 0.02, s: float = 1.2, values: bool = True):
    """'ij,jk->ik': A, B n x n fp32, tile^2 tiles, `density` of tiles, row-tile
    occupancy Zipf(s) (p ~ (r+1)^-s), columns uniform, U(-1,1) values."""
    rng = np.random.default_rng(seed)
    g = n // tile
    k = int(round(density * g * g))
    ac = _zipf_tiles(rng, g, g, k, s)
    bc = _zipf_tiles(rng, g, g, k, s)
    if values:
        av = rng.uniform(-1, 1, size=(k, tile, tile)).astype(np.float32)
        bv = rng.uniform(-1, 1, size=(k, tile, tile)).astype(np.float32)
    else:
        av = bv = np.zeros((0, tile, tile), np.float32)
    return dict(
        name=f"sparse_{n}_x_sparse_t{tile}_d{density:g}_zipf{s:g}_fp32",
        lhs=Rel(ac, av, (n, n), (tile, tile)), rhs=Rel(bc, bv, (n, n), (tile, tile)),
        join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)], kernel_string="ij,jk->ik", dtype="fp32")


def workload_batched_banded(seed: int = 0, b: int = 32, n: int = 4096, tile: int = 64,
                            band: int = 8, values: bool = True):
    """'bij,bjk->bik' as 3-D relations with tile (1, tile, tile): A per batch
    the causal band {(i, j): 0 <= i - j < band} of tiles, B dense; bf16 N(0,1)."""
    rng = np.random.default_rng(seed)
    g = n // tile
    band_tiles = [(i, j) for i in range(g) for j in range(g) if 0 <= i - j < band]
    ac = np.array([(bb, i, j) for bb in range(b) for (i, j) in band_tiles], dtype=np.int32)
    av = _normal(rng, (len(ac), 1, tile, tile), dtype="bf16", values=values)
    bc = _all_tiles((b, g, g))
    bv = _normal(rng, (len(bc), 1, tile, tile), dtype="bf16", values=values)
    return dict(
        name=f"batched_banded_b{b}_{n}_t{tile}_band{band}_bf16",
        lhs=Rel(ac, av, (b, n, n), (1, tile, tile)), rhs=Rel(bc, bv, (b, n, n), (1, tile, tile)),
        join_keys=[(0, 0), (2, 1)], agg_keys=[(0, 0), (0, 1), (1, 2)],
        kernel_string="bij,bjk->bik", dtype="bf16")


def workload_order3(seed: int = 0, n: int = 2048, l: int = 512, tile: int = 32,
                    density: float = 0.005, values: bool = True):
    """'ijk,kl->ijl': X n^3 fp32 tile^3 tiles at `density`, N(0,1); W n x l fp32
    dense N(0,1); output stays a relation."""
    rng = np.random.default_rng(seed)
    g = n // tile
    xc = _choose_tiles(rng, (g, g, g), density)
    xv = _normal(rng, (len(xc), tile, tile, tile), values=values)
    wc = _all_tiles((g, l // tile))
    wv = _normal(rng, (len(wc), tile, tile), values=values)
    return dict(
        name=f"order3_{n}^3_t{tile}_d{density:g}_x_dense_{n}x{l}_fp32",
        lhs=Rel(xc, xv, (n, n, n), (tile, tile, tile)), rhs=Rel(wc, wv, (n, l), (tile, tile)),
        join_keys=[(2, 0)], agg_keys=[(0, 0), (0, 1), (1, 1)], kernel_string="ijk,kl->ijl",
        dtype="fp32")


WORKLOADS = {
    "blocksparse_1k": workload_blocksparse_1k,
    "blocksparse_16k_bf16": workload_blocksparse_16k,
    "sparse_sparse_zipf": workload_sparse_sparse_zipf,
    "batched_banded_bf16": workload_batched_banded,
    "order3": workload_order3,
}
