"""Writes tests/golden/join_order.npz: join pair-order golden vectors.

The pair ORDER of the reference's joins is pinned by no reference test (its
tests compare counts and pair sets only), so this script runs the
reference's own jax-free join module, kernels/pallas_gather.py, loaded by
file path from the read-only reference checkout, on seeded inputs and
stores inputs and outputs as fixtures.  coordinate_join
(execution/sparse_dispatch.py:29-82) builds and probes the same dict in the
same loops as coordinate_join_hash (kernels/pallas_gather.py:59-74), so the
hash vectors pin both; the module that holds coordinate_join imports jax and
is not importable here.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np

REF = Path("/root/reference/kernels/pallas_gather.py")
OUT = Path(__file__).resolve().parent / "join_order.npz"


def _load():
    spec = importlib.util.spec_from_file_location("ref_pallas_gather", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def cases():
    """(name, lhs_coords, rhs_coords, join_dims) with duplicate keys, several
    key columns, skew and the cross product."""
    rng = np.random.RandomState(42)
    out = []
    # the reference test's own random input (tests/test_pallas.py:326-338)
    out.append(("rs42_50x2_k10", rng.randint(0, 5, size=(50, 2)).astype(np.int32),
                rng.randint(0, 5, size=(50, 2)).astype(np.int32), [(1, 0)]))
    rng = np.random.default_rng(7)
    out.append(("dup_200x3_k2", rng.integers(0, 4, size=(200, 3)).astype(np.int32),
                rng.integers(0, 4, size=(150, 3)).astype(np.int32), [(2, 0), (0, 1)]))
    out.append(("skew_300x2", np.stack([rng.integers(0, 3, 300), (rng.zipf(1.5, 300) % 17)],
                                       axis=1).astype(np.int32),
                np.stack([(rng.zipf(1.5, 260) % 17), rng.integers(0, 9, 260)],
                         axis=1).astype(np.int32), [(1, 0)]))
    out.append(("same_dim_int", rng.integers(0, 6, size=(80, 2)).astype(np.int32),
                rng.integers(0, 6, size=(90, 2)).astype(np.int32), [0, 1]))
    out.append(("cross_7x5", rng.integers(0, 9, size=(7, 2)).astype(np.int32),
                rng.integers(0, 9, size=(5, 2)).astype(np.int32), []))
    out.append(("large_4000x2", rng.integers(0, 64, size=(4000, 2)).astype(np.int32),
                rng.integers(0, 64, size=(3000, 2)).astype(np.int32), [(1, 0)]))
    out.append(("three_keys_3d", rng.integers(0, 3, size=(500, 3)).astype(np.int32),
                rng.integers(0, 3, size=(400, 4)).astype(np.int32), [(0, 3), (1, 1), (2, 0)]))
    return out


def main():
    mod = _load()
    arrays = {}
    names = []
    for name, lc, rc, jd in cases():
        h_l, h_r = mod.coordinate_join_hash(lc, rc, jd)
        s_l, s_r = mod.coordinate_join_sorted(lc, rc, jd)
        norm = [(d, d) for d in jd] if jd and isinstance(jd[0], int) else list(jd)
        arrays[f"{name}__lhs"] = lc
        arrays[f"{name}__rhs"] = rc
        arrays[f"{name}__keys"] = np.array(norm, dtype=np.int32).reshape(-1, 2)
        arrays[f"{name}__int_dims"] = np.array(bool(jd) and isinstance(jd[0], int))
        arrays[f"{name}__hash_lhs"] = np.asarray(h_l, dtype=np.int64)
        arrays[f"{name}__hash_rhs"] = np.asarray(h_r, dtype=np.int64)
        arrays[f"{name}__sorted_lhs"] = np.asarray(s_l, dtype=np.int64)
        arrays[f"{name}__sorted_rhs"] = np.asarray(s_r, dtype=np.int64)
        names.append(name)
    arrays["names"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(names)} cases)")


if __name__ == "__main__":
    main()
