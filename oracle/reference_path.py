"""NumPy restatement of the reference's sparse-einsum path (the oracle).

Test infrastructure only (see ``oracle/__init__.py``).  Every function
restates one reference function; the docstring names the reference
file:line range it follows.  Relations are plain tuples here
``Rel(coords, values, shape, tile_shape)`` so that the oracle shares no code
with the product package.
"""

from __future__ import annotations

from math import prod
from typing import NamedTuple

import numpy as np


class Rel(NamedTuple):
    """Tensor-relational form: coords int32 [T, nd], values [T, *tile]
    (tensor/sparse.py:27-47)."""

    coords: np.ndarray
    values: np.ndarray
    shape: tuple
    tile_shape: tuple


# ---------------------------------------------------------------------------
# bf16 helpers (the reference has no bf16; bf16 inputs mean fp32 math on
# bf16-rounded values).

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Rounds float32 values to the nearest bfloat16 (ties to even), returned
    as float32.  NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values that are already
    bf16-representable."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# Tiling.

def extract_coo(data) -> tuple[np.ndarray, np.ndarray, tuple]:
    """COO extraction (tensor/sparse.py:234-270): scipy sparse -> row/col
    stack; dense -> np.nonzero in row-major order; values always float64."""
    try:
        import scipy.sparse as sp

        if sp.issparse(data):
            coo = sp.coo_matrix(data)
            idx = np.stack([coo.row, coo.col], axis=1).astype(np.int32)
            return idx, np.asarray(coo.data, dtype=np.float64), tuple(coo.shape)
    except ImportError:  # pragma: no cover
        pass
    arr = np.asarray(data, dtype=np.float64)
    nz = np.nonzero(arr)
    if len(nz[0]) == 0:
        return np.zeros((0, arr.ndim), np.int32), np.zeros((0,), np.float64), tuple(arr.shape)
    return np.stack(nz, axis=1).astype(np.int32), arr[nz], tuple(arr.shape)


def to_relation(indices: np.ndarray, values: np.ndarray, shape: tuple, tile_shape: tuple) -> Rel:
    """Coordinate-to-tile bucketing (tensor/sparse.py:160-219): drop zero
    values (:184-187), tile coord = idx // tile, offset = idx % tile
    (:200-201), distinct tile coords in lexicographic order via
    np.unique(axis=0) (:204-206), scatter into float64 zero tiles (:210-212).
    Raises ValueError when a tile does not divide the shape (:174-179)."""
    nd = len(shape)
    for d in range(nd):
        if shape[d] % tile_shape[d] != 0:
            raise ValueError(
                f"tile_shape[{d}]={tile_shape[d]} does not evenly divide shape[{d}]={shape[d]}")
    keep = values != 0
    idx = indices[keep]
    vals = values[keep]
    if len(vals) == 0:
        return Rel(np.zeros((0, nd), np.int32), np.zeros((0, *tile_shape), np.float64),
                   tuple(shape), tuple(tile_shape))
    t = np.array(tile_shape, dtype=np.int32)
    tc = idx // t
    within = idx % t
    uniq, inv = np.unique(tc, axis=0, return_inverse=True)
    inv = np.asarray(inv).reshape(-1)
    out = np.zeros((len(uniq), *tile_shape), np.float64)
    out[(inv,) + tuple(within[:, d] for d in range(nd))] = vals
    return Rel(uniq.astype(np.int32), out, tuple(shape), tuple(tile_shape))


def dense_to_relation(dense: np.ndarray, tile_shape: tuple) -> Rel:
    """SparseTensor(name, dense).to_relation(tile_shape) without the
    per-scheme statistics (tensor/sparse.py:104-117 then :160-219)."""
    idx, vals, shape = extract_coo(dense)
    return to_relation(idx, vals, shape, tile_shape)


def divisors(n: int) -> list:
    """Divisors of n ascending (core/notation.py:27-44); n <= 0 raises."""
    if n <= 0:
        raise ValueError(f"n must be positive, got {n}")
    return [d for d in range(1, n + 1) if n % d == 0]


def all_tile_shapes(shape: tuple) -> list:
    """Every tile shape of a tensor, the product of the per-dimension
    divisor lists in itertools.product order (tensor/base.py:39-49)."""
    out = [()]
    for n in shape:
        out = [ts + (d,) for ts in out for d in divisors(n)]
    return out


def sparsity_metrics(indices: np.ndarray, values: np.ndarray, tile_shapes) -> dict:
    """Per-tile-shape statistics (tensor/sparse.py:124-158): over the entries
    with value != 0 (:139-141), num_tuples = number of distinct rows of
    indices // tile_shape (np.unique(axis=0), :156-157) and value_count[d] =
    number of distinct values in column d (:152-154); all zero when no entry
    is nonzero (:143-147).  Returns {tile_shape: (num_tuples, value_count)}."""
    nz = np.asarray(indices)[np.asarray(values) != 0]
    out = {}
    for ts in tile_shapes:
        nd = len(ts)
        if len(nz) == 0:
            out[tuple(ts)] = (0, tuple(0 for _ in range(nd)))
            continue
        tc = nz // np.array(ts, dtype=np.int64)
        vc = tuple(len(np.unique(tc[:, d])) for d in range(nd))
        out[tuple(ts)] = (len(np.unique(tc, axis=0)), vc)
    return out


def relation_to_dense(rel: Rel) -> np.ndarray:
    """SparseTensorRelation.to_dense (tensor/sparse.py:75-90): tiles written in
    order into a zero array of the values' dtype."""
    out = np.zeros(rel.shape, dtype=rel.values.dtype)
    for t in range(rel.coords.shape[0]):
        c = rel.coords[t]
        sl = tuple(slice(int(c[d]) * rel.tile_shape[d], (int(c[d]) + 1) * rel.tile_shape[d])
                   for d in range(len(rel.shape)))
        out[sl] = rel.values[t]
    return out


# ---------------------------------------------------------------------------
# Join.

def coordinate_join(lhs_coords: np.ndarray, rhs_coords: np.ndarray, join_keys) -> tuple:
    """Hash join (execution/sparse_dispatch.py:29-82): no keys -> lhs-major
    cross product (:53-59); else a dict from lhs key tuple to the lhs
    indices in ascending order (:65-69), probed by each rhs row in order
    (:71-80).  Pair order: rhs index ascending, then lhs index ascending."""
    n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
    if not join_keys:
        return np.repeat(np.arange(n_l), n_r), np.tile(np.arange(n_r), n_l)
    ld = [k[0] for k in join_keys]
    rd = [k[1] for k in join_keys]
    table: dict = {}
    for i in range(n_l):
        table.setdefault(tuple(int(lhs_coords[i, d]) for d in ld), []).append(i)
    lm, rm = [], []
    for j in range(n_r):
        key = tuple(int(rhs_coords[j, d]) for d in rd)
        for i in table.get(key, ()):
            lm.append(i)
            rm.append(j)
    return np.array(lm, dtype=np.int64), np.array(rm, dtype=np.int64)


def _norm_join_dims(join_dims):
    if join_dims and isinstance(join_dims[0], (int, np.integer)):
        return [(int(d), int(d)) for d in join_dims]
    return [tuple(k) for k in join_dims]


def coordinate_join_hash(lhs_coords, rhs_coords, join_dims) -> tuple:
    """kernels/pallas_gather.py:19-76: join_dims may be ints (same dim on both
    sides, :39-42); an empty side returns empty int64 arrays (:47-48) before
    the cross-product case (:50-54); otherwise the same dict join and order
    as coordinate_join (:59-74)."""
    keys = _norm_join_dims(join_dims)
    if lhs_coords.shape[0] == 0 or rhs_coords.shape[0] == 0:
        return np.array([], dtype=np.int64), np.array([], dtype=np.int64)
    return coordinate_join(lhs_coords, rhs_coords, keys)


def coordinate_join_sorted(lhs_coords, rhs_coords, join_dims) -> tuple:
    """kernels/pallas_gather.py:79-174: both sides stably sorted by key tuple
    (np.lexsort over the reversed key columns, :131-132), merged; for each
    equal-key group the lhs-major nested product of the two sorted runs
    (:144-172).  Pair order: key ascending, lhs sorted rank, rhs sorted rank."""
    keys = _norm_join_dims(join_dims)
    n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
    if n_l == 0 or n_r == 0:
        return np.array([], dtype=np.int64), np.array([], dtype=np.int64)
    if not keys:
        return np.repeat(np.arange(n_l), n_r), np.tile(np.arange(n_r), n_l)
    lk = np.stack([lhs_coords[:, a].astype(np.int64) for a, _ in keys], axis=1)
    rk = np.stack([rhs_coords[:, b].astype(np.int64) for _, b in keys], axis=1)
    lo = np.lexsort(lk.T[::-1])
    ro = np.lexsort(rk.T[::-1])
    slk, srk = lk[lo], rk[ro]
    lm, rm = [], []
    i = j = 0
    while i < n_l and j < n_r:
        a, b = tuple(slk[i]), tuple(srk[j])
        if a < b:
            i += 1
        elif a > b:
            j += 1
        else:
            i0 = i
            while i < n_l and tuple(slk[i]) == a:
                i += 1
            j0 = j
            while j < n_r and tuple(srk[j]) == b:
                j += 1
            for ii in range(i0, i):
                for jj in range(j0, j):
                    lm.append(int(lo[ii]))
                    rm.append(int(ro[jj]))
    return np.array(lm, dtype=np.int64), np.array(rm, dtype=np.int64)


# ---------------------------------------------------------------------------
# Tile einsum.

def add_batch_dim(kernel_string: str, batch_label: str = "z") -> str:
    """execution/sparse_dispatch.py:481-503."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    ins, out = kernel_string.split("->")
    return ",".join(batch_label + t for t in ins.split(",")) + "->" + batch_label + out


def infer_output_tile_shape(kernel_string: str, lhs_tile: tuple, rhs_tile: tuple) -> tuple:
    """execution/sparse_dispatch.py:506-545: label sizes from the lhs term,
    overridden by the rhs term (:533-541); KeyError for an unknown output
    label (:544)."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    ins, out = kernel_string.split("->")
    terms = ins.split(",")
    sizes: dict = {}
    if len(terms) >= 1:
        for d, lab in enumerate(terms[0]):
            if d < len(lhs_tile):
                sizes[lab] = lhs_tile[d]
    if len(terms) >= 2:
        for d, lab in enumerate(terms[1]):
            if d < len(rhs_tile):
                sizes[lab] = rhs_tile[d]
    return tuple(sizes[lab] for lab in out)


def kernel_einsum(lhs_values, rhs_values, lhs_idx, rhs_idx, kernel_string, precision="fp32"):
    """execution/sparse_dispatch.py:85-126: empty pairs -> zeros of the lhs
    dtype with the inferred output tile shape (:108-115); else gather the
    matched tiles (:118-119) and einsum with a prepended batch label
    (:123-126).  The reference's jnp.einsum runs in float32 (JAX's default
    x64=False turns the float64 relation values into float32).
    precision="fp32": float32 operands, float32 einsum (BLAS-backed, the
    reference's arithmetic); precision="fp64": float64 "truth", returned as
    float64."""
    lhs_idx = np.asarray(lhs_idx)
    if len(lhs_idx) == 0:
        shape = infer_output_tile_shape(kernel_string, lhs_values.shape[1:], rhs_values.shape[1:])
        return np.zeros((0, *shape), dtype=lhs_values.dtype)
    dt = np.float32 if precision == "fp32" else np.float64
    L = np.asarray(lhs_values, dtype=dt)[lhs_idx]
    R = np.asarray(rhs_values, dtype=dt)[np.asarray(rhs_idx)]
    return batched_einsum(add_batch_dim(kernel_string), L, R).astype(dt, copy=False)


# dtype of jnp.array(x) for a host array with JAX's default 64-bit types off
_JNP_CANON = {np.dtype(np.float64): np.dtype(np.float32), np.dtype(np.int64): np.dtype(np.int32),
              np.dtype(np.uint64): np.dtype(np.uint32)}


def jnp_einsum_dtype(lhs_dtype, rhs_dtype):
    """Result dtype of jnp.einsum(jnp.array(l), jnp.array(r)) with 64-bit
    types off (execution/sparse_dispatch.py:125): each operand canonicalised
    (float64 -> float32, int64 -> int32, uint64 -> uint32); a floating
    operand makes the result floating (float16 with float16 or integers,
    float32 otherwise); two integer or boolean operands give their promoted
    type, canonicalised again."""
    ld = _JNP_CANON.get(np.dtype(lhs_dtype), np.dtype(lhs_dtype))
    rd = _JNP_CANON.get(np.dtype(rhs_dtype), np.dtype(rhs_dtype))
    floats = [d for d in (ld, rd) if d.kind == "f"]
    if floats:
        return np.dtype(np.float16) if all(d == np.float16 for d in floats) else np.dtype(np.float32)
    res = np.promote_types(ld, rd)
    return _JNP_CANON.get(res, res)


def kernel_einsum_typed(lhs_values, rhs_values, lhs_idx, rhs_idx, kernel_string):
    """kernel_einsum (execution/sparse_dispatch.py:85-126) with the dtypes of
    its jnp.array / jnp.einsum calls (:125) kept: a floating result is formed
    in float64 and returned in jnp_einsum_dtype; an integer or boolean result
    is formed exactly in int64 from the canonicalised operands and reduced to
    the result type (truncation mod 2^bits, "nonzero" for booleans), which is
    what wrapping arithmetic in the result type gives."""
    lhs_values, rhs_values = np.asarray(lhs_values), np.asarray(rhs_values)
    res = jnp_einsum_dtype(lhs_values.dtype, rhs_values.dtype)
    lhs_idx = np.asarray(lhs_idx)
    if len(lhs_idx) == 0:
        shape = infer_output_tile_shape(kernel_string, lhs_values.shape[1:], rhs_values.shape[1:])
        return np.zeros((0, *shape), dtype=lhs_values.dtype)

    def canon(v):
        return v.astype(_JNP_CANON.get(v.dtype, v.dtype))

    L = canon(lhs_values)[lhs_idx]
    R = canon(rhs_values)[np.asarray(rhs_idx)]
    spec = add_batch_dim(kernel_string)
    if res.kind == "f":
        return np.einsum(spec, L.astype(np.float64), R.astype(np.float64)).astype(res)
    exact = np.einsum(spec, L.astype(np.int64), R.astype(np.int64))
    if res == np.bool_:
        return exact != 0
    return exact.astype(res)


def reverse_einsum_string(kernel_string: str) -> tuple:
    """autodiff/custom_vjp.py:31-62: "A,B->C" -> ("C,B->A", "A,C->B");
    ValueError without "->"."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    ins, out = kernel_string.split("->")
    terms = ins.split(",")
    return f"{out},{terms[1]}->{terms[0]}", f"{terms[0]},{out}->{terms[1]}"


def pair_einsum_vjp(lhs_values, rhs_values, lhs_idx, rhs_idx, kernel_string, g):
    """The backward of sparse_einsum_raw (autodiff/custom_vjp.py:254-275) in
    float64: zero gradients shaped like the values (:259-260), per-pair
    einsums with the reversed strings and the batch label (:266-270), summed
    into the operand tiles with np.add.at, the restatement of
    .at[indices].add (:271-272)."""
    L = np.asarray(lhs_values, dtype=np.float64)
    Rv = np.asarray(rhs_values, dtype=np.float64)
    gl = np.zeros(L.shape, np.float64)
    gr = np.zeros(Rv.shape, np.float64)
    li, ri = np.asarray(lhs_idx, dtype=np.int64), np.asarray(rhs_idx, dtype=np.int64)
    if len(li):
        sl, sr = reverse_einsum_string(kernel_string)
        G = np.asarray(g, dtype=np.float64)
        np.add.at(gl, li, np.einsum(add_batch_dim(sl), G, Rv[ri]))
        np.add.at(gr, ri, np.einsum(add_batch_dim(sr), L[li], G))
    return gl, gr


def batched_einsum(spec: str, L: np.ndarray, R: np.ndarray) -> np.ndarray:
    """np.einsum(spec, L, R), routed through np.matmul when the operands are
    in matmul layout: a common label prefix (batch), lhs = M + K,
    rhs = K + N, out = M + N.  Other specs go to np.einsum."""
    ins, c = spec.split("->")
    a, b = ins.split(",")
    p = 0
    while p < min(len(a), len(b), len(c)) and a[p] == b[p] == c[p]:
        p += 1
    a2, b2, c2 = a[p:], b[p:], c[p:]
    k = "".join(x for x in a2 if x in b2 and x not in c2)
    m = a2[:len(a2) - len(k)]
    n = b2[len(k):]
    plain = (len(set(a + b)) == len(a + b) - len(k) - p and a2 == m + k and b2 == k + n
             and c2 == m + n and not set(m) & set(b2) and not set(n) & set(a2))
    if not plain:
        return np.einsum(spec, L, R)
    bshape = L.shape[:p]
    ms, ks, ns = L.shape[p:p + len(m)], L.shape[p + len(m):], R.shape[p + len(k):]
    Mi, Ki, Ni = int(np.prod(ms)), int(np.prod(ks)), int(np.prod(ns))
    out = np.matmul(L.reshape(*bshape, Mi, Ki), R.reshape(*bshape, Ki, Ni))
    return out.reshape(*bshape, *ms, *ns)


def compute_output_coords(lhs_coords, rhs_coords, lhs_idx, rhs_idx, agg_keys, n_out=None):
    """execution/sparse_dispatch.py:174-223: out[:, d] = coords of the source
    operand (0 = lhs, 1 = rhs) at agg dim, int32; empty -> (0, n_out)."""
    n_out = len(agg_keys) if n_out is None else n_out
    if len(lhs_idx) == 0:
        return np.zeros((0, n_out), np.int32)
    out = np.zeros((len(lhs_idx), n_out), np.int32)
    for d, (src, dim) in enumerate(agg_keys):
        out[:, d] = (lhs_coords[lhs_idx, dim] if src == 0 else rhs_coords[rhs_idx, dim])
    return out


def segment_sum(values: np.ndarray, output_coords: np.ndarray) -> tuple:
    """execution/sparse_dispatch.py:129-171: group pair indices by coordinate
    tuple in pair order (:156-159), sort the distinct tuples (:161), add the
    pair tiles sequentially in pair order in the values dtype starting from
    zeros (:164-169)."""
    if len(values) == 0:
        nd = output_coords.shape[1] if output_coords.ndim > 1 else 0
        tile = values.shape[1:] if values.ndim > 1 else ()
        return np.zeros((0, nd), np.int32), np.zeros((0, *tile), dtype=values.dtype)
    groups: dict = {}
    for i in range(len(output_coords)):
        groups.setdefault(tuple(int(x) for x in output_coords[i]), []).append(i)
    keys = sorted(groups)
    agg = np.zeros((len(keys), *values.shape[1:]), dtype=values.dtype)
    for u, k in enumerate(keys):
        for i in groups[k]:
            agg[u] += values[i]
    return np.array(keys, dtype=np.int32), agg


def segment_plan(output_coords: np.ndarray) -> tuple:
    """The grouping half of segment_sum (:155-162) as explicit arrays: sorted
    distinct coordinates, the stable permutation of pairs by coordinate
    (pair order inside a segment), segment offsets and each pair's segment."""
    P = len(output_coords)
    if P == 0:
        nd = output_coords.shape[1] if output_coords.ndim > 1 else 0
        return (np.zeros((0, nd), np.int32), np.zeros(0, np.int32), np.zeros(1, np.int32),
                np.zeros(0, np.int32))
    oc = np.asarray(output_coords, dtype=np.int64)
    perm = np.lexsort(oc.T[::-1]) if oc.shape[1] else np.arange(P)
    s = oc[perm]
    new = np.ones(P, bool)
    if oc.shape[1]:
        new[1:] = np.any(s[1:] != s[:-1], axis=1)
    else:
        new[1:] = False
    seg_of_sorted = np.cumsum(new) - 1
    offsets = np.concatenate([np.nonzero(new)[0], [P]]).astype(np.int32)
    seg_ids = np.empty(P, np.int32)
    seg_ids[perm] = seg_of_sorted
    return s[new].astype(np.int32), perm.astype(np.int32), offsets, seg_ids


def execute_sparse(lhs: Rel, rhs: Rel, join_keys, kernel_string, agg_keys, output_shape=None,
                   output_tile_shape=None, precision="fp32") -> Rel:
    """execution/sparse_dispatch.py:226-297: infer the output tile shape
    (:263-266) and shape (:269-273), join (:276), per-pair einsum (:279-281),
    output coordinates (:284-287), segment sum (:290)."""
    if output_tile_shape is None:
        output_tile_shape = infer_output_tile_shape(kernel_string, lhs.tile_shape, rhs.tile_shape)
    if output_shape is None:
        output_shape = tuple(lhs.shape[d] if s == 0 else rhs.shape[d] for s, d in agg_keys)
    li, ri = coordinate_join(lhs.coords, rhs.coords, join_keys)
    tiles = kernel_einsum(lhs.values, rhs.values, li, ri, kernel_string, precision)
    oc = compute_output_coords(lhs.coords, rhs.coords, li, ri, agg_keys, len(output_tile_shape))
    coords, vals = segment_sum(tiles, oc)
    return Rel(coords, vals, tuple(output_shape), tuple(output_tile_shape))


def block_sparse_matmul_generic(lhs: Rel, rhs: Rel, block_shape=None, precision="fp32") -> Rel:
    """kernels/pallas_matmul.py:33-113: 2-D only (:55-59), inner tile dims must
    match (:68-73), join [(1,0)], empty -> float64 zeros with tile
    (m_tile, n_tile) from block_shape or the operands (:61-66, :79-86), then
    the three phases with agg [(0,0),(1,1)] (:89-106)."""
    if len(lhs.shape) != 2 or len(rhs.shape) != 2:
        raise ValueError("block_sparse_matmul requires 2D tensors")
    if block_shape is not None:
        m_t, _, n_t = block_shape
    else:
        m_t, n_t = lhs.tile_shape[0], rhs.tile_shape[1]
    if lhs.tile_shape[1] != rhs.tile_shape[0]:
        raise ValueError("Inner tile dimensions must match")
    li, ri = coordinate_join(lhs.coords, rhs.coords, [(1, 0)])
    out_shape = (lhs.shape[0], rhs.shape[1])
    if len(li) == 0:
        return Rel(np.zeros((0, 2), np.int32), np.zeros((0, m_t, n_t), np.float64), out_shape,
                   (m_t, n_t))
    tiles = kernel_einsum(lhs.values, rhs.values, li, ri, "ij,jk->ik", precision)
    oc = compute_output_coords(lhs.coords, rhs.coords, li, ri, [(0, 0), (1, 1)])
    coords, vals = segment_sum(tiles, oc)
    return Rel(coords, vals, out_shape, (m_t, n_t))


def block_sparse_matmul(lhs_coords, lhs_values, rhs_coords, rhs_values, block_shape, lhs_shape,
                        rhs_shape, precision="fp32") -> Rel:
    """kernels/pallas_matmul.py:116-158: wrap raw arrays as relations (int32
    coords, float64 values, :145-156) and call the generic matmul."""
    m, k, n = block_shape
    lhs = Rel(np.asarray(lhs_coords, np.int32), np.asarray(lhs_values, np.float64),
              tuple(lhs_shape), (m, k))
    rhs = Rel(np.asarray(rhs_coords, np.int32), np.asarray(rhs_values, np.float64),
              tuple(rhs_shape), (k, n))
    return block_sparse_matmul_generic(lhs, rhs, block_shape, precision)


def rel_l2(x: np.ndarray, ref: np.ndarray) -> float:
    """||x - ref||_2 / ||ref||_2 over all values (0 when both are zero)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = float(np.linalg.norm(ref.ravel()))
    num = float(np.linalg.norm((x - ref).ravel()))
    return num / den if den > 0 else num
