"""The tensor-relational sparse einsum on the GPU (reference:
execution/sparse_dispatch.py).

Phases, each a HIP kernel family in libejhip.so:
  1. coordinate join     -> matched (lhs_idx, rhs_idx), reference pair order
  2. segment plan        -> pairs grouped by output coordinate (sorted)
  3. tile einsum         -> fused with the gather and the segment sum
                            (default), or per pair + a separate segment sum
                            (``fused=False``, the reference's phase split)

Function names, arguments, results and errors follow the reference.
Arguments may be host NumPy arrays (results come back as NumPy, as in the
reference) or GPU torch tensors (results stay on the GPU).
"""

from __future__ import annotations

import threading
import weakref

import numpy as np

from .. import _device, _lib
from ..tensor.sparse import SparseTensorRelation, _is_torch

__all__ = [
    "coordinate_join", "kernel_einsum", "segment_sum", "execute_sparse",
    "execute_sharded_sparse", "_add_batch_dim", "_infer_output_tile_shape",
    "_compute_output_coords", "_partition_matched_pairs",
]


# ---------------------------------------------------------------------------
# Residency helpers.

def _on_host(*xs) -> bool:
    """True when any array argument is host-resident (NumPy / CPU tensor)."""
    for x in xs:
        if isinstance(x, SparseTensorRelation):
            if not x.is_device:
                return True
        elif x is not None and not (_is_torch(x) and x.is_cuda):
            return True
    return False


def _dev(x, dtype=None):
    import torch

    dev = _device.require_gpu()
    if _is_torch(x):
        t = x
    else:
        t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(device=dev, dtype=dtype or t.dtype).contiguous()


def _dev_values(v):
    """Floating tile values on the GPU as float32, or bfloat16 when already
    bfloat16: float64 and float16 become float32, as the reference's
    jnp.array turns float64 relation values into float32 before its einsum
    (sparse_dispatch.py:125).  Integer and boolean values take
    _einsum_operands / _segsum_operand, which keep integer arithmetic."""
    import torch

    dt = v.dtype if _is_torch(v) else torch.from_numpy(np.zeros(0, dtype=v.dtype)).dtype
    if not dt.is_floating_point:
        raise TypeError(f"tile values must be floating point, got {dt}: the GPU path "
                        "computes in float32 / bfloat16")
    t = _dev(v)
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.to(torch.float32)
    return t


# ---------------------------------------------------------------------------
# Value dtypes.  The reference hands host tile values to jnp.array with
# 64-bit types off (float64 -> float32, int64 -> int32, uint64 -> uint32,
# sparse_dispatch.py:125) and jnp.einsum promotes the two operands: with a
# floating operand the result is floating (bfloat16 when every floating
# operand is bfloat16, else float32; float16 stays float16), two integer
# (or boolean) operands give their promoted integer type, computed with
# wrapping integer arithmetic.  segment_sum keeps the values' own numpy
# dtype (:164-169).  Integer einsums run on the library's int32 kernel: a
# result of a narrower integer type is the int32 result truncated, which
# equals the narrower wrapping arithmetic; a boolean result is "nonzero",
# which equals the OR of ANDs of a boolean contraction.

_CANON = {np.dtype(np.float64): np.dtype(np.float32), np.dtype(np.int64): np.dtype(np.int32),
          np.dtype(np.uint64): np.dtype(np.uint32)}


_TORCH_NP: dict = {}


def _value_np_dtype(v):
    """numpy dtype of an array's elements, or None for bfloat16 tensors."""
    if _is_torch(v):
        dt = _TORCH_NP.get(v.dtype, 0)
        if dt == 0:
            import torch

            dt = None if v.dtype == torch.bfloat16 else torch.empty(0, dtype=v.dtype).numpy().dtype
            _TORCH_NP[v.dtype] = dt
        return dt
    return np.asarray(v).dtype


def _kind(dt) -> str:
    if dt is None or dt.kind == "f":
        return "f"
    if dt.kind in "iub":
        return "i"
    raise TypeError(f"tile values of dtype {dt} are not supported (floating, integer or "
                    "boolean values are)")


def _einsum_types(lhs_values, rhs_values):
    """(compute, result) of the tile einsum on these values: compute is the
    torch dtype both operands take on the device (float32, bfloat16 or
    int32); result is the reference's result dtype (a torch dtype for
    floating results, a numpy dtype for integer / boolean ones)."""
    import torch

    ld, rd = _value_np_dtype(lhs_values), _value_np_dtype(rhs_values)
    kl, kr = _kind(ld), _kind(rd)
    if "f" in (kl, kr):
        floats = [d for d, k in ((ld, kl), (rd, kr)) if k == "f"]
        if all(d is None for d in floats):
            return torch.bfloat16, torch.bfloat16
        if all(d is not None and d == np.float16 for d in floats):
            return torch.float32, torch.float16
        return torch.float32, torch.float32
    res = np.promote_types(_CANON.get(ld, ld), _CANON.get(rd, rd))
    return torch.int32, _CANON.get(res, res)


def _int32_bits(v):
    """Integer / boolean values as int32 on the device: the jnp.array
    canonical value (64-bit types truncated to 32 bits), uint32 by its bits."""
    import torch

    if _is_torch(v):
        t = v
        if t.dtype in (torch.int64,):
            t = t.to(torch.int32)
        elif t.dtype == getattr(torch, "uint64", None):
            t = t.view(torch.int64).to(torch.int32)
        elif t.dtype == getattr(torch, "uint32", None):
            t = t.view(torch.int32)
        return _dev(t.to(torch.int32))
    a = np.asarray(v)
    a = a.astype(_CANON.get(a.dtype, a.dtype), copy=False)
    a = a.view(np.int32) if a.dtype == np.uint32 else a.astype(np.int32)
    return _dev(a)


def _einsum_operands(lhs_values, rhs_values):
    """(a, b, result): both operands on the device in the compute dtype of
    _einsum_types, and the result dtype."""
    import torch

    compute, result = _einsum_types(lhs_values, rhs_values)
    if compute == torch.int32:
        return _int32_bits(lhs_values), _int32_bits(rhs_values), result

    def flt(v):
        dt = _value_np_dtype(v)
        if dt is not None and dt.kind in "iub":
            # jnp.array's integer canonicalisation first, then the promotion
            # converts the integer's value
            if _is_torch(v):
                t = v.to(torch.int32) if v.dtype == torch.int64 else v
                return _dev(t).to(compute)
            a = np.asarray(v)
            return _dev(a.astype(_CANON.get(a.dtype, a.dtype)).astype(np.float32)).to(compute)
        return _dev_values(v).to(compute)

    return flt(lhs_values), flt(rhs_values), result


def _to_result(t, result):
    """An einsum result computed in float32 / bfloat16 / int32 in the
    reference's result dtype (on the device; uint32 as a torch uint32 view
    where torch has the type)."""
    import torch

    if isinstance(result, torch.dtype):
        return t if t.dtype == result else t.to(result)
    if result == np.int32:
        return t
    if result == np.bool_:
        return t != 0
    if result == np.uint32:
        u = getattr(torch, "uint32", None)
        return t.view(u) if u is not None else t
    return t.to(torch.from_numpy(np.zeros(0, dtype=result)).dtype)


def _host_result(t, result):
    """_to_result for host callers: a numpy array of the result dtype."""
    import torch

    if isinstance(result, torch.dtype):
        return _host(_to_result(t, result))
    a = t.cpu().numpy()
    if result == np.uint32:
        return a.view(np.uint32)
    return a.astype(result)


def _dev_coords(c, ndim):
    import torch

    t = _dev(c, torch.int32)
    if t.numel() == 0:
        return t.reshape(0, ndim)
    return t.reshape(t.shape[0], -1)


def _host(t):
    import torch

    if not _is_torch(t):
        return t
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.cpu().numpy()


def _grid(rel: SparseTensorRelation, d: int) -> int:
    t = rel.tile_shape[d] if d < len(rel.tile_shape) else 1
    s = rel.shape[d] if d < len(rel.shape) else 1
    return max(1, -(-s // max(t, 1)))


def _host_col_max(coords, d) -> int:
    if _is_torch(coords) or coords.shape[0] == 0:
        return 0
    return int(np.max(coords[:, d])) + 1


def _retry_radices(fn, make_radices, cols):
    """Runs fn(radices) with radices from grid metadata; if a coordinate
    falls outside them (the library's EJ_E_RANGE status), sizes the radices
    from the data and runs again."""
    try:
        return fn(make_radices(None))
    except _lib.RangeError:
        pass
    maxima = []
    for coords, d in cols:
        lo, hi = _device.coords_range(coords)
        if coords.shape[0] and lo[d] < 0:
            raise _NegativeCoords()
        maxima.append(hi[d] + 1 if coords.shape[0] else 1)
    return fn(make_radices(maxima))


class _NegativeCoords(Exception):
    """A joined or output coordinate column holds negative values.  The
    kernels pack coordinates >= 0; the public functions catch this and run
    again on coordinates shifted column by column (_shift_columns)."""


def _column_shifts(lc, rc, keys, out_cols):
    """Per-column shifts (<= 0) that make the coordinates the kernels pack
    non-negative: columns linked by a join key share one shift (the minimum
    over them), so equal keys stay equal and every order stays as it was.
    keys: [(lhs_dim, rhs_dim)]; out_cols: [(0 | 1, dim)] also packed.
    Returns (lhs shifts, rhs shifts)."""
    lo = [_device.coords_range(c)[0] if c.shape[0] else [0] * c.shape[1] for c in (lc, rc)]
    parent = {}

    def find(x):
        while parent.setdefault(x, x) != x:
            x = parent[x]
        return x

    for a, b in keys:
        parent[find((0, a))] = find((1, b))
    low = {}
    for side, cols in ((0, range(lc.shape[1])), (1, range(rc.shape[1]))):
        for c in cols:
            r = find((side, c))
            low[r] = min(low.get(r, 0), lo[side][c])
    shifts = ([0] * lc.shape[1], [0] * rc.shape[1])
    used = {find((0, a)) for a, _ in keys} | {find((s, d)) for s, d in out_cols}
    for side, n in ((0, lc.shape[1]), (1, rc.shape[1])):
        for c in range(n):
            r = find((side, c))
            if r in used:
                shifts[side][c] = low[r]
    return shifts


def _shift_columns(coords, shifts):
    """coords - shifts, column by column (int32 on the device)."""
    import torch

    if not any(shifts) or coords.shape[0] == 0:
        return coords
    _, hi = _device.coords_range(coords)
    if any(h - s >= 2 ** 31 for h, s in zip(hi, shifts)):
        raise ValueError("coordinate range exceeds 2^31")
    return coords - torch.tensor(shifts, dtype=torch.int32, device=coords.device)


# ---------------------------------------------------------------------------
# Phase 1: join.

def _join_radices(lhs: SparseTensorRelation, rhs: SparseTensorRelation, keys, maxima):
    """Key radices from grid metadata (and, if given, the data's column maxima)."""
    out = []
    for i, (a, b) in enumerate(keys):
        r = max(_grid(lhs, a), _grid(rhs, b), _host_col_max(lhs.coords, a),
                _host_col_max(rhs.coords, b))
        if maxima is not None:
            r = max(r, maxima[2 * i], maxima[2 * i + 1])
        out.append(r)
    return out


def _join_dev(lhs: SparseTensorRelation, rhs: SparseTensorRelation, join_keys, lc, rc,
              order=_lib.EJ_ORDER_PROBE):
    keys = [tuple(k) for k in join_keys]
    cols = [c for a, b in keys for c in ((lc, a), (rc, b))]
    return _retry_radices(lambda r: _device.join(lc, rc, keys, r, order),
                          lambda m: _join_radices(lhs, rhs, keys, m), cols)


def _segment_run(rhs: SparseTensorRelation, join_keys, agg_keys) -> int:
    """Length of the runs of consecutive output segments that contract the
    same lhs tiles in the same order, or 0 when the relations do not show
    one.  With the last output dimension taken from the rhs, the earlier ones
    from the lhs, and every rhs tile present (a dense rhs whose only other
    dimensions are join dimensions), the segments of one lhs-derived output
    prefix are consecutive, one per rhs grid step along that dimension, and
    each pairs the same lhs tiles with a different rhs tile.  The einsum
    kernels use it to read each lhs tile once for several output tiles; they
    check it on the data, so a wrong value costs speed only."""
    if not agg_keys or agg_keys[-1][0] != 1 or any(s != 0 for s, _ in agg_keys[:-1]):
        return 0
    d = agg_keys[-1][1]
    rdims = {b for _, b in join_keys}
    if d in rdims or len(rdims) + 1 != rhs.ndim:
        return 0
    full = 1
    for x in range(rhs.ndim):
        full *= _grid(rhs, x)
    if rhs.num_tuples != full:
        return 0
    return _grid(rhs, d)


# Pair counts of recent joins: a bound for the next execute_sparse on the
# same relations, which can then queue its whole step without waiting for
# the count (a wrong bound is detected and costs one rerun, never a wrong
# result).  -1: the queued path found a coordinate outside the metadata
# radices; do not retry it.  A hint belongs to the pair of coordinate arrays
# the caller passed (host arrays or device tensors, never the per-call
# device copies of host arrays): it is keyed by their ids and holds weak
# references to them, so a hint whose arrays were freed, or whose id now
# names another array, is never used.
_pair_hints: dict = {}
_PAIR_HINTS_MAX = 256
_pair_hints_lock = threading.Lock()


def _hint_key(lhs: SparseTensorRelation, rhs: SparseTensorRelation, rest: tuple):
    return (id(lhs.coords), id(rhs.coords), *rest)


def _hint_get(key, lhs: SparseTensorRelation, rhs: SparseTensorRelation):
    with _pair_hints_lock:
        ent = _pair_hints.get(key)
    if ent is None:
        return None
    wl, wr, bound = ent
    if wl() is not lhs.coords or wr() is not rhs.coords:
        with _pair_hints_lock:
            if _pair_hints.get(key) is ent:
                del _pair_hints[key]
        return None
    return bound


def _hint_set(key, lhs: SparseTensorRelation, rhs: SparseTensorRelation, bound: int):
    try:
        ent = (weakref.ref(lhs.coords), weakref.ref(rhs.coords), int(bound))
    except TypeError:  # coordinates that cannot be weakly referenced get no hint
        return
    with _pair_hints_lock:
        if key not in _pair_hints and len(_pair_hints) >= _PAIR_HINTS_MAX:
            _pair_hints.pop(next(iter(_pair_hints)))
        _pair_hints[key] = ent


def _dense_step(lhs, rhs, keys, agg, lc, rc, operands, out_dtype, events):
    """The whole step on the dense-rhs plan (one plan launch, then the fused
    einsum) when the join's structure suits it and the rhs holds every tile
    of its grid; None otherwise.  A device-side miss (coordinates that break
    the dense structure) is remembered for these coordinate arrays, so later
    calls go straight to the general plan."""
    nl, nr = lc.shape[1], rc.shape[1]
    if nl != lhs.ndim or nr != rhs.ndim:
        return None
    rgrid = [_grid(rhs, d) for d in range(nr)]
    n_full = 1
    for g in rgrid:
        n_full *= g
    if rc.shape[0] != n_full or not _device.dense_plan_applies(lc.shape[0], nl, nr, keys, agg):
        return None
    key = _hint_key(lhs, rhs, ("dense", tuple(lc.shape), tuple(rc.shape), tuple(keys),
                                tuple(agg)))
    if _hint_get(key, lhs, rhs) == -1:
        return None
    lgrid = [_grid(lhs, d) for d in range(nl)]
    desc, a, b = operands()
    step = _device.DenseStep(lc, rc, keys, agg, lgrid, rgrid, desc, a, b, out_dtype)
    status = "unsupported"
    if step.supported:
        status, res = _device.run_dense_step(step, events)
        if status == "ok":
            return res, step
    _hint_set(key, lhs, rhs, -1)
    return None


def _row_step(lhs, rhs, keys, agg, lc, rc, operands, out_dtype, bound, pair_key, events):
    """The whole step on the sorted row plan (three plan launches, then the
    fused einsum) when the join's structure suits it: (result, step,
    row hint key), or None.  A pair bound that proves too small is raised to
    the count and the step queued once more; a device-side miss (data not
    sorted, or beyond the plan's counts) is remembered for these coordinate
    arrays, so later calls go straight to the general plan."""
    nl, nr = lc.shape[1], rc.shape[1]
    if nl != lhs.ndim or nr != rhs.ndim:
        return None
    lgrid = [_grid(lhs, d) for d in range(nl)]
    rgrid = [_grid(rhs, d) for d in range(nr)]
    if not _device.row_plan_applies(lc.shape[0], lgrid, rgrid, keys, agg):
        return None
    rkey = _hint_key(lhs, rhs, ("row", tuple(lc.shape), tuple(rc.shape), tuple(keys),
                                tuple(agg)))
    if _hint_get(rkey, lhs, rhs) == -1:
        return None
    for _ in range(2):
        desc, a, b = operands()
        step = _device.RowStep(lc, rc, keys, agg, lgrid, rgrid, desc, a, b, bound, out_dtype)
        status, res = _device.run_row_step(step, events)
        if status == "ok":
            _hint_set(pair_key, lhs, rhs, res[0])
            return res, step, rkey
        if status != "bound":
            break
        bound = res[0]
        _hint_set(pair_key, lhs, rhs, bound)
    _hint_set(rkey, lhs, rhs, -1)
    return None


# ---------------------------------------------------------------------------
# Repeated calls.  A queued step on device relations keeps its prepared plan
# and einsum (a DenseStep or QueuedStep: argument lists, capacities, output
# dtype) keyed by the call's arguments, so that calling execute_sparse again
# on the same relations only allocates the outputs, queues the join, plan and
# einsum and waits for the plan's counts.  Nothing computed on the GPU is
# reused: every call joins, plans and multiplies on the data as it is then.
# An entry is used only while the relations are the same objects holding the
# same tensors (identity, address, shape, dtype) and the same metadata.

class _StepEntry:
    __slots__ = ("lref", "rref", "sig", "kind", "step", "hint_key", "fin")


_steps: dict = {}
_STEPS_MAX = 64
_steps_lock = threading.Lock()


def _rel_sig(rel):
    c, v = rel.coords, rel.values
    return (id(c), id(v), c.data_ptr(), v.data_ptr(), c.shape, v.shape, c.dtype, v.dtype,
            rel.shape, rel.tile_shape)


def _step_key(lhs, rhs, kernel_string, join_keys, agg_keys, output_shape, output_tile_shape,
              out_dtype):
    return (id(lhs), id(rhs), kernel_string, tuple(map(tuple, join_keys)),
            tuple(map(tuple, agg_keys)), output_shape if output_shape is None else
            tuple(output_shape), output_tile_shape if output_tile_shape is None else
            tuple(output_tile_shape), out_dtype)


def _run_cached_step(key, lhs, rhs, output_shape, output_tile_shape, events):
    """The call through its prepared step, or None when there is no valid
    entry (the caller then takes the full path)."""
    ent = _steps.get(key)
    if ent is None or ent.lref() is not lhs or ent.rref() is not rhs:
        return None
    if not (_is_torch(lhs.values) and _is_torch(rhs.values) and _is_torch(lhs.coords)
            and _is_torch(rhs.coords)):
        return None
    if ent.sig != (_rel_sig(lhs), _rel_sig(rhs), _device.current_device_index()):
        with _steps_lock:
            _steps.pop(key, None)
        return None
    if ent.kind == "dense":
        status, res = _device.run_dense_step(ent.step, events)
    elif ent.kind == "row":
        status, res = _device.run_row_step(ent.step, events)
    else:
        status, res = _device.run_queued_step(ent.step, events)
    if status != "ok":
        # the data changed under the same tensors: remember what the full
        # path needs (as it would) and let it answer
        with _steps_lock:
            _steps.pop(key, None)
        hk = ent.hint_key
        if ent.kind == "dense":
            _hint_set(hk, lhs, rhs, -1)
        elif ent.kind == "row":
            pair_key, row_key = hk
            if status == "bound":
                _hint_set(pair_key, lhs, rhs, res[0])
            else:
                _hint_set(row_key, lhs, rhs, -1)
        else:
            _hint_set(hk, lhs, rhs, res[0] if status == "bound" else -1)
        return None
    P, U, coords, vals, _ = res
    return P, U, coords, vals, ent


def _remember_step(key, lhs, rhs, kind, step, hint_key, fin):
    """Keeps a prepared step for the next call on the same relations when
    the step reads the relations' own tensors (no per-call copy or cast)."""
    if not (_is_torch(lhs.values) and _is_torch(rhs.values) and _is_torch(lhs.coords)
            and _is_torch(rhs.coords)):
        return
    if (step.plan_head[0], step.plan_head[3], step.einsum_head[2], step.einsum_head[3]) != (
            lhs.coords.data_ptr(), rhs.coords.data_ptr(), lhs.values.data_ptr(),
            rhs.values.data_ptr()):
        return
    try:
        lref, rref = weakref.ref(lhs), weakref.ref(rhs)
    except TypeError:
        return
    ent = _StepEntry()
    ent.lref, ent.rref = lref, rref
    ent.sig = (_rel_sig(lhs), _rel_sig(rhs), _device.current_device_index())
    ent.kind, ent.step, ent.hint_key, ent.fin = kind, step, hint_key, fin
    with _steps_lock:
        if key not in _steps and len(_steps) >= _STEPS_MAX:
            _steps.pop(next(iter(_steps)))
        _steps[key] = ent


def coordinate_join(lhs: SparseTensorRelation, rhs: SparseTensorRelation, join_keys):
    """Matched tile pairs on join_keys = [(lhs_dim, rhs_dim), ...]
    (reference: sparse_dispatch.py:29-82).

    Pair order is the reference hash join's: rhs index ascending, then lhs
    index ascending; no keys gives the lhs-major cross product.  Returns int64
    (lhs_idx, rhs_idx)."""
    host = _on_host(lhs, rhs)
    lc = _dev_coords(lhs.coords, lhs.ndim)
    rc = _dev_coords(rhs.coords, rhs.ndim)
    try:
        li, ri = _join_dev(lhs, rhs, join_keys, lc, rc)
    except _NegativeCoords:
        keys = [tuple(k) for k in join_keys]
        sl, sr = _column_shifts(lc, rc, keys, [])
        lc, rc = _shift_columns(lc, sl), _shift_columns(rc, sr)
        li, ri = _join_dev(SparseTensorRelation(lc, lhs.values, lhs.shape, lhs.tile_shape),
                           SparseTensorRelation(rc, rhs.values, rhs.shape, rhs.tile_shape),
                           keys, lc, rc)
    return (_host(li), _host(ri)) if host else (li, ri)


# ---------------------------------------------------------------------------
# Phase 2: tile einsum.

def _add_batch_dim(kernel_string: str, batch_label: str = "z") -> str:
    """"ij,jk->ik" -> "zij,zjk->zik" (reference: sparse_dispatch.py:481-503)."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    inputs_str, output_str = kernel_string.split("->")
    return ",".join(batch_label + t for t in inputs_str.split(",")) + "->" + batch_label + output_str


def _infer_output_tile_shape(kernel_string: str, lhs_tile_shape, rhs_tile_shape) -> tuple:
    """Output tile shape from label sizes, rhs sizes overriding lhs
    (reference: sparse_dispatch.py:506-545); KeyError for a label absent
    from both inputs."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    inputs_str, output_str = kernel_string.split("->")
    terms = inputs_str.split(",")
    sizes = {}
    if len(terms) >= 1:
        for d, lab in enumerate(terms[0]):
            if d < len(lhs_tile_shape):
                sizes[lab] = lhs_tile_shape[d]
    if len(terms) >= 2:
        for d, lab in enumerate(terms[1]):
            if d < len(rhs_tile_shape):
                sizes[lab] = rhs_tile_shape[d]
    return tuple(sizes[lab] for lab in output_str)


def kernel_einsum(lhs_values, rhs_values, lhs_indices, rhs_indices, kernel_string: str):
    """einsum(kernel_string) of every matched tile pair, [P, *out_tile] of the
    dtype the reference's jnp.einsum returns (sparse_dispatch.py:85-126):
    float32 (float64 and float32 values, or a float with an integer),
    bfloat16 for bfloat16 tiles (summed in fp32 and rounded once), float16
    for float16 tiles (summed in fp32), or for integer / boolean tiles their
    promoted integer type (int64 counted as int32, as jnp.array makes it),
    computed with wrapping integer arithmetic.  No pairs gives zeros of the
    lhs values' dtype."""
    host = _on_host(lhs_values, rhs_values, lhs_indices, rhs_indices)
    n = int(lhs_indices.shape[0]) if hasattr(lhs_indices, "shape") else len(lhs_indices)
    lt, rt = tuple(lhs_values.shape[1:]), tuple(rhs_values.shape[1:])
    if n == 0:
        out_tile = _infer_output_tile_shape(kernel_string, lt, rt)
        if host:
            return np.zeros((0, *out_tile), dtype=_host(lhs_values[:0]).dtype)
        import torch

        return torch.zeros((0, *out_tile), dtype=lhs_values.dtype, device=lhs_values.device)
    _add_batch_dim(kernel_string)  # same ValueError as the reference for a missing "->"
    desc = _device.describe(kernel_string, lt, rt)
    a, b, result = _einsum_operands(lhs_values, rhs_values)
    li = _dev(np.asarray(lhs_indices) if not _is_torch(lhs_indices) else lhs_indices)
    ri = _dev(np.asarray(rhs_indices) if not _is_torch(rhs_indices) else rhs_indices)
    import torch

    out = _device.pair_einsum(desc, a, b, li.to(torch.int64), ri.to(torch.int64))
    return _host_result(out, result) if host else _to_result(out, result)


# ---------------------------------------------------------------------------
# Phase 3: aggregation.

def _compute_output_coords(lhs, rhs, lhs_indices, rhs_indices, join_keys, agg_keys,
                           output_shape, output_tile_shape):
    """Per-pair output tile coordinate, int32 [P, len(output_tile_shape)]
    (reference: sparse_dispatch.py:174-223)."""
    import torch

    host = _on_host(lhs, rhs, lhs_indices, rhs_indices)
    n_out = len(output_tile_shape)
    P = int(lhs_indices.shape[0]) if hasattr(lhs_indices, "shape") else len(lhs_indices)
    if P == 0:
        z = np.zeros((0, n_out), np.int32)
        return z if host else torch.zeros((0, n_out), dtype=torch.int32,
                                          device=_device.require_gpu())
    lc = _dev_coords(lhs.coords, lhs.ndim)
    rc = _dev_coords(rhs.coords, rhs.ndim)
    li = _dev(lhs_indices, torch.int64)
    ri = _dev(rhs_indices, torch.int64)
    oc = _device.output_coords(lc, rc, li, ri, [tuple(k) for k in agg_keys][:n_out])
    if oc.shape[1] < n_out:
        oc = torch.cat([oc, oc.new_zeros((P, n_out - oc.shape[1]))], dim=1)
    return _host(oc) if host else oc


def _plan_from_coords(oc):
    """Segment plan of bare output coordinates (int32 [P, nd] on the GPU)."""
    import torch

    P, nd = oc.shape
    idx = torch.arange(P, dtype=torch.int64, device=oc.device)
    agg = [(0, d) for d in range(nd)]
    if nd == 0:
        return _device.segment_plan(oc, oc, idx, idx, agg, [])
    # No grid metadata: size the radices from the data directly.  Negative
    # coordinates are planned shifted by their column's minimum (the order of
    # the unique coordinates does not change) and shifted back.
    lo, hi = _device.coords_range(oc)
    shift = [min(0, x) for x in lo]
    if any(h - s >= 2 ** 31 for h, s in zip(hi, shift)):
        raise ValueError("coordinate range exceeds 2^31")
    if any(shift):
        oc = _shift_columns(oc, shift)
    coords, offsets, perm, seg_ids = _device.segment_plan(
        oc, oc, idx, idx, agg, [h - s + 1 for h, s in zip(hi, shift)])
    if any(shift):
        coords = coords + torch.tensor(shift, dtype=torch.int32, device=coords.device)
    return coords, offsets, perm, seg_ids


def _segsum_operand(values):
    """(values on the device in a dtype the library sums, result converter):
    the library sums float64, float32, float16, bfloat16, int32 and int64
    values in their own arithmetic; other integer types are summed as int32 /
    int64 (unsigned ones by their bits) and truncated back, which equals
    their own wrapping arithmetic; booleans are summed as int32 and read as
    "nonzero", which equals numpy's boolean +=, a logical OR."""
    import torch

    if _is_torch(values):
        t = _dev(values)
        dt = t.dtype
        if dt in (torch.float64, torch.float32, torch.float16, torch.bfloat16, torch.int32,
                  torch.int64):
            return t, lambda r: r
        if dt == torch.bool:
            return t.to(torch.int32), lambda r: r != 0
        for u, w in ((getattr(torch, "uint32", None), torch.int32),
                     (getattr(torch, "uint64", None), torch.int64)):
            if u is not None and dt == u:
                return t.view(w), lambda r, u=u: r.view(u)
        if not dt.is_floating_point and not dt.is_complex:
            return t.to(torch.int32), lambda r, dt=dt: r.to(dt)
        raise TypeError(f"segment_sum does not take values of dtype {dt}")
    a = np.ascontiguousarray(values)
    dt = a.dtype
    if dt in (np.float64, np.float32, np.float16, np.int32, np.int64):
        return _dev(a), lambda r: r
    if dt in (np.uint32, np.uint64):
        w = np.int32 if dt == np.uint32 else np.int64
        return _dev(a.view(w)), lambda r, dt=dt: r.cpu().numpy().view(dt)
    if dt == np.bool_:
        return _dev(a.astype(np.int32)), lambda r: r != 0
    if dt.kind in "iu":
        return _dev(a.astype(np.int32)), lambda r, dt=dt: r.cpu().numpy().astype(dt)
    raise TypeError(f"segment_sum does not take values of dtype {dt}")


def segment_sum(values, output_coords):
    """Sums the pair tiles of equal output coordinate (reference:
    sparse_dispatch.py:129-171).  Returns (unique_coords int32 [U, nd] in
    ascending lexicographic order, aggregated [U, *tile] in the values' dtype,
    as the reference keeps it, :165); tiles are added in pair order, as the
    reference does: float32 and bfloat16 values in fp32 (a bfloat16 sum
    rounded once), float64 and float16 in their own arithmetic, integers with
    wrapping, booleans as a logical OR.  Output coordinates may be negative."""
    import torch

    host = _on_host(values, output_coords)
    if (values.shape[0] if hasattr(values, "shape") else len(values)) == 0:
        nd = output_coords.shape[1] if output_coords.ndim > 1 else 0
        tile = tuple(values.shape[1:]) if values.ndim > 1 else ()
        if host:
            return np.zeros((0, nd), np.int32), np.zeros((0, *tile), dtype=_host(values[:0]).dtype)
        return (torch.zeros((0, nd), dtype=torch.int32, device=values.device),
                torch.zeros((0, *tile), dtype=values.dtype, device=values.device))
    oc = _dev_coords(output_coords, output_coords.shape[1] if output_coords.ndim > 1 else 0)
    vals, back = _segsum_operand(values)
    coords, offsets, perm, _ = _plan_from_coords(oc)
    agg = back(_device.segment_sum(vals, perm, offsets))
    if host:
        return _host(coords), agg if isinstance(agg, np.ndarray) else _host(agg)
    return coords, agg


# ---------------------------------------------------------------------------
# End to end.

def _empty_result(lhs, n_out, out_tile, output_shape, host, out_dtype=None):
    import torch

    if host:
        dt = _host(lhs.values[:0]).dtype
        return SparseTensorRelation(np.zeros((0, n_out), np.int32),
                                    np.zeros((0, *out_tile), dtype=dt), output_shape, out_tile)
    dev = _device.require_gpu()
    dt = out_dtype or (lhs.values.dtype if _is_torch(lhs.values) else torch.float32)
    return SparseTensorRelation(torch.zeros((0, n_out), dtype=torch.int32, device=dev),
                                torch.zeros((0, *out_tile), dtype=dt, device=dev),
                                output_shape, out_tile)


def execute_sparse(lhs: SparseTensorRelation, rhs: SparseTensorRelation, join_keys,
                   kernel_string: str, agg_keys, output_shape=None, output_tile_shape=None, *,
                   fused: bool = True, out_dtype=None,
                   _einsum_events=None) -> SparseTensorRelation:
    try:
        return _execute_sparse(lhs, rhs, join_keys, kernel_string, agg_keys, output_shape,
                               output_tile_shape, fused=fused, out_dtype=out_dtype,
                               _einsum_events=_einsum_events)
    except _NegativeCoords:
        pass
    # Negative joined or output coordinates: run on columns shifted to be
    # non-negative (joined columns by one shift, so the pairs and their order
    # are the same) and shift the output coordinates back.
    host = _on_host(lhs, rhs)
    keys = [tuple(k) for k in join_keys]
    agg = [tuple(k) for k in agg_keys]
    lc = _dev_coords(lhs.coords, lhs.ndim)
    rc = _dev_coords(rhs.coords, rhs.ndim)
    sl, sr = _column_shifts(lc, rc, keys, agg)
    out = _execute_sparse(
        SparseTensorRelation(_shift_columns(lc, sl), lhs.values, lhs.shape, lhs.tile_shape),
        SparseTensorRelation(_shift_columns(rc, sr), rhs.values, rhs.shape, rhs.tile_shape),
        keys, kernel_string, agg, output_shape, output_tile_shape, fused=fused,
        out_dtype=out_dtype)
    back = [(sl if s == 0 else sr)[d] for s, d in agg][:out.coords.shape[1]]
    back += [0] * (out.coords.shape[1] - len(back))
    if any(back) and out.coords.shape[0]:
        if _is_torch(out.coords):
            import torch

            coords = out.coords + torch.tensor(back, dtype=torch.int32, device=out.coords.device)
        else:
            coords = (out.coords + np.asarray(back, dtype=np.int32)).astype(np.int32)
        out = SparseTensorRelation(coords, out.values, out.shape, out.tile_shape)
    return out.to_host() if host and out.is_device else out


def _execute_sparse(lhs: SparseTensorRelation, rhs: SparseTensorRelation, join_keys,
                    kernel_string: str, agg_keys, output_shape=None, output_tile_shape=None, *,
                    fused: bool = True, out_dtype=None,
                    _einsum_events=None) -> SparseTensorRelation:
    """Sparse tensor-relational einsum (reference: sparse_dispatch.py:226-297).

    join_keys: [(lhs_dim, rhs_dim)] contracted tile dims; kernel_string: the
    per-tile einsum; agg_keys: [(0 | 1, dim)] sources of the output tile
    coordinates.  Output tile shape and shape are inferred as the reference
    does when omitted.  ``fused=True`` (default) runs the gather, the tile
    einsum and the segment sum as one kernel writing every output tile once;
    ``fused=False`` runs the reference's phase split (per-pair results, then
    the segment sum in pair order).  Returns coords int32 [U, nd] sorted and
    values [U, *output_tile_shape] summed in fp32, of dtype ``out_dtype``: by
    default the operands' dtype, as in the reference (float32, or bfloat16
    for bfloat16 tiles, rounded once from the fp32 sum); ``torch.float32``
    keeps fp32 results for bfloat16 tiles.  ``_einsum_events`` (measurement
    only): a list that collects timing events recorded around the fused
    einsum of a queued call.  Integer or boolean tiles (and a float with an
    integer) follow the reference's jnp promotion (kernel_einsum) and run on
    the library's integer kernel; joined and output coordinates may be
    negative."""
    step_key = None
    if fused:
        step_key = _step_key(lhs, rhs, kernel_string, join_keys, agg_keys, output_shape,
                             output_tile_shape, out_dtype)
        hit = _run_cached_step(step_key, lhs, rhs, output_shape, output_tile_shape,
                               _einsum_events)
        if hit is not None:
            P, U, coords, vals, ent = hit
            ots, osh = ent.step.result_tile, ent.step.result_shape
            if P == 0:
                return _empty_result(lhs, len(ots), ots, osh, False, out_dtype)
            vals = vals[:U]
            if ent.fin is not None:
                vals = _to_result(vals, ent.fin)
            return SparseTensorRelation._from_parts(coords[:U], vals, osh, ots)
    if output_tile_shape is None:
        output_tile_shape = _infer_output_tile_shape(kernel_string, lhs.tile_shape,
                                                     rhs.tile_shape)
    if output_shape is None:
        output_shape = tuple(lhs.shape[d] if s == 0 else rhs.shape[d] for s, d in agg_keys)
    output_tile_shape = tuple(output_tile_shape)
    output_shape = tuple(output_shape)
    _add_batch_dim(kernel_string)
    host = _on_host(lhs, rhs)
    agg = [tuple(k) for k in agg_keys]

    lc = _dev_coords(lhs.coords, lhs.ndim)
    rc = _dev_coords(rhs.coords, rhs.ndim)
    n_out = len(output_tile_shape)

    import torch

    compute, result = _einsum_types(lhs.values, rhs.values)
    integer = compute == torch.int32
    if integer and out_dtype is not None:
        raise TypeError("out_dtype applies to floating tiles; integer tiles give the "
                        "reference's integer result dtype")
    if out_dtype is None and compute != result:
        fin = result  # computed in float32 / int32, returned in the reference's dtype
    else:
        fin = None

    def operands():
        desc = _device.describe(kernel_string, lhs.tile_shape, rhs.tile_shape)
        desc.seg_group = _segment_run(rhs, [tuple(k) for k in join_keys], agg)
        a, b, _ = _einsum_operands(lhs.values, rhs.values)
        return desc, a, b

    def radices(maxima):
        out = []
        for d, (s, dim) in enumerate(agg):
            rel = lhs if s == 0 else rhs
            r = max(_grid(rel, dim), _host_col_max(rel.coords, dim))
            if maxima is not None:
                r = max(r, maxima[d])
            out.append(r)
        return out

    keys = [tuple(k) for k in join_keys]
    hint_key = None
    bound = None
    queued = None
    if fused and keys and lc.shape[0] and rc.shape[0] and not integer:
        done = _dense_step(lhs, rhs, keys, agg, lc, rc, operands, out_dtype, _einsum_events)
        if done is not None:
            queued, step = done
            dkey = _hint_key(lhs, rhs, ("dense", tuple(lc.shape), tuple(rc.shape), tuple(keys),
                                         tuple(agg)))
            kind = "dense"
    if queued is None and fused and keys and lc.shape[0] and rc.shape[0] and not integer:
        j_rad = _join_radices(lhs, rhs, keys, None)
        hint_key = _hint_key(lhs, rhs, (tuple(lc.shape), tuple(rc.shape), tuple(keys),
                                        tuple(j_rad), tuple(agg)))
        bound = _hint_get(hint_key, lhs, rhs)
        if bound is not None and bound > 0:
            done = _row_step(lhs, rhs, keys, agg, lc, rc, operands, out_dtype, bound, hint_key,
                             _einsum_events)
            if done is not None:
                queued, step, rkey = done
                kind, dkey = "row", (hint_key, rkey)
            else:
                bound = _hint_get(hint_key, lhs, rhs)
        if queued is None and bound is not None and bound > 0:
            desc, a, b = operands()
            step = _device.QueuedStep(lc, rc, keys, j_rad, agg, radices(None), desc, a, b,
                                      bound, out_dtype)
            status, res = _device.run_queued_step(step, _einsum_events)
            if status == "ok":
                queued, kind, dkey = res, "queued", hint_key
                _hint_set(hint_key, lhs, rhs, res[0])
            else:
                bound = res[0] if status == "bound" else -1
                _hint_set(hint_key, lhs, rhs, bound)
    if queued is not None:
        P, U, coords, vals, _ = queued
        step.result_tile, step.result_shape = output_tile_shape, output_shape
        if (step_key is not None and not host and tuple(step.out_tile) == output_tile_shape
                and step.n_out == n_out):
            _remember_step(step_key, lhs, rhs, kind, step, dkey, fin)
        if P == 0:
            return _empty_result(lhs, n_out, output_tile_shape, output_shape, host, out_dtype)
        coords, vals = coords[:U], vals[:U]
    else:
        li, ri = _join_dev(lhs, rhs, join_keys, lc, rc)
        if hint_key is not None and (bound is None or bound >= 0):
            _hint_set(hint_key, lhs, rhs, li.numel())
        if li.numel() == 0:
            return _empty_result(lhs, n_out, output_tile_shape, output_shape, host, out_dtype)
        cols = [((lc if s == 0 else rc), dim) for s, dim in agg]
        coords, offsets, perm, _ = _retry_radices(
            lambda r: _device.segment_plan(lc, rc, li, ri, agg, r), radices, cols)
        desc, a, b = operands()
        if fused:
            _device.drop_small_grouping(desc, offsets.numel() - 1)
            vals = _device.segment_einsum(desc, a, b, li, ri, perm, offsets, out_dtype)
        else:
            pair_vals = _device.pair_einsum(desc, a, b, li, ri, out_dtype=out_dtype)
            vals = _device.segment_sum(pair_vals, perm, offsets)
    if coords.shape[1] != n_out:
        import torch

        coords = coords[:, :n_out] if coords.shape[1] > n_out else torch.cat(
            [coords, coords.new_zeros((coords.shape[0], n_out - coords.shape[1]))], dim=1)
    if tuple(vals.shape[1:]) != output_tile_shape and vals[0].numel() == int(
            np.prod(output_tile_shape)):
        vals = vals.reshape((vals.shape[0], *output_tile_shape))
    if fin is not None:
        if host:
            out = SparseTensorRelation(_host(coords), _host_result(vals, fin), output_shape,
                                       output_tile_shape)
            return out
        vals = _to_result(vals, fin)
    out = SparseTensorRelation(coords, vals, output_shape, output_tile_shape)
    return out.to_host() if host else out


def _partition_matched_pairs(num_matches: int, num_devices: int) -> list:
    """Contiguous, near-equal pair ranges per device, remainder to the first
    devices (reference: sparse_dispatch.py:300-327)."""
    if num_matches == 0:
        return [(0, 0)] * num_devices
    base, rem = divmod(num_matches, num_devices)
    parts, off = [], 0
    for d in range(num_devices):
        size = base + (1 if d < rem else 0)
        parts.append((off, off + size))
        off += size
    return parts


def execute_sharded_sparse(lhs, rhs, join_keys, kernel_string, agg_keys, output_shape=None,
                           output_tile_shape=None, mesh=None, num_devices=None):
    """Single-GPU form of the reference's multi-device entry
    (sparse_dispatch.py:330-478): without a mesh, or with one device, it is
    execute_sparse, exactly as in the reference (:377-393).  More devices are
    outside this library (one process drives one GPU)."""
    if num_devices is None:
        num_devices = 1 if mesh is None else len(getattr(mesh, "devices", [None]).flat)
    if mesh is None or num_devices <= 1:
        return execute_sparse(lhs, rhs, join_keys, kernel_string, agg_keys, output_shape,
                              output_tile_shape)
    raise NotImplementedError("multi-device sparse execution is not part of this library: "
                              "run one process per GPU, each on its share of the segments")
