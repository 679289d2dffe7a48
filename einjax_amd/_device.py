"""Device-side phases of the sparse-einsum path, on HIP through libejhip.so.

Every function takes and returns torch tensors resident on the current
GPU; torch supplies the memory and the current stream, all arithmetic runs
in the library's kernels.  Sizes that depend on the data (pairs, segments,
tiles) come back through the library's *_count calls, one host
synchronisation each, or, in queued_segment_einsum, through coherent host
memory that the plan fills and marks with a ticket while the einsum is
already queued.
"""

from __future__ import annotations

import ctypes
import threading
from math import prod

import numpy as np
import torch

from . import _lib
from ._lib import check, i32_array, i64_array

_VALUE_DTYPES = {torch.float32: _lib.EJ_F32, torch.bfloat16: _lib.EJ_BF16}
# Tile einsums also take int32 tiles (integer arithmetic, int32 results).
_EINSUM_DTYPES = {**_VALUE_DTYPES, torch.int32: _lib.EJ_I32}
# Segment sums keep the values' dtype.
_SEGSUM_DTYPES = {**_VALUE_DTYPES, torch.float64: _lib.EJ_F64, torch.float16: _lib.EJ_F16,
                  torch.int32: _lib.EJ_I32, torch.int64: _lib.EJ_I64}


_gpu_checked = False


def require_gpu() -> torch.device:
    """The current GPU; raises when none is visible (there is no CPU path)."""
    global _gpu_checked
    if not _gpu_checked:
        if not torch.cuda.is_available():
            raise RuntimeError("the sparse-einsum path runs on a ROCm GPU and none is visible")
        _lib.load()
        _gpu_checked = True
    return torch.device("cuda", torch._C._cuda_getDevice())


def current_device_index() -> int:
    return torch._C._cuda_getDevice()


def stream_ptr() -> ctypes.c_void_p:
    """hipStream_t of torch's current stream on the current device."""
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice()))


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None and t.numel() > 0 else 0)


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def value_code(t: torch.Tensor) -> int:
    try:
        return _VALUE_DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"tile values must be float32 or bfloat16 on the device, got {t.dtype}")


def einsum_code(t: torch.Tensor) -> int:
    try:
        return _EINSUM_DTYPES[t.dtype]
    except KeyError:
        raise TypeError("tile einsum values must be float32, bfloat16 or int32 on the device, "
                        f"got {t.dtype}")


def as_coords(t: torch.Tensor, device) -> torch.Tensor:
    t = t.to(device=device, dtype=torch.int32)
    if t.dim() == 1:
        t = t.reshape(-1, 1) if t.numel() else t.reshape(0, 0)
    return t.contiguous()


def as_index(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.int64).contiguous().reshape(-1)


# ---------------------------------------------------------------------------

def coords_range(coords: torch.Tensor) -> tuple[list[int], list[int]]:
    """Per-column (min, max) of int32 coordinates [n, ncols]."""
    n, nc = coords.shape
    lo_hi = (ctypes.c_int32 * max(1, 2 * nc))()
    ws = workspace(8 * max(nc, 1), coords.device)
    check(_lib.load().ej_coords_range(ptr(coords), n, nc, lo_hi, ptr(ws), ws.numel(),
                                      stream_ptr()), "ej_coords_range")
    return [lo_hi[2 * c] for c in range(nc)], [lo_hi[2 * c + 1] for c in range(nc)]


def join(lhs_coords: torch.Tensor, rhs_coords: torch.Tensor, join_keys, radices,
         order: int = _lib.EJ_ORDER_PROBE) -> tuple[torch.Tensor, torch.Tensor]:
    """Matched (lhs_idx, rhs_idx) int64 pairs in the reference's order."""
    lib = _lib.load()
    dev = lhs_coords.device
    n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
    nk = len(join_keys)
    ld = i32_array([k[0] for k in join_keys])
    rd = i32_array([k[1] for k in join_keys])
    rad = i64_array(radices)
    nbytes = ctypes.c_size_t()
    check(lib.ej_join_workspace_size(n_l, n_r, order, ctypes.byref(nbytes)),
          "ej_join_workspace_size")
    ws = workspace(nbytes.value, dev)
    n_pairs = ctypes.c_int64()
    check(lib.ej_join_count(ptr(lhs_coords), n_l, lhs_coords.shape[1], ptr(rhs_coords), n_r,
                            rhs_coords.shape[1], nk, ld, rd, rad, order, ptr(ws), ws.numel(),
                            ctypes.byref(n_pairs), stream_ptr()), "ej_join_count")
    P = n_pairs.value
    li = torch.empty(P, dtype=torch.int64, device=dev)
    ri = torch.empty(P, dtype=torch.int64, device=dev)
    check(lib.ej_join_fill(n_l, n_r, nk, order, ptr(ws), ws.numel(), P, ptr(li), ptr(ri), P,
                           stream_ptr()), "ej_join_fill")
    return li, ri


def output_coords(lhs_coords, rhs_coords, lhs_idx, rhs_idx, agg_keys) -> torch.Tensor:
    n_out = len(agg_keys)
    P = lhs_idx.numel()
    out = torch.empty((P, n_out), dtype=torch.int32, device=lhs_coords.device)
    check(_lib.load().ej_output_coords(
        ptr(lhs_coords), lhs_coords.shape[0], lhs_coords.shape[1], ptr(rhs_coords),
        rhs_coords.shape[0], rhs_coords.shape[1], ptr(lhs_idx), ptr(rhs_idx), P, n_out, i32_array([s for s, _ in agg_keys]),
        i32_array([d for _, d in agg_keys]), ptr(out), stream_ptr()), "ej_output_coords")
    return out


def segment_plan(lhs_coords, rhs_coords, lhs_idx, rhs_idx, agg_keys, radices):
    """Groups pairs by output coordinate.

    Returns (out_coords int32 [U, n_out], seg_offsets int32 [U+1],
    perm int32 [P], seg_ids int32 [P])."""
    lib = _lib.load()
    dev = lhs_coords.device
    P = lhs_idx.numel()
    n_out = len(agg_keys)
    src = i32_array([s for s, _ in agg_keys])
    dim = i32_array([d for _, d in agg_keys])
    rad = i64_array(radices)
    nbytes = ctypes.c_size_t()
    check(lib.ej_segment_workspace_size(P, ctypes.byref(nbytes)), "ej_segment_workspace_size")
    ws = workspace(nbytes.value, dev)
    n_seg = ctypes.c_int64()
    check(lib.ej_segment_count(ptr(lhs_coords), lhs_coords.shape[0], lhs_coords.shape[1],
                               ptr(rhs_coords), rhs_coords.shape[0], rhs_coords.shape[1],
                               ptr(lhs_idx), ptr(rhs_idx), P, n_out, src, dim, rad, ptr(ws),
                               ws.numel(), ctypes.byref(n_seg), stream_ptr()),
          "ej_segment_count")
    U = n_seg.value
    out_coords = torch.empty((U, n_out), dtype=torch.int32, device=dev)
    offsets = torch.empty(U + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(P, dtype=torch.int32, device=dev)
    seg_ids = torch.empty(P, dtype=torch.int32, device=dev)
    check(lib.ej_segment_fill(P, U, n_out, rad, ptr(ws), ws.numel(), ptr(out_coords),
                              ptr(offsets), ptr(perm), ptr(seg_ids), U, stream_ptr()),
          "ej_segment_fill")
    return out_coords, offsets, perm, seg_ids


def gather_tiles(values: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """values[idx] for whole tiles (the reference's fancy-index gather)."""
    n = idx.numel()
    out = torch.empty((n, *values.shape[1:]), dtype=values.dtype, device=values.device)
    tile_bytes = values.element_size() * prod(values.shape[1:])
    if n == 0 or tile_bytes == 0:
        return out
    check(_lib.load().ej_gather_tiles(ptr(values), values.shape[0], tile_bytes, ptr(idx), n,
                                      ptr(out), stream_ptr()), "ej_gather_tiles")
    return out


def describe(kernel_string: str, lhs_tile, rhs_tile) -> _lib.EinsumDesc:
    d = _lib.EinsumDesc()
    check(_lib.load().ej_einsum_describe(kernel_string.encode(), i64_array(lhs_tile),
                                         len(lhs_tile), i64_array(rhs_tile), len(rhs_tile),
                                         ctypes.byref(d)), "ej_einsum_describe")
    return d


def _out_tile(desc: _lib.EinsumDesc) -> tuple:
    return tuple(int(desc.out_ext[i]) for i in range(desc.n_out))


def _set_out_dtype(desc, values: torch.Tensor, out_dtype) -> torch.dtype:
    """Output dtype of an einsum on `values`: out_dtype, or by default the
    operands' own dtype (float32, or bfloat16 for bfloat16 tiles), as the
    reference's jnp.einsum returns.  Written into the descriptor."""
    dt = values.dtype if out_dtype is None else out_dtype
    if values.dtype == torch.int32 or dt == torch.int32:
        if dt != values.dtype:
            raise TypeError(f"int32 tiles give int32 results, not {dt}")
        desc.out_dtype = _lib.EJ_I32
        return dt
    if dt not in _VALUE_DTYPES:
        raise TypeError(f"einsum outputs are float32 or bfloat16, got {dt}")
    desc.out_dtype = _VALUE_DTYPES[dt]
    return dt


def pair_einsum(desc, lhs_values, rhs_values, lhs_idx=None, rhs_idx=None, n_pairs=None,
                out_dtype=None):
    """[P, *out_tile]: the tile einsum of every matched pair, summed in fp32,
    in out_dtype (default: the operands' dtype); int32 tiles give int32
    results, formed with wrapping integer arithmetic."""
    code = einsum_code(lhs_values)
    if rhs_values.dtype != lhs_values.dtype:
        raise TypeError("both operands must have the same value dtype")
    P = lhs_idx.numel() if lhs_idx is not None else int(n_pairs)
    odt = _set_out_dtype(desc, lhs_values, out_dtype)
    out = torch.empty((P, *_out_tile(desc)), dtype=odt, device=lhs_values.device)
    check(_lib.load().ej_pair_einsum(ctypes.byref(desc), code, ptr(lhs_values), ptr(rhs_values),
                                     lhs_values.shape[0], rhs_values.shape[0], ptr(lhs_idx),
                                     ptr(rhs_idx), P, ptr(out), stream_ptr()), "ej_pair_einsum")
    return out


def segment_einsum(desc, lhs_values, rhs_values, lhs_idx, rhs_idx, perm, seg_offsets,
                   out_dtype=None):
    """[U, *out_tile]: fused gather + tile einsum + segment sum, summed in
    fp32 (int32 tiles: in wrapping integer arithmetic), in out_dtype
    (default: the operands' dtype)."""
    code = einsum_code(lhs_values)
    if rhs_values.dtype != lhs_values.dtype:
        raise TypeError("both operands must have the same value dtype")
    U = seg_offsets.numel() - 1
    odt = _set_out_dtype(desc, lhs_values, out_dtype)
    out = torch.empty((U, *_out_tile(desc)), dtype=odt, device=lhs_values.device)
    check(_lib.load().ej_segment_einsum(ctypes.byref(desc), code, ptr(lhs_values),
                                        ptr(rhs_values), lhs_values.shape[0], rhs_values.shape[0],
                                        ptr(lhs_idx), ptr(rhs_idx), ptr(perm), ptr(seg_offsets),
                                        U, ptr(out), stream_ptr()), "ej_segment_einsum")
    return out


class _Counts(threading.local):
    """Per-thread count buffer in coherent host memory (ej_host_alloc, kept
    for the thread's lifetime): the counts of ej_pair_plan_async (U, plan
    range flag, pairs planned, -, P, join range flag) and, in slot 6, the
    ticket of the call whose counts they are."""

    addr: int = 0
    view = None
    ticket: int = 0


_counts = _Counts()


def _next_ticket(ticket: int) -> int:
    """The ticket after `ticket`: 1 .. 2^30 - 1, cycling (the plans take
    tickets below 2^30)."""
    return ticket % ((1 << 30) - 1) + 1


def _count_buffer():
    """(host address, int64[8] view, new ticket) of this thread's count buffer."""
    if not _counts.addr:
        p = ctypes.c_void_p()
        check(_lib.load().ej_host_alloc(64, ctypes.byref(p)), "ej_host_alloc")
        _counts.addr = p.value
        _counts.view = (ctypes.c_int64 * 8).from_address(p.value)
    _counts.ticket = _next_ticket(_counts.ticket)
    # The plans publish differently packed words in slot 6 (the general plan
    # its ticket, the dense and row plans ticket, flags and counts in one
    # word), and a previous call's word could read as this call's ticket in
    # another packing; every previous publication has been waited for, so
    # clearing the slot leaves only this call's word to wait for.
    _counts.view[6] = 0
    return _counts.addr, _counts.view, _counts.ticket


def _wait_ticket(view, ticket: int) -> None:
    """Waits until the GPU has stored `ticket` in view[6] (it stores the
    counts first).  Spins briefly, then synchronizes the stream and checks
    once more, so an error that stops the stream cannot leave it spinning."""
    for _ in range(200000):
        if view[6] == ticket:
            return
    torch.cuda.current_stream().synchronize()
    if view[6] != ticket:
        raise RuntimeError("the queued plan did not report its counts")


# Grouped fused einsums (several output segments per workgroup sharing each
# lhs stage) pay only with enough workgroups to fill the GPU.  Whole steps,
# block-sparse x dense 'ij,jk->ik', grouped against one segment per
# workgroup: fp32 32^2 tiles (groups of 4) 27.1/22.5 us at 992 segments,
# 37.2/57.4 us at 4096; bf16 128^2 tiles (groups of 2) 32.0/22.4 us at 64,
# 38.2/30.1 at 768, 70.2/66.0 at 1984, 160.4/196.2 at 4096 segments.
GROUP_MIN_SEGMENTS = 2048


def drop_small_grouping(desc, n_segments: int) -> None:
    """Clears the descriptor's seg_group hint when at most n_segments
    segments are too few for grouped workgroups."""
    if n_segments < GROUP_MIN_SEGMENTS:
        desc.seg_group = 0


def _carve(sizes_bytes):
    """Offsets (bytes, 256-byte aligned) of consecutive regions of one
    buffer, and its total size in int64 elements."""
    offs, off = [], 0
    for n in sizes_bytes:
        offs.append(off)
        off += (max(int(n), 1) + 255) // 256 * 256
    return offs, off // 8


class QueuedStep:
    """ej_pair_plan_async + ej_segment_einsum_async for one combination of
    coordinate arrays, join and output keys, radices, descriptor, operand
    values and pair bound.  Everything that depends only on those is
    computed once here (workspace sizes, capacities, the argument lists);
    run_queued_step queues one call: join, segment plan and fused einsum back
    to back on the current stream, with one wait for the plan's counts.  The
    step holds the tensors' addresses, not the tensors: whoever reuses it
    checks that the same tensors are still in place."""

    def __init__(self, lhs_coords, rhs_coords, join_keys, join_radices, agg_keys, agg_radices,
                 desc, lhs_values, rhs_values, pair_bound: int, out_dtype=None):
        lib = self.lib = _lib.load()
        self.dev = lhs_coords.device
        code = value_code(lhs_values)
        if rhs_values.dtype != lhs_values.dtype:
            raise TypeError("both operands must have the same value dtype")
        n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
        nk = len(join_keys)
        self.cap_p = cap_p = max(int(pair_bound), 1)
        self.cap_u = cap_u = max(1, min(cap_p, prod(agg_radices)))
        drop_small_grouping(desc, cap_u)
        self.n_out = n_out = len(agg_keys)
        nbytes = ctypes.c_size_t()
        check(lib.ej_join_workspace_size(n_l, n_r, _lib.EJ_ORDER_PROBE, ctypes.byref(nbytes)),
              "ej_join_workspace_size")
        jws = nbytes.value
        check(lib.ej_segment_workspace_size(cap_p, ctypes.byref(nbytes)),
              "ej_segment_workspace_size")
        sws = nbytes.value
        self.odt = _set_out_dtype(desc, lhs_values, out_dtype)
        self.out_tile = _out_tile(desc)
        self.desc = desc
        # The einsum's segments per workgroup when it runs grouped (its
        # seg_group hint): the plan may also write the run order of those groups.
        gq = ctypes.c_int32(1)
        check(lib.ej_segment_einsum_group(ctypes.byref(desc), code, ctypes.byref(gq)),
              "ej_segment_einsum_group")
        self.group = group = gq.value if gq.value > 1 else 0
        n_order = 1 + (cap_u + group - 1) // group if group else 1
        (self.o_jws, self.o_sws, self.o_li, self.o_ri, self.o_off, self.o_perm,
         self.o_ord), self.ws_elems = _carve([jws, sws, 8 * cap_p, 8 * cap_p, 4 * (cap_u + 1),
                                              4 * cap_p, 4 * n_order])
        self.jws_size, self.sws_size = jws, sws
        self.order_written = ctypes.c_int32(0)
        self._arrays = arr = (i32_array([k[0] for k in join_keys]),
                              i32_array([k[1] for k in join_keys]), i64_array(join_radices),
                              i32_array([s for s, _ in agg_keys]), i32_array([d for _, d in agg_keys]),
                              i64_array(agg_radices))
        self.plan_head = (lhs_coords.data_ptr(), n_l, lhs_coords.shape[1], rhs_coords.data_ptr(),
                          n_r, rhs_coords.shape[1], nk, arr[0], arr[1], arr[2], n_out, arr[3],
                          arr[4], arr[5], cap_p)
        self.einsum_head = (ctypes.byref(desc), code, lhs_values.data_ptr(),
                            rhs_values.data_ptr(), lhs_values.shape[0], rhs_values.shape[0])


def run_queued_step(step: QueuedStep, einsum_events=None):
    """Queues one call of a prepared QueuedStep and waits for the plan's
    counts.  Returns (status, result): "ok" with result = (P, U, coords
    [cap_u, n_out], values [cap_u, *out_tile], workspace) (the first U rows
    of coords and values are the output), "bound" with result = (P,) when P
    exceeded the step's pair bound, "range" when a coordinate fell outside
    its radix (result None).  Either failure leaves nothing but ignored
    output: every kernel clips its work to the device-side counts.
    einsum_events: an optional list; when given, a (start, end) pair of
    timing events recorded around the einsum launch is appended to it."""
    lib, dev = step.lib, step.dev
    stream = stream_ptr()
    ws = torch.empty(step.ws_elems, dtype=torch.int64, device=dev)
    coords = torch.empty((step.cap_u, step.n_out), dtype=torch.int32, device=dev)
    out = torch.empty((step.cap_u, *step.out_tile), dtype=step.odt, device=dev)
    w = ws.data_ptr()
    li, ri, off, perm = w + step.o_li, w + step.o_ri, w + step.o_off, w + step.o_perm
    order = w + step.o_ord if step.group else None
    base, counts, ticket = _count_buffer()
    check(lib.ej_pair_plan_async(*step.plan_head, w + step.o_jws, step.jws_size,
                                 w + step.o_sws, step.sws_size, li, ri, coords.data_ptr(), off,
                                 perm, step.cap_u, step.group, order,
                                 ctypes.byref(step.order_written), base, ticket, stream),
          "ej_pair_plan_async")
    if einsum_events is not None:
        einsum_events.append((torch.cuda.Event(enable_timing=True),
                              torch.cuda.Event(enable_timing=True)))
        einsum_events[-1][0].record()
    check(lib.ej_segment_einsum_async(*step.einsum_head, li, ri, perm, off, step.cap_u,
                                      w + step.o_sws,
                                      order if step.order_written.value else None, step.group,
                                      out.data_ptr(), stream), "ej_segment_einsum_async")
    if einsum_events is not None:
        einsum_events[-1][1].record()
    _wait_ticket(counts, ticket)
    U, bad_plan, _, _, P, bad_join = (int(counts[i]) for i in range(6))
    if bad_join:
        return "range", None
    if P > step.cap_p:
        return "bound", (P,)
    if bad_plan:
        return "range", None
    if U > step.cap_u:  # cannot happen: U <= min(P, prod(agg_radices))
        raise RuntimeError(f"segment count {U} exceeds its bound {step.cap_u}")
    return "ok", (P, U, coords, out, ws)


def queued_segment_einsum(lhs_coords, rhs_coords, join_keys, join_radices, agg_keys,
                          agg_radices, desc, lhs_values, rhs_values, pair_bound: int,
                          out_dtype=None, einsum_events=None):
    """Join, segment plan and fused segment einsum queued back to back on the
    current stream, with the pair count bounded by pair_bound instead of
    read first (QueuedStep + run_queued_step).  The plan stores its counts in
    coherent host memory followed by this call's ticket; the host waits only
    for the ticket (the einsum is already queued behind the plan), then
    checks the counts.

    Returns (status, result).  status "ok": result = (P, coords [U, n_out],
    seg_offsets, perm, values [U, *out_tile], li, ri), views clipped to the
    counts.  "bound": P exceeded pair_bound (result[0] = P); "range": a
    coordinate fell outside its radix.  Either way the caller runs the exact
    path; every kernel clips its work to the device-side counts, so an
    exceeded bound costs a rerun, never a stray access."""
    step = QueuedStep(lhs_coords, rhs_coords, join_keys, join_radices, agg_keys, agg_radices,
                      desc, lhs_values, rhs_values, pair_bound, out_dtype)
    status, res = run_queued_step(step, einsum_events)
    if status != "ok":
        return status, res
    P, U, coords, out, ws = res
    b = ws.view(torch.uint8)
    li = b[step.o_li:step.o_li + 8 * P].view(torch.int64)
    ri = b[step.o_ri:step.o_ri + 8 * P].view(torch.int64)
    offsets = b[step.o_off:step.o_off + 4 * (U + 1)].view(torch.int32)
    perm = b[step.o_perm:step.o_perm + 4 * P].view(torch.int32)
    return "ok", (P, coords[:U], offsets, perm, out[:U], li, ri)


class _DenseCounts(threading.local):
    """Per-thread device counters of the dense plan, one buffer per (device,
    stream): zeroed once, left zero by every plan.  Its first entry is the
    segment count that the einsum queued behind the plan reads while it runs,
    so a buffer is only ever reused by work queued after that einsum on the
    same stream; a step queued on another stream gets a buffer of its own."""

    bufs: dict = {}

    def __init__(self):
        self.bufs = {}


_dense_state = _DenseCounts()


def _dense_counts(dev, stream: int) -> torch.Tensor:
    key = (dev, stream)
    buf = _dense_state.bufs.get(key)
    if buf is None:
        buf = _dense_state.bufs[key] = torch.zeros(8, dtype=torch.int64, device=dev)
    return buf


def dense_plan_applies(n_lhs: int, lhs_ncols: int, rhs_ncols: int, join_keys, agg_keys) -> bool:
    """Whether the structure of a join suits ej_dense_plan_async (the device
    then checks the data): rhs join dims 0 .. nk-1 with increasing lhs dims,
    output = a prefix of the lhs dims then the rhs dims after the join dims,
    every other lhs dim joined, 1 .. 16384 lhs tiles."""
    nk = len(join_keys)
    if nk < 1 or nk > rhs_ncols or not 1 <= n_lhs <= 16384:
        return False
    by_r = sorted((b, a) for a, b in join_keys)
    if [b for b, _ in by_r] != list(range(nk)):
        return False
    ld = [a for _, a in by_r]
    if any(x >= y for x, y in zip(ld, ld[1:])):
        return False
    nlo = 0
    while nlo < len(agg_keys) and tuple(agg_keys[nlo]) == (0, nlo):
        nlo += 1
    rest = [tuple(k) for k in agg_keys[nlo:]]
    if nlo < 1 or rest != [(1, d) for d in range(nk, rhs_ncols)]:
        return False
    return all(d in ld for d in range(nlo, lhs_ncols))


class DenseStep:
    """ej_dense_plan_async + ej_segment_einsum_async for one combination of
    coordinate arrays, join and output keys, grids, descriptor and operand
    values, with everything that depends only on those computed once
    (run_dense_step queues one call).  supported is False when the join's
    structure cannot take the dense plan (beyond its 32-bit indices).  The
    step holds the tensors' addresses, not the tensors: whoever reuses it
    checks that the same tensors are still in place."""

    def __init__(self, lhs_coords, rhs_coords, join_keys, agg_keys, lhs_grid, rhs_grid, desc,
                 lhs_values, rhs_values, out_dtype=None):
        lib = self.lib = _lib.load()
        self.dev = lhs_coords.device
        code = value_code(lhs_values)
        if rhs_values.dtype != lhs_values.dtype:
            raise TypeError("both operands must have the same value dtype")
        n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
        nk = len(join_keys)
        NK = prod(int(rhs_grid[d]) for d in range(nk, len(rhs_grid)))
        nlo = len(agg_keys) - (len(rhs_grid) - nk)
        self.cap_p = cap_p = n_l * NK
        self.supported = not (cap_p >= 1 << 30 or prod(int(g) for g in rhs_grid) >= 1 << 31)
        if not self.supported:
            return  # beyond the plan's 32-bit indices
        self.cap_u = cap_u = max(1, min(n_l, prod(int(lhs_grid[d]) for d in range(nlo))) * NK)
        drop_small_grouping(desc, cap_u)
        self.n_out = n_out = len(agg_keys)
        self.odt = _set_out_dtype(desc, lhs_values, out_dtype)
        self.out_tile = _out_tile(desc)
        self.desc = desc
        gq = ctypes.c_int32(1)
        check(lib.ej_segment_einsum_group(ctypes.byref(desc), code, ctypes.byref(gq)),
              "ej_segment_einsum_group")
        self.group = group = gq.value if gq.value > 1 else 0
        n_order = 1 + (cap_u + group - 1) // group if group else 1
        (self.o_li, self.o_ri, self.o_off, self.o_ord), self.ws_elems = _carve(
            [8 * cap_p, 8 * cap_p, 4 * (cap_u + 1), 4 * n_order])
        self.order_written = ctypes.c_int32(0)
        self._arrays = arr = (i32_array([k[0] for k in join_keys]),
                              i32_array([k[1] for k in join_keys]), i64_array(lhs_grid),
                              i64_array(rhs_grid), i32_array([a for a, _ in agg_keys]),
                              i32_array([b for _, b in agg_keys]))
        self.plan_head = (lhs_coords.data_ptr(), n_l, lhs_coords.shape[1], rhs_coords.data_ptr(),
                          n_r, rhs_coords.shape[1], nk, arr[0], arr[1], arr[2], arr[3], n_out,
                          arr[4], arr[5])
        self.einsum_head = (ctypes.byref(desc), code, lhs_values.data_ptr(),
                            rhs_values.data_ptr(), lhs_values.shape[0], rhs_values.shape[0])


def run_dense_step(step: DenseStep, einsum_events=None):
    """Queues one call of a prepared DenseStep: the one-launch dense plan and
    the fused segment einsum back to back on the current stream, then waits
    for the plan's ticket.  Returns (status, result): "ok" with result =
    (P, U, coords [cap_u, n_out], values [cap_u, *out_tile], workspace) (the
    first U rows of coords and values are the output); "miss" when the data
    does not have the dense structure (the queued einsum did no work);
    "unsupported" when the library refuses the structure."""
    lib, dev = step.lib, step.dev
    stream = stream_ptr()
    ws = torch.empty(step.ws_elems, dtype=torch.int64, device=dev)
    coords = torch.empty((step.cap_u, step.n_out), dtype=torch.int32, device=dev)
    out = torch.empty((step.cap_u, *step.out_tile), dtype=step.odt, device=dev)
    w = ws.data_ptr()
    li, ri, off = w + step.o_li, w + step.o_ri, w + step.o_off
    order = w + step.o_ord if step.group else None
    dcounts = _dense_counts(dev, stream.value).data_ptr()
    base, counts, ticket = _count_buffer()
    st = lib.ej_dense_plan_async(*step.plan_head, li, ri, step.cap_p, coords.data_ptr(), off,
                                 step.cap_u, step.group, order, ctypes.byref(step.order_written),
                                 dcounts, base, ticket, stream)
    if st == _lib.EJ_E_UNSUPPORTED:
        return "unsupported", None
    check(st, "ej_dense_plan_async")
    if einsum_events is not None:
        einsum_events.append((torch.cuda.Event(enable_timing=True),
                              torch.cuda.Event(enable_timing=True)))
        einsum_events[-1][0].record()
    check(lib.ej_segment_einsum_async(*step.einsum_head, li, ri, None, off, step.cap_u, dcounts,
                                      order if step.order_written.value else None, step.group,
                                      out.data_ptr(), stream), "ej_segment_einsum_async")
    if einsum_events is not None:
        einsum_events[-1][1].record()
    word = _wait_packed_ticket(counts, ticket)
    U, miss = word & 0xFFFFFFFF, (word >> 32) & 1
    if miss:
        return "miss", None
    return "ok", (step.cap_p, U, coords, out, ws)


# Limits of ej_row_plan_async (the library refuses beyond them).
ROW_MAX_LHS, ROW_MAX_JOIN, ROW_MAX_FREE, ROW_MAX_RUNS = 16384, 65536, 8192, 8192
_ROW_COUNT_MASK = (1 << 21) - 1


def row_plan_applies(n_lhs: int, lhs_grid, rhs_grid, join_keys, agg_keys) -> bool:
    """Whether a join suits ej_row_plan_async (the device then checks the
    data): the structure of the dense plan (dense_plan_applies) with a rhs
    that need not be full, within the plan's limits on lhs tiles, join keys,
    free indices and runs."""
    nl, nr, nk = len(lhs_grid), len(rhs_grid), len(join_keys)
    if not dense_plan_applies(min(n_lhs, ROW_MAX_LHS), nl, nr, join_keys, agg_keys):
        return False
    nlo = len(agg_keys) - (nr - nk)
    runs = min(n_lhs, prod(int(g) for g in lhs_grid[:nlo]))
    return (1 <= n_lhs <= ROW_MAX_LHS and prod(int(g) for g in rhs_grid[:nk]) <= ROW_MAX_JOIN
            and prod(int(g) for g in rhs_grid[nk:]) <= ROW_MAX_FREE and runs <= ROW_MAX_RUNS)


def _ticket20(ticket: int) -> int:
    """A count-buffer ticket folded to 1 .. 2^20 - 1 (consecutive tickets stay
    distinct), for the row plan's packed word."""
    return (ticket - 1) % ((1 << 20) - 1) + 1


class RowStep:
    """ej_row_plan_async + ej_segment_einsum_async for one combination of
    sorted coordinate arrays, join and output keys, grids, descriptor,
    operand values and pair bound, with everything that depends only on those
    computed once (run_row_step queues one call).  The step holds the
    tensors' addresses, not the tensors: whoever reuses it checks that the
    same tensors are still in place."""

    def __init__(self, lhs_coords, rhs_coords, join_keys, agg_keys, lhs_grid, rhs_grid, desc,
                 lhs_values, rhs_values, pair_bound: int, out_dtype=None):
        lib = self.lib = _lib.load()
        self.dev = lhs_coords.device
        code = value_code(lhs_values)
        if rhs_values.dtype != lhs_values.dtype:
            raise TypeError("both operands must have the same value dtype")
        n_l, n_r = lhs_coords.shape[0], rhs_coords.shape[0]
        nk = len(join_keys)
        NK = prod(int(rhs_grid[d]) for d in range(nk, len(rhs_grid)))
        nlo = len(agg_keys) - (len(rhs_grid) - nk)
        self.cap_p = cap_p = max(int(pair_bound), 1)
        runs = min(n_l, prod(int(lhs_grid[d]) for d in range(nlo)))
        self.cap_u = cap_u = max(1, min(cap_p, runs * NK))
        drop_small_grouping(desc, cap_u)
        desc.seg_group = 0  # a sparse rhs shows no runs of segments sharing lhs tiles
        self.n_out = n_out = len(agg_keys)
        self.odt = _set_out_dtype(desc, lhs_values, out_dtype)
        self.out_tile = _out_tile(desc)
        self.desc = desc
        nbytes = ctypes.c_size_t()
        check(lib.ej_row_plan_workspace_size(n_l, n_r, prod(int(rhs_grid[d]) for d in range(nk)),
                                             ctypes.byref(nbytes)), "ej_row_plan_workspace_size")
        self.rws_size = nbytes.value
        (self.o_rws, self.o_li, self.o_ri, self.o_off), self.ws_elems = _carve(
            [self.rws_size, 8 * cap_p, 8 * cap_p, 4 * (cap_u + 1)])
        self._arrays = arr = (i32_array([k[0] for k in join_keys]),
                              i32_array([k[1] for k in join_keys]), i64_array(lhs_grid),
                              i64_array(rhs_grid), i32_array([a for a, _ in agg_keys]),
                              i32_array([b for _, b in agg_keys]))
        self.plan_head = (lhs_coords.data_ptr(), n_l, lhs_coords.shape[1], rhs_coords.data_ptr(),
                          n_r, rhs_coords.shape[1], nk, arr[0], arr[1], arr[2], arr[3], n_out,
                          arr[4], arr[5])
        self.einsum_head = (ctypes.byref(desc), code, lhs_values.data_ptr(),
                            rhs_values.data_ptr(), lhs_values.shape[0], rhs_values.shape[0])


def run_row_step(step: RowStep, einsum_events=None):
    """Queues one call of a prepared RowStep: the three-launch row plan and
    the fused segment einsum back to back on the current stream, then waits
    for the plan's packed count word.  Returns (status, result): "ok" with
    result = (P, U, coords [cap_u, n_out], values [cap_u, *out_tile],
    workspace) (the first U rows of coords and values are the output);
    "bound" with result = (P,) when the pairs or segments exceeded the
    step's capacities (P below 2^21 - 1: a larger bound will do); "miss"
    when the data does not have the sorted structure or is beyond the plan's
    2^21 counts; "unsupported" when the library refuses the structure.  The
    einsum does no work after a failure."""
    lib, dev = step.lib, step.dev
    stream = stream_ptr()
    ws = torch.empty(step.ws_elems, dtype=torch.int64, device=dev)
    coords = torch.empty((step.cap_u, step.n_out), dtype=torch.int32, device=dev)
    out = torch.empty((step.cap_u, *step.out_tile), dtype=step.odt, device=dev)
    w = ws.data_ptr()
    li, ri, off = w + step.o_li, w + step.o_ri, w + step.o_off
    dcounts = _dense_counts(dev, stream.value).data_ptr()
    base, counts, ticket = _count_buffer()
    t20 = _ticket20(ticket)
    st = lib.ej_row_plan_async(*step.plan_head, li, ri, step.cap_p, coords.data_ptr(), off,
                               step.cap_u, w + step.o_rws, step.rws_size, dcounts, base, t20,
                               stream)
    if st == _lib.EJ_E_UNSUPPORTED:
        return "unsupported", None
    check(st, "ej_row_plan_async")
    if einsum_events is not None:
        einsum_events.append((torch.cuda.Event(enable_timing=True),
                              torch.cuda.Event(enable_timing=True)))
        einsum_events[-1][0].record()
    check(lib.ej_segment_einsum_async(*step.einsum_head, li, ri, None, off, step.cap_u, dcounts,
                                      None, 0, out.data_ptr(), stream), "ej_segment_einsum_async")
    if einsum_events is not None:
        einsum_events[-1][1].record()
    word = _wait_word(counts, t20, 44, "the row plan")
    flag = (word >> 42) & 3
    P, U = (word >> 21) & _ROW_COUNT_MASK, word & _ROW_COUNT_MASK
    if flag & 1:
        return "miss", None
    if flag & 2:
        if P >= _ROW_COUNT_MASK or U >= _ROW_COUNT_MASK:
            return "miss", None
        return "bound", (P,)
    return "ok", (P, U, coords, out, ws)


def dense_segment_einsum(lhs_coords, rhs_coords, join_keys, agg_keys, lhs_grid, rhs_grid, desc,
                         lhs_values, rhs_values, out_dtype=None, einsum_events=None):
    """Join, segment plan (ej_dense_plan_async: one launch, for a dense rhs
    and increasing lhs coordinates) and the fused segment einsum, queued back
    to back on the current stream (DenseStep + run_dense_step); the host
    waits only for the plan's ticket.

    Returns (status, result): "ok" with result = (P, coords [U, n_out],
    seg_offsets, None, values [U, *out_tile], li, ri); "miss" when the data
    does not have the dense structure (the queued einsum did no work);
    "unsupported" when the join's structure does not suit the dense plan."""
    step = DenseStep(lhs_coords, rhs_coords, join_keys, agg_keys, lhs_grid, rhs_grid, desc,
                     lhs_values, rhs_values, out_dtype)
    if not step.supported:
        return "unsupported", None
    status, res = run_dense_step(step, einsum_events)
    if status != "ok":
        return status, res
    P, U, coords, out, ws = res
    b = ws.view(torch.uint8)
    li = b[step.o_li:step.o_li + 8 * P].view(torch.int64)
    ri = b[step.o_ri:step.o_ri + 8 * P].view(torch.int64)
    offsets = b[step.o_off:step.o_off + 4 * (U + 1)].view(torch.int32)
    return "ok", (P, coords[:U], offsets, None, out[:U], li, ri)


def _wait_word(view, ticket: int, shift: int, who: str) -> int:
    """Waits until the GPU has stored a word whose bits from `shift` up hold
    `ticket` in view[6] and returns it (as _wait_ticket, bounded by a stream
    sync)."""
    mask = (1 << 64) - 1  # the int64 view's word, read unsigned
    for _ in range(200000):
        w = view[6] & mask
        if w >> shift == ticket:
            return w
    torch.cuda.current_stream().synchronize()
    w = view[6] & mask
    if w >> shift != ticket:
        raise RuntimeError(f"{who} did not report its counts")
    return w


def _wait_packed_ticket(view, ticket: int) -> int:
    """Waits until the GPU has stored the word ticket << 33 | flag << 32 | U
    in view[6] and returns it (as _wait_ticket, bounded by a stream sync)."""
    return _wait_word(view, ticket, 33, "the dense plan")


def segment_sum(pair_values: torch.Tensor, perm, seg_offsets) -> torch.Tensor:
    """[U, *tile] in the pair values' dtype: per-segment sums in plan order,
    formed in fp32 for float32 / bfloat16 values (a bf16 sum rounded once),
    in the values' own arithmetic for float64, float16 (each addition rounded
    to float16, as numpy adds float16) and int32 / int64 (wrapping)."""
    try:
        code = _SEGSUM_DTYPES[pair_values.dtype]
    except KeyError:
        raise TypeError(f"segment sums take float64, float32, float16, bfloat16, int32 or int64 "
                        f"values on the device, got {pair_values.dtype}")
    U = seg_offsets.numel() - 1
    tile = tuple(pair_values.shape[1:])
    out = torch.empty((U, *tile), dtype=pair_values.dtype, device=pair_values.device)
    check(_lib.load().ej_segment_sum(ptr(pair_values), code, max(prod(tile), 1), ptr(perm),
                                     ptr(seg_offsets), U, ptr(out), stream_ptr()),
          "ej_segment_sum")
    return out


def bucket_dense(dense: torch.Tensor, tile_shape) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense tensor -> (coords int32 [T, nd], values [T, *tile_shape]).

    The tiles keep the input dtype: float64, float32 or bfloat16."""
    lib = _lib.load()
    code = _elem_code(dense)
    out_dtype = dense.dtype
    dense = dense.contiguous()
    nd = dense.dim()
    shape = i64_array(dense.shape)
    tile = i64_array(tile_shape)
    nbytes = ctypes.c_size_t()
    check(lib.ej_bucket_workspace_size(nd, shape, tile, ctypes.byref(nbytes)),
          "ej_bucket_workspace_size")
    ws = workspace(nbytes.value, dense.device)
    n_tiles = ctypes.c_int64()
    check(lib.ej_bucket_dense_count(ptr(dense), code, nd, shape, tile, ptr(ws), ws.numel(),
                                    ctypes.byref(n_tiles), stream_ptr()), "ej_bucket_dense_count")
    T = n_tiles.value
    coords = torch.empty((T, nd), dtype=torch.int32, device=dense.device)
    values = torch.empty((T, *tile_shape), dtype=out_dtype, device=dense.device)
    check(lib.ej_bucket_dense_fill(ptr(dense), code, nd, shape, tile, ptr(ws), ws.numel(), T,
                                   ptr(coords), ptr(values), T, stream_ptr()),
          "ej_bucket_dense_fill")
    return coords, values


def relation_to_dense(coords, values, shape, tile_shape) -> torch.Tensor:
    code = _elem_code(values)
    dense = torch.empty(tuple(shape), dtype=values.dtype, device=values.device)
    check(_lib.load().ej_relation_to_dense(ptr(coords), ptr(values), coords.shape[0], code,
                                           len(shape), i64_array(shape), i64_array(tile_shape),
                                           ptr(dense), stream_ptr()), "ej_relation_to_dense")
    return dense


def _elem_code(t: torch.Tensor) -> int:
    """Element dtype of a dense tensor or COO values: float64, float32 or bfloat16."""
    if t.dtype == torch.float64:
        return _lib.EJ_F64
    return value_code(t)


def _coo_count(dense: torch.Tensor):
    lib = _lib.load()
    code = _elem_code(dense)
    nd = dense.dim()
    shape = i64_array(dense.shape)
    nbytes = ctypes.c_size_t()
    check(lib.ej_extract_coo_workspace_size(nd, shape, code, ctypes.byref(nbytes)),
          "ej_extract_coo_workspace_size")
    ws = workspace(nbytes.value, dense.device)
    nnz = ctypes.c_int64()
    check(lib.ej_extract_coo_count(ptr(dense), code, nd, shape, ptr(ws), ws.numel(),
                                   ctypes.byref(nnz), stream_ptr()), "ej_extract_coo_count")
    return nnz.value, ws, code, shape


def count_nonzero(dense: torch.Tensor) -> int:
    """Number of elements != 0 (NaN included) of a dense tensor."""
    dense = dense.contiguous()
    if dense.dim() == 0:
        dense = dense.reshape(1)
    return _coo_count(dense)[0]


def extract_coo(dense: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense tensor -> (indices int32 [nnz, nd], values float64 [nnz]): the
    elements != 0 in row-major order."""
    lib = _lib.load()
    dense = dense.contiguous()
    nd = dense.dim()
    n, ws, code, shape = _coo_count(dense)
    idx = torch.empty((n, nd), dtype=torch.int32, device=dense.device)
    vals = torch.empty((n,), dtype=torch.float64, device=dense.device)
    check(lib.ej_extract_coo_fill(ptr(dense), code, nd, shape, ptr(ws), ws.numel(), n, ptr(idx),
                                  ptr(vals), n, stream_ptr()), "ej_extract_coo_fill")
    return idx, vals


def bucket_coo(indices: torch.Tensor, values: torch.Tensor, shape,
               tile_shape) -> tuple[torch.Tensor, torch.Tensor]:
    """COO entries -> (coords int32 [T, nd], values [T, *tile_shape]).

    The tiles have the values' dtype (float64, float32 or bfloat16).
    Entries equal to zero are dropped; an element listed twice keeps its last
    nonzero entry."""
    lib = _lib.load()
    nd = len(shape)
    indices = indices.to(dtype=torch.int32).reshape(-1, nd).contiguous()
    values = values.contiguous().reshape(-1)
    code = _elem_code(values)
    out_dtype = values.dtype
    n = values.numel()
    sh, ts = i64_array(shape), i64_array(tile_shape)
    nbytes = ctypes.c_size_t()
    check(lib.ej_bucket_coo_workspace_size(n, code, nd, sh, ts, ctypes.byref(nbytes)),
          "ej_bucket_coo_workspace_size")
    ws = workspace(nbytes.value, values.device)
    n_tiles = ctypes.c_int64()
    check(lib.ej_bucket_coo_count(ptr(indices), ptr(values), code, n, nd, sh, ts, ptr(ws),
                                  ws.numel(), ctypes.byref(n_tiles), stream_ptr()),
          "ej_bucket_coo_count")
    T = n_tiles.value
    coords = torch.empty((T, nd), dtype=torch.int32, device=values.device)
    tiles = torch.empty((T, *tile_shape), dtype=out_dtype, device=values.device)
    check(lib.ej_bucket_coo_fill(ptr(indices), ptr(values), code, n, nd, sh, ts, ptr(ws),
                                 ws.numel(), T, ptr(coords), ptr(tiles), T, stream_ptr()),
          "ej_bucket_coo_fill")
    return coords, tiles


def scheme_stats(tile_shapes, shape, dense: torch.Tensor | None = None,
                 indices: torch.Tensor | None = None, values: torch.Tensor | None = None,
                 bitmap_cap: int = 0):
    """(num_tuples [S], value_count [S][nd]) as Python ints for each tile
    shape, over the nonzero elements of a dense tensor or of COO entries."""
    lib = _lib.load()
    nd = len(shape)
    S = len(tile_shapes)
    if S == 0:
        return [], []
    # numpy buffers: with 1,728 tile shapes, Python lists and ctypes arrays
    # cost milliseconds per call on the host
    ts = np.asarray(tile_shapes, dtype=np.int64)
    if ts.shape != (S, nd):
        raise ValueError(f"tile shapes must all have {nd} dims, got an array of shape {ts.shape}")
    flat = np.ascontiguousarray(ts).reshape(-1)
    sh = i64_array(shape)
    nt = np.zeros(S, dtype=np.int64)
    vc = np.zeros(S * nd, dtype=np.int64)
    p_flat, p_nt, p_vc = (a.ctypes.data_as(_lib._P_i64) for a in (flat, nt, vc))
    nbytes = ctypes.c_size_t()
    if dense is not None:
        dense = dense.contiguous()
        check(lib.ej_scheme_stats_workspace_size(nd, sh, S, p_flat, -1, 0, ctypes.byref(nbytes)),
              "ej_scheme_stats_workspace_size")
        ws = workspace(nbytes.value, dense.device)
        check(lib.ej_scheme_stats_dense(ptr(dense), _elem_code(dense), nd, sh, S, p_flat, ptr(ws),
                                        ws.numel(), p_nt, p_vc, stream_ptr()),
              "ej_scheme_stats_dense")
    else:
        indices = indices.to(dtype=torch.int32).reshape(-1, nd).contiguous()
        values = values.contiguous().reshape(-1)
        n = values.numel()
        check(lib.ej_scheme_stats_workspace_size(nd, sh, S, p_flat, n, bitmap_cap,
                                                 ctypes.byref(nbytes)),
              "ej_scheme_stats_workspace_size")
        ws = workspace(nbytes.value, values.device)
        check(lib.ej_scheme_stats_coo(ptr(indices), ptr(values), _elem_code(values), n, nd, sh,
                                      S, p_flat, bitmap_cap, ptr(ws), ws.numel(), p_nt, p_vc,
                                      stream_ptr()), "ej_scheme_stats_coo")
    return nt.tolist(), list(map(tuple, vc.reshape(S, nd).tolist()))


def index_plan(idx: torch.Tensor, n_targets: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(perm int32 [n], offsets int32 [n_targets + 1]): positions grouped by
    target, ascending inside a target; out-of-range targets come last."""
    lib = _lib.load()
    idx = idx.to(dtype=torch.int64).contiguous().reshape(-1)
    n = idx.numel()
    nbytes = ctypes.c_size_t()
    check(lib.ej_index_plan_workspace_size(n, ctypes.byref(nbytes)),
          "ej_index_plan_workspace_size")
    ws = workspace(nbytes.value, idx.device)
    perm = torch.empty((n,), dtype=torch.int32, device=idx.device)
    offsets = torch.empty((n_targets + 1,), dtype=torch.int32, device=idx.device)
    check(lib.ej_index_plan(ptr(idx), n, n_targets, ptr(perm), ptr(offsets), ptr(ws), ws.numel(),
                            stream_ptr()), "ej_index_plan")
    return perm, offsets


def pair_einsum_vjp(kernel_string: str, lhs_values: torch.Tensor, rhs_values: torch.Tensor,
                    lhs_idx: torch.Tensor, rhs_idx: torch.Tensor, grad_out: torch.Tensor,
                    need_lhs: bool = True, need_rhs: bool = True):
    """(grad_lhs, grad_rhs) with the operands' tile shapes (None when not
    requested): the gradients of the per-pair tile einsum for the cotangent
    grad_out [P, *out_tile].  bfloat16 operands with a bfloat16 cotangent give
    bfloat16 gradients (bf16 einsums, fp32 sums); otherwise the cotangent is
    taken in float32 and the gradients are float32."""
    lib = _lib.load()
    code = value_code(lhs_values)
    if rhs_values.dtype != lhs_values.dtype:
        raise TypeError("both operands must have the same value dtype")
    lt, rt = tuple(lhs_values.shape[1:]), tuple(rhs_values.shape[1:])
    nl, nr = lhs_values.shape[0], rhs_values.shape[0]
    li = lhs_idx.to(dtype=torch.int64).contiguous().reshape(-1)
    ri = rhs_idx.to(dtype=torch.int64).contiguous().reshape(-1)
    P = li.numel()
    gdt = torch.bfloat16 if (lhs_values.dtype == torch.bfloat16 and
                             grad_out.dtype == torch.bfloat16) else torch.float32
    gcode = _VALUE_DTYPES[gdt]
    g = grad_out.to(dtype=gdt).contiguous()
    dev = lhs_values.device
    gl = torch.empty((nl, *lt), dtype=gdt, device=dev) if need_lhs else None
    gr = torch.empty((nr, *rt), dtype=gdt, device=dev) if need_rhs else None
    nbytes = ctypes.c_size_t()
    check(lib.ej_pair_einsum_vjp_workspace_size(P, nl, nr, max(prod(lt), 1), max(prod(rt), 1),
                                                code, gcode, ctypes.byref(nbytes)),
          "ej_pair_einsum_vjp_workspace_size")
    ws = workspace(nbytes.value, dev)
    check(lib.ej_pair_einsum_vjp(kernel_string.encode(), i64_array(lt), len(lt), i64_array(rt),
                                 len(rt), code, ptr(lhs_values.contiguous()), nl,
                                 ptr(rhs_values.contiguous()), nr, ptr(li), ptr(ri), P, gcode,
                                 ptr(g), ptr(gl), ptr(gr), ptr(ws), ws.numel(), stream_ptr()),
          "ej_pair_einsum_vjp")
    return gl, gr
