"""The allocation-free queued pair plan (ej_pair_plan_async_noalloc) against
ej_pair_plan_async with caller workspaces, through the C ABI.

Two calls in a row on each path, the second with a smaller input, so that
the second call runs on scratch holding the first call's leftovers: pairs,
output coordinates, segment offsets, permutation, run order and counts
must be bit-identical to the workspace entry point's.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import generators as G

from einjax_amd import _device, _lib

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


def _args(w: dict, cap_p: int, group: int):
    """Device buffers and the argument lists of both entry points for
    workload w's coordinates: (head, tail, buffers)."""
    L, Rr = w["lhs"], w["rhs"]
    lc = torch.from_numpy(L.coords).cuda()
    rc = torch.from_numpy(Rr.coords).cuda()
    keys, agg = w["join_keys"], w["agg_keys"]
    grid = lambda r, d: r.shape[d] // r.tile_shape[d]
    jrad = [max(grid(L, a), grid(Rr, b)) for a, b in keys]
    arad = [grid(L if s == 0 else Rr, d) for s, d in agg]
    cap_u = min(cap_p, int(np.prod(arad)))
    n_out = len(agg)
    dev = lc.device
    fill = lambda shape, dt: torch.full(shape, -7, dtype=dt, device=dev)
    li, ri = fill((cap_p,), torch.int64), fill((cap_p,), torch.int64)
    coords, offsets = fill((cap_u, n_out), torch.int32), fill((cap_u + 1,), torch.int32)
    perm = fill((cap_p,), torch.int32)
    order = fill((1 + (cap_u + group - 1) // group,), torch.int32) if group else None
    written = ctypes.c_int32(-1)
    counts = torch.full((8,), -7, dtype=torch.int64).pin_memory()
    ld = _lib.i32_array([k[0] for k in keys])
    rd = _lib.i32_array([k[1] for k in keys])
    src = _lib.i32_array([s for s, _ in agg])
    dim = _lib.i32_array([d for _, d in agg])
    head = (_device.ptr(lc), lc.shape[0], lc.shape[1], _device.ptr(rc), rc.shape[0], rc.shape[1],
            len(keys), ld, rd, _lib.i64_array(jrad), n_out, src, dim, _lib.i64_array(arad), cap_p)
    tail = (_device.ptr(li), _device.ptr(ri), _device.ptr(coords), _device.ptr(offsets),
            _device.ptr(perm), cap_u, group, _device.ptr(order), ctypes.byref(written),
            ctypes.c_void_p(counts.data_ptr()), 0, _device.stream_ptr())
    bufs = dict(lc=lc, rc=rc, li=li, ri=ri, coords=coords, offsets=offsets, perm=perm,
                order=order, written=written, counts=counts, cap_u=cap_u, dev=dev)
    return head, tail, bufs


def _plan(noalloc: bool, w: dict, cap_p: int, group: int):
    """Runs one entry point on workload w's coordinates; returns the results
    clipped to the counts, as host arrays."""
    lib = _lib.load()
    head, tail, b = _args(w, cap_p, group)
    lc, rc, dev = b["lc"], b["rc"], b["dev"]
    li, ri, coords, offsets, perm = b["li"], b["ri"], b["coords"], b["offsets"], b["perm"]
    order, written, counts, cap_u = b["order"], b["written"], b["counts"], b["cap_u"]
    if noalloc:
        _lib.check(lib.ej_pair_plan_async_noalloc(*head, *tail), "ej_pair_plan_async_noalloc")
    else:
        nb = ctypes.c_size_t()
        _lib.check(lib.ej_join_workspace_size(lc.shape[0], rc.shape[0], _lib.EJ_ORDER_PROBE,
                                              ctypes.byref(nb)), "ej_join_workspace_size")
        jws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        _lib.check(lib.ej_segment_workspace_size(cap_p, ctypes.byref(nb)),
                   "ej_segment_workspace_size")
        sws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        _lib.check(lib.ej_pair_plan_async(*head, _device.ptr(jws), jws.numel(), _device.ptr(sws),
                                          sws.numel(), *tail), "ej_pair_plan_async")
    torch.cuda.synchronize()
    c = counts.tolist()
    U, P = c[0], c[4]
    assert c[1] == 0 and c[5] == 0 and P <= cap_p and U <= cap_u
    out = dict(counts=c[:6], li=li[:P].cpu().numpy(), ri=ri[:P].cpu().numpy(),
               perm=perm[:P].cpu().numpy(), coords=coords[:U].cpu().numpy(),
               offsets=offsets[:U + 1].cpu().numpy(), written=written.value)
    if written.value:
        out["order"] = order[:1 + (U + group - 1) // group].cpu().numpy()
    return out


def _same(a: dict, b: dict):
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(np.asarray(a[k]), np.asarray(b[k]), err_msg=k)


@pytest.mark.parametrize("seq", ["blocksparse", "zipf"])
def test_noalloc_plan_matches_workspace_plan(gpu, seq):
    """The one-pass plan with a run order (128^2-tile block-sparse x dense,
    4096 output tiles, then 256) and the general sort plan (Zipf sparse x
    sparse, 18-bit output keys, 54,516 pairs, then a 4096^2 instance)."""
    if seq == "blocksparse":
        calls = [(G.workload_blocksparse_16k(values=False), 2),
                 (G.workload_blocksparse_16k(seed=1, m=4096, n=1024, values=False), 2)]
    else:
        calls = [(G.workload_sparse_sparse_zipf(values=False), 0),
                 (G.workload_sparse_sparse_zipf(seed=2, n=4096, values=False), 0)]
    for w, group in calls:
        note("noalloc plan", w["name"], "group", group)
        P = _plan(False, w, 1 << 17, group)["counts"][4]
        for cap in (P, P + 1000):
            got = _plan(True, w, cap, group)
            ref = _plan(False, w, cap, group)
            _same(got, ref)
            assert ref["counts"][0] == len(ref["coords"]) > 0 and ref["counts"][4] == P
            assert ref["written"] == (1 if group else 0)


def test_noalloc_plan_rejects_oversize(gpu):
    """A plan that needs more than the 64 MiB scratch is refused before any
    work is queued, with a message naming the limit."""
    note("noalloc oversize")
    w = G.workload_blocksparse_1k(values=False)
    with pytest.raises(_lib.CapacityError, match="static scratch"):
        _plan(True, w, 2_000_000, 0)  # ~80 MB of segment workspace


def test_noalloc_plan_allocates_no_device_memory(gpu):
    """The property the entry point exists for: after a warm call, a call
    leaves the driver's free device memory unchanged (every buffer it gets is
    the caller's or the static scratch)."""
    note("noalloc plan: device memory before and after a call")
    lib = _lib.load()
    w = G.workload_sparse_sparse_zipf(seed=2, n=4096, values=False)
    head, tail, bufs = _args(w, 1 << 16, 0)
    for _ in range(2):  # warm: code objects, scratch and runtime pools are in place
        _lib.check(lib.ej_pair_plan_async_noalloc(*head, *tail), "ej_pair_plan_async_noalloc")
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        _lib.check(lib.ej_pair_plan_async_noalloc(*head, *tail), "ej_pair_plan_async_noalloc")
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0
    assert bufs["counts"][4].item() > 0
