"""The three-launch plan for a join of two sorted sparse relations
(ej_row_plan_async).

The plan's pairs, grouped by segment, must equal the oracle's join and
segment plan (reference: execution/sparse_dispatch.py:29-82, :129-171) pair
for pair, in the reference's accumulation order; execute_sparse through it
must give results bitwise identical to the general plan's; data that breaks
the sorted structure is detected on the device and answered by the general
plan, and capacities that are too small are reported with the counts.
"""

import ctypes

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R

import einjax_amd as ej
from einjax_amd import SparseTensorRelation, _device, _lib
from einjax_amd.execution import sparse_dispatch as sd

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


def grid(r: R.Rel):
    return [s // t for s, t in zip(r.shape, r.tile_shape)]


def dev_rel(r: R.Rel, dtype="fp32"):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    vals = torch.from_numpy(np.ascontiguousarray(r.values, dtype=np.float32)).cuda().to(tdt)
    return SparseTensorRelation(torch.from_numpy(np.ascontiguousarray(r.coords)).cuda(), vals,
                                r.shape, r.tile_shape)


def sparse_rel(rng, grid_shape, tile, density, drop_rows=()):
    """Tiles of a grid kept with probability `density` (at least one), in
    lexicographic order; rows (first coordinate) in drop_rows left empty."""
    keep = rng.random(grid_shape) < density
    for r in drop_rows:
        keep[r] = False
    if not keep.any():
        keep.flat[0] = True
    coords = np.ascontiguousarray(np.argwhere(keep), dtype=np.int32)
    vals = rng.standard_normal((len(coords), *tile)).astype(np.float32)
    return R.Rel(coords, vals, tuple(g * t for g, t in zip(grid_shape, tile)), tuple(tile))


def rel_from_mask(rng, keep):
    """1x1 tiles at the mask's true entries (at least one), lexicographic."""
    if not keep.any():
        keep.flat[0] = True
    coords = np.ascontiguousarray(np.argwhere(keep), dtype=np.int32)
    vals = rng.standard_normal((len(coords), *(1,) * keep.ndim)).astype(np.float32)
    return R.Rel(coords, vals, keep.shape, (1,) * keep.ndim)


def workloads():
    rng = np.random.default_rng(11)
    yield "zipf_small", G.workload_sparse_sparse_zipf(n=4096, tile=64, density=0.05)
    # empty rhs rows, lhs tiles that meet them, 1-tile runs
    L = sparse_rel(rng, (40, 30), (4, 4), 0.15)
    Rr = sparse_rel(rng, (30, 50), (4, 4), 0.1, drop_rows=(0, 3, 4, 17, 29))
    yield "gaps", dict(lhs=L, rhs=Rr, join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)],
                       kernel_string="ij,jk->ik", dtype="fp32")
    # batched: join on the batch and the contraction dim, output (b, i, k)
    L = sparse_rel(rng, (3, 12, 10), (1, 4, 4), 0.3)
    Rr = sparse_rel(rng, (3, 10, 14), (1, 4, 4), 0.25)
    yield "batched", dict(lhs=L, rhs=Rr, join_keys=[(0, 0), (2, 1)],
                          agg_keys=[(0, 0), (0, 1), (1, 2)], kernel_string="bij,bjk->bik",
                          dtype="fp32")
    # two join keys, a 3-D rhs with one free dim
    L = sparse_rel(rng, (9, 6, 5), (2, 2, 2), 0.2)
    Rr = sparse_rel(rng, (6, 5, 7), (2, 2, 2), 0.2)
    yield "two_key", dict(lhs=L, rhs=Rr, join_keys=[(1, 0), (2, 1)], agg_keys=[(0, 0), (1, 2)],
                          kernel_string="ajk,jkb->ab", dtype="fp32")
    # no free dim: every output segment is a whole lhs run
    L = sparse_rel(rng, (20, 16), (4, 4), 0.3)
    Rr = sparse_rel(rng, (16,), (4,), 0.6)
    yield "no_free_dim", dict(lhs=L, rhs=Rr, join_keys=[(1, 0)], agg_keys=[(0, 0)],
                              kernel_string="ij,j->i", dtype="fp32")
    # long runs (1x1 tiles, 3,000 free indices: one set of cursors per run):
    # run 0 holds all 2,500 lhs tiles (three 1,024-tile chunks, ~24k pairs:
    # the per-pair walks), run 1 exactly 1,024 tiles over sparse rhs rows (one
    # chunk, ~6k pairs kept in LDS), run 2 ~250 tiles
    keep = np.zeros((3, 2500), dtype=bool)
    keep[0] = True
    keep[1, :1024] = True
    keep[2] = rng.random(2500) < 0.1
    L = rel_from_mask(rng, keep)
    rk = rng.random((2500, 3000)) < np.where(np.arange(2500) < 1024, 0.002, 0.004)[:, None]
    Rr = rel_from_mask(rng, rk)
    yield "long_runs", dict(lhs=L, rhs=Rr, join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)],
                            kernel_string="ij,jk->ik", dtype="fp32")
    # more runs (3,000 lhs rows) than count and fill blocks
    L = rel_from_mask(rng, rng.random((3000, 6)) < 0.3)
    Rr = rel_from_mask(rng, rng.random((6, 40)) < 0.3)
    yield "many_runs", dict(lhs=L, rhs=Rr, join_keys=[(1, 0)], agg_keys=[(0, 0), (1, 1)],
                            kernel_string="ij,jk->ik", dtype="fp32")


WL = list(workloads())


def oracle_segments(L, Rr, keys, agg):
    li, ri = R.coordinate_join(L.coords, Rr.coords, keys)
    oc = R.compute_output_coords(L.coords, Rr.coords, li, ri, agg)
    uc, perm, off, _ = R.segment_plan(oc)
    return li, uc, [(li[perm[off[u]:off[u + 1]]], ri[perm[off[u]:off[u + 1]]])
                    for u in range(len(uc))]


def run_row(L, Rr, keys, agg, cap_p=None, cap_u=None, lc=None, rc=None, direct=False):
    """ej_row_plan_async through the C ABI; host results clipped to the counts."""
    lib = _lib.load()
    lc = torch.from_numpy(np.ascontiguousarray(L.coords)).cuda() if lc is None else lc
    rc = torch.from_numpy(np.ascontiguousarray(Rr.coords)).cuda() if rc is None else rc
    lg, rg = grid(L), grid(Rr)
    nk = len(keys)
    cap_p = cap_p or max(1, len(L.coords) * len(Rr.coords))
    cap_u = cap_u or cap_p
    li = torch.full((cap_p,), -7, dtype=torch.int64, device="cuda")
    ri = torch.full((cap_p,), -7, dtype=torch.int64, device="cuda")
    coords = torch.full((cap_u, len(agg)), -7, dtype=torch.int32, device="cuda")
    off = torch.full((cap_u + 1,), -7, dtype=torch.int32, device="cuda")
    nbytes = ctypes.c_size_t()
    assert lib.ej_row_plan_workspace_size(lc.shape[0], rc.shape[0], int(np.prod(rg[:nk])),
                                          ctypes.byref(nbytes)) == 0
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device="cuda")
    dcounts = run_row.dcounts
    if direct:
        p = ctypes.c_void_p()
        assert lib.ej_host_alloc(64, ctypes.byref(p)) == 0
        counts_addr, view = p.value, (ctypes.c_int64 * 8).from_address(p.value)
        ticket = run_row.ticket = run_row.ticket % 1000 + 1
    else:
        counts = torch.full((8,), -7, dtype=torch.int64).pin_memory()
        counts_addr, ticket = counts.data_ptr(), 0
    st = lib.ej_row_plan_async(
        _device.ptr(lc), lc.shape[0], lc.shape[1], _device.ptr(rc), rc.shape[0], rc.shape[1], nk,
        _lib.i32_array([k[0] for k in keys]), _lib.i32_array([k[1] for k in keys]),
        _lib.i64_array(lg), _lib.i64_array(rg), len(agg), _lib.i32_array([a for a, _ in agg]),
        _lib.i32_array([b for _, b in agg]), _device.ptr(li), _device.ptr(ri), cap_p,
        _device.ptr(coords), _device.ptr(off), cap_u, _device.ptr(ws), nbytes.value,
        _device.ptr(dcounts), ctypes.c_void_p(counts_addr), ticket, _device.stream_ptr())
    if st != _lib.EJ_OK:
        return st, None
    torch.cuda.synchronize()
    if direct:
        word = view[6] & ((1 << 64) - 1)
        lib.ej_host_free(ctypes.c_void_p(counts_addr))
        assert word >> 44 == ticket
        m = (1 << 21) - 1
        flag, P, U = (word >> 42) & 3, (word >> 21) & m, word & m
        c = [U if not flag else 0, flag, min(P, cap_p), 0, P, 0]
    else:
        c = counts.tolist()[:6]
    assert int(dcounts[6]) == 0 and int(dcounts[7]) == 0  # left ready for the next call
    assert dcounts[:6].tolist() == c
    U, P = c[0], c[4]
    res = dict(counts=c, li=li[:P].cpu().numpy() if not c[1] else None,
               ri=ri[:P].cpu().numpy() if not c[1] else None, coords=coords[:U].cpu().numpy(),
               off=off[:U + 1].cpu().numpy())
    return st, res


run_row.ticket = 0


@pytest.fixture(autouse=True)
def _counts_buffer(gpu):
    run_row.dcounts = torch.zeros(8, dtype=torch.int64, device="cuda")
    yield


@pytest.mark.parametrize("idx", range(len(WL)))
@pytest.mark.parametrize("direct", [False, True])
def test_row_plan_matches_oracle_segments(gpu, idx, direct):
    """Output coordinates and, segment by segment, the pairs in the
    reference's accumulation order, bit-exact; the counts through the copy
    and through the packed word."""
    name, w = WL[idx]
    note("row plan vs oracle", name, "direct" if direct else "copy")
    L, Rr, keys, agg = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"]
    li_o, uc, segs = oracle_segments(L, Rr, keys, agg)
    st, res = run_row(L, Rr, keys, agg, direct=direct)
    assert st == _lib.EJ_OK and res["counts"][1] == 0, (name, st, res and res["counts"])
    assert res["counts"][4] == len(li_o) and res["counts"][0] == len(uc)
    npt.assert_array_equal(res["coords"], uc)
    assert res["off"][-1] == len(li_o)
    for u, (sl, sr) in enumerate(segs):
        a, b = res["off"][u], res["off"][u + 1]
        npt.assert_array_equal(res["li"][a:b], sl, err_msg=f"{name} segment {u}")
        npt.assert_array_equal(res["ri"][a:b], sr, err_msg=f"{name} segment {u}")


def test_row_plan_reports_capacity_and_bad_data(gpu):
    """Pairs or segments beyond the capacities: flag 2 with the true counts
    and nothing for the einsum; unsorted, duplicated or out-of-grid rows on
    either side: flag 1; a good call after each failure gives the full plan."""
    note("row plan capacities and checks")
    name, w = WL[1]
    L, Rr, keys, agg = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"]
    li_o, uc, _ = oracle_segments(L, Rr, keys, agg)
    P, U = len(li_o), len(uc)
    st, res = run_row(L, Rr, keys, agg, cap_p=P - 1)
    assert st == _lib.EJ_OK and res["counts"] == [0, 2, P - 1, 0, P, 0]
    st, res = run_row(L, Rr, keys, agg, cap_p=P, cap_u=U - 1)
    assert st == _lib.EJ_OK and res["counts"] == [0, 2, P, 0, P, 0]
    st, res = run_row(L, Rr, keys, agg, cap_p=P, cap_u=U, direct=True)
    assert st == _lib.EJ_OK and res["counts"] == [U, 0, P, 0, P, 0]

    def with_coords(r, c):
        return R.Rel(c, r.values, r.shape, r.tile_shape)

    bad = []
    c = L.coords.copy()
    c[[5, 6]] = c[[6, 5]]
    bad.append(("lhs swapped", with_coords(L, c), Rr))
    c = L.coords.copy()
    c[9] = c[8]
    bad.append(("lhs duplicate", with_coords(L, c), Rr))
    c = L.coords.copy()
    c[-1, 0] = grid(L)[0]
    bad.append(("lhs outside its grid", with_coords(L, c), Rr))
    c = Rr.coords.copy()
    c[[3, 4]] = c[[4, 3]]
    bad.append(("rhs swapped", L, with_coords(Rr, c)))
    c = Rr.coords.copy()
    c[0, 1] = -1
    bad.append(("rhs negative", L, with_coords(Rr, c)))
    for what, bl, br in bad:
        note("row plan bad data", what)
        st, res = run_row(bl, br, keys, agg)
        assert st == _lib.EJ_OK and res["counts"][1] == 1 and res["counts"][0] == 0, what
        st, res = run_row(L, Rr, keys, agg)
        assert st == _lib.EJ_OK and res["counts"] == [U, 0, P, 0, P, 0], what


def test_row_plan_refuses_other_structures(gpu):
    """Structures the plan cannot take are refused on the host (no launch)."""
    note("row plan structures")
    name, w = WL[1]
    L, Rr = w["lhs"], w["rhs"]
    st, _ = run_row(L, Rr, [(0, 0)], [(0, 1), (1, 1)])  # output not a lhs prefix
    assert st == _lib.EJ_E_UNSUPPORTED
    st, _ = run_row(L, Rr, [(1, 1)], [(0, 0), (1, 0)])  # joined on the rhs's last dim
    assert st == _lib.EJ_E_UNSUPPORTED
    assert b"row plan" in _lib.load().ej_last_error()


@pytest.mark.parametrize("idx", [0, 1, 2, 3])
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_row_step_bitwise_equals_general_plan(gpu, idx, dtype, monkeypatch):
    """execute_sparse through the row plan (the second call on the same
    relations, with the first call's pair count as its bound) against the
    general plan: the same coordinates and bitwise the same values; both
    within tolerance of the oracle."""
    name, w = WL[idx]
    note("row step vs general", name, dtype)
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    if dtype == "bf16":
        L = R.Rel(L.coords, R.bf16_round(L.values), L.shape, L.tile_shape)
        Rr = R.Rel(Rr.coords, R.bf16_round(Rr.values), Rr.shape, Rr.tile_shape)
    lhs, rhs = dev_rel(L, dtype), dev_rel(Rr, dtype)
    used = []
    real = _device.run_row_step

    def spy(step, ev=None):
        st, res = real(step, ev)
        used.append(st)
        return st, res

    monkeypatch.setattr(_device, "run_row_step", spy)
    sd._pair_hints.clear()
    sd._steps.clear()
    first = ej.execute_sparse(lhs, rhs, keys, ks, agg)  # exact path: sets the pair hint
    assert not used
    got = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    assert used == ["ok"]
    again = ej.execute_sparse(lhs, rhs, keys, ks, agg)  # the remembered step
    assert used == ["ok", "ok"]
    for res in (got, again):
        assert torch.equal(res.coords, first.coords)
        assert torch.equal(res.values.view(torch.int32 if dtype == "fp32" else torch.int16),
                           first.values.view(torch.int32 if dtype == "fp32" else torch.int16))
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)
    sd._steps.clear()
    general = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    assert torch.equal(got.coords, general.coords)
    assert torch.equal(got.values, general.values)
    want = R.execute_sparse(L, Rr, keys, ks, agg, precision="fp64")
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    tol = 1e-2 if dtype == "bf16" else 1e-5
    assert R.rel_l2(got.values.float().cpu().numpy(), want.values) <= tol


@pytest.mark.parametrize("idx", [0, 2])
def test_row_step_bf16_with_fp32_output(gpu, idx, monkeypatch):
    """bf16 relations with out_dtype=float32 through the row step: fp32
    output tiles, bitwise the general plan's, within 1e-5 of float64 math on
    the bf16-rounded inputs."""
    name, w = WL[idx]
    note("row step bf16 -> fp32", name)
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    L = R.Rel(L.coords, R.bf16_round(L.values), L.shape, L.tile_shape)
    Rr = R.Rel(Rr.coords, R.bf16_round(Rr.values), Rr.shape, Rr.tile_shape)
    lhs, rhs = dev_rel(L, "bf16"), dev_rel(Rr, "bf16")
    used = []
    real = _device.run_row_step
    monkeypatch.setattr(_device, "run_row_step",
                        lambda step, ev=None: used.append(1) or real(step, ev))
    sd._pair_hints.clear()
    sd._steps.clear()
    f32 = torch.float32
    ej.execute_sparse(lhs, rhs, keys, ks, agg, out_dtype=f32)
    got = ej.execute_sparse(lhs, rhs, keys, ks, agg, out_dtype=f32)
    assert used and got.values.dtype == f32
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)
    sd._steps.clear()
    general = ej.execute_sparse(lhs, rhs, keys, ks, agg, out_dtype=f32)
    assert torch.equal(got.coords, general.coords) and torch.equal(got.values, general.values)
    want = R.execute_sparse(L, Rr, keys, ks, agg, precision="fp64")
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    assert R.rel_l2(got.values.cpu().numpy(), want.values) <= 1e-5


def test_row_steps_on_two_streams(gpu, monkeypatch):
    """Two row steps of different sizes queued from one thread on two
    streams, back to back without a wait between them: each stream's plan
    has its own device counters, so both results equal the same steps run
    alone on one stream, bitwise."""
    note("row steps on two streams")
    used = []
    real = _device.run_row_step
    monkeypatch.setattr(_device, "run_row_step",
                        lambda step, ev=None: used.append(1) or real(step, ev))
    runs = []
    for idx in (0, 5):
        name, w = WL[idx]
        runs.append((dev_rel(w["lhs"]), dev_rel(w["rhs"]), w["join_keys"], w["kernel_string"],
                     w["agg_keys"]))
    sd._pair_hints.clear()
    sd._steps.clear()
    alone = [ej.execute_sparse(*r) for r in runs]  # exact path: sets the pair hints
    alone = [ej.execute_sparse(*r) for r in runs]
    torch.cuda.synchronize()
    assert len(used) == 2
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            a = ej.execute_sparse(*runs[0])
        with torch.cuda.stream(s2):
            b = ej.execute_sparse(*runs[1])
        torch.cuda.synchronize()
        for got, want in ((a, alone[0]), (b, alone[1])):
            assert torch.equal(got.coords, want.coords)
            assert torch.equal(got.values, want.values)
    assert len(used) == 8


def test_row_step_host_relations(gpu, monkeypatch):
    """Host (NumPy) relations called repeatedly: the later calls take the row
    step on device copies and return host arrays with the reference's dtypes
    (int32 coordinates, float32 values), equal to the first call's."""
    name, w = WL[1]
    note("row step, host relations", name)
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    lhs = SparseTensorRelation(L.coords, L.values, L.shape, L.tile_shape)
    rhs = SparseTensorRelation(Rr.coords, Rr.values, Rr.shape, Rr.tile_shape)
    used = []
    real = _device.run_row_step
    monkeypatch.setattr(_device, "run_row_step",
                        lambda step, ev=None: used.append(1) or real(step, ev))
    sd._pair_hints.clear()
    sd._steps.clear()
    res = [ej.execute_sparse(lhs, rhs, keys, ks, agg) for _ in range(3)]
    assert used
    for r in res:
        assert isinstance(r.coords, np.ndarray) and isinstance(r.values, np.ndarray)
        assert r.coords.dtype == np.int32 and r.values.dtype == np.float32
        npt.assert_array_equal(r.coords, res[0].coords)
        npt.assert_array_equal(r.values, res[0].values)
    want = R.execute_sparse(L, Rr, keys, ks, agg, precision="fp64")
    npt.assert_array_equal(res[-1].coords, want.coords)
    assert R.rel_l2(res[-1].values, want.values) <= 1e-5


@pytest.mark.parametrize("idx", [0, 1])
@pytest.mark.parametrize("dt", [torch.float64, torch.float16], ids=["f64", "f16"])
def test_row_step_other_float_dtypes(gpu, idx, dt, monkeypatch):
    """float64 and float16 relations through the row step (operands in fp32,
    results in the reference's dtype: float32 for float64 tiles, float16 for
    float16 tiles): bitwise the exact path's result, the oracle's
    coordinates, values within tolerance of float64 math."""
    name, w = WL[idx]
    note("row step dtype", name, dt)
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    vals = lambda r: torch.from_numpy(np.ascontiguousarray(r.values, dtype=np.float64)).cuda().to(dt)
    lhs = SparseTensorRelation(torch.from_numpy(np.ascontiguousarray(L.coords)).cuda(), vals(L),
                               L.shape, L.tile_shape)
    rhs = SparseTensorRelation(torch.from_numpy(np.ascontiguousarray(Rr.coords)).cuda(),
                               vals(Rr), Rr.shape, Rr.tile_shape)
    used = []
    real = _device.run_row_step
    monkeypatch.setattr(_device, "run_row_step",
                        lambda step, ev=None: used.append(1) or real(step, ev))
    sd._pair_hints.clear()
    sd._steps.clear()
    first = ej.execute_sparse(lhs, rhs, keys, ks, agg)  # exact path
    got = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    again = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    assert len(used) == 2
    want_dt = torch.float32 if dt == torch.float64 else torch.float16
    for res in (first, got, again):
        assert res.values.dtype == want_dt
    assert torch.equal(got.coords, first.coords) and torch.equal(got.values, first.values)
    assert torch.equal(again.values, first.values)
    Lh = R.Rel(L.coords, vals(L).double().cpu().numpy(), L.shape, L.tile_shape)
    Rh = R.Rel(Rr.coords, vals(Rr).double().cpu().numpy(), Rr.shape, Rr.tile_shape)
    want = R.execute_sparse(Lh, Rh, keys, ks, agg, precision="fp64")
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    tol = 1e-5 if dt == torch.float64 else 2e-3
    assert R.rel_l2(got.values.double().cpu().numpy(), want.values) <= tol


def test_row_step_full_size_zipf(gpu, monkeypatch):
    """The 32768^2 Zipf sparse x sparse workload (P = 54,516, U = 31,573)
    through the row plan: bitwise equal to the exact path's result and within
    fp32 tolerance of the oracle on a sample of segments."""
    note("row step, Zipf at full size")
    w = G.workload_sparse_sparse_zipf()
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    lhs, rhs = dev_rel(L), dev_rel(Rr)
    used = []
    real = _device.run_row_step
    monkeypatch.setattr(_device, "run_row_step",
                        lambda step, ev=None: used.append(1) or real(step, ev))
    sd._pair_hints.clear()
    sd._steps.clear()
    first = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    got = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    assert used and first.num_tuples == 31573
    assert torch.equal(got.coords, first.coords) and torch.equal(got.values, first.values)
    li, ri = R.coordinate_join(L.coords, Rr.coords, keys)
    assert len(li) == 54516


def test_row_step_answers_changed_data(gpu):
    """Coordinates rewritten in place (same tensors) so that the lhs is no
    longer sorted: the remembered row step reports a miss and the call is
    answered by the general plan, as the oracle answers it."""
    note("row step, data changed under the same tensors")
    name, w = WL[0]
    L, Rr, keys, agg, ks = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"], w["kernel_string"]
    lhs, rhs = dev_rel(L), dev_rel(Rr)
    sd._pair_hints.clear()
    sd._steps.clear()
    ej.execute_sparse(lhs, rhs, keys, ks, agg)
    ej.execute_sparse(lhs, rhs, keys, ks, agg)
    perm = np.arange(len(L.coords))
    perm[[0, 1]] = [1, 0]
    c2 = L.coords[perm]
    v2 = L.values[perm]
    lhs.coords.copy_(torch.from_numpy(c2).cuda())
    lhs.values.copy_(torch.from_numpy(v2).cuda())
    got = ej.execute_sparse(lhs, rhs, keys, ks, agg)
    want = R.execute_sparse(R.Rel(c2, v2, L.shape, L.tile_shape), Rr, keys, ks, agg,
                            precision="fp64")
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    assert R.rel_l2(got.values.cpu().numpy(), want.values) <= 1e-5
