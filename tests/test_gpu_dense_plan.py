"""The one-launch plan for a join against a dense rhs (ej_dense_plan_async).

The plan's pairs, grouped by segment, must equal the oracle's join and
segment plan (reference: execution/sparse_dispatch.py:29-82, :129-171)
pair for pair, in the reference's accumulation order; execute_sparse on it
must give results bitwise identical to the general plan's; and data that
breaks the dense structure must be detected on the device and answered by
the general plan, with the oracle's results.
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


def dev_rel(r: R.Rel, dtype="fp32", shape=None):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    vals = torch.from_numpy(np.ascontiguousarray(r.values, dtype=np.float32)).cuda().to(tdt)
    return SparseTensorRelation(torch.from_numpy(np.ascontiguousarray(r.coords)).cuda(), vals,
                                shape or r.shape, r.tile_shape)


def grid(r: R.Rel, shape=None):
    shape = shape or r.shape
    return [s // t for s, t in zip(shape, r.tile_shape)]


def run_plan(L, Rr, keys, agg, group=0, lshape=None):
    """ej_dense_plan_async through the C ABI; host results clipped to the counts."""
    lib = _lib.load()
    lc, rc = torch.from_numpy(L.coords).cuda(), torch.from_numpy(Rr.coords).cuda()
    lg, rg = grid(L, lshape), grid(Rr)
    nk = len(keys)
    NK = int(np.prod(rg[nk:])) if len(rg) > nk else 1
    cap_p = len(L.coords) * NK
    cap_u = cap_p
    li = torch.full((cap_p,), -7, dtype=torch.int64, device="cuda")
    ri = torch.full((cap_p,), -7, dtype=torch.int64, device="cuda")
    coords = torch.full((cap_u, len(agg)), -7, dtype=torch.int32, device="cuda")
    off = torch.full((cap_u + 1,), -7, dtype=torch.int32, device="cuda")
    order = torch.full((1 + cap_u,), -7, dtype=torch.int32, device="cuda")
    dcounts = torch.zeros(8, dtype=torch.int64, device="cuda")
    counts = torch.full((8,), -7, dtype=torch.int64).pin_memory()
    written = ctypes.c_int32(-1)
    st = lib.ej_dense_plan_async(
        _device.ptr(lc), lc.shape[0], lc.shape[1], _device.ptr(rc), rc.shape[0], rc.shape[1], nk,
        _lib.i32_array([k[0] for k in keys]), _lib.i32_array([k[1] for k in keys]),
        _lib.i64_array(lg), _lib.i64_array(rg), len(agg), _lib.i32_array([a for a, _ in agg]),
        _lib.i32_array([b for _, b in agg]), _device.ptr(li), _device.ptr(ri), cap_p,
        _device.ptr(coords), _device.ptr(off), cap_u, group,
        _device.ptr(order) if group else None, ctypes.byref(written), _device.ptr(dcounts),
        ctypes.c_void_p(counts.data_ptr()), 0, _device.stream_ptr())
    if st != _lib.EJ_OK:
        return st, None
    torch.cuda.synchronize()
    c = counts.tolist()
    U, P = c[0], c[4]
    assert int(dcounts[6]) == 0 and int(dcounts[7]) == 0  # left ready for the next call
    assert dcounts[:6].tolist() == c[:6]
    res = dict(counts=c[:6], dev_u=int(dcounts[0]), li=li[:P].cpu().numpy(),
               ri=ri[:P].cpu().numpy(), coords=coords[:U].cpu().numpy(),
               off=off[:U + 1].cpu().numpy(), written=written.value)
    if group:
        res["order"] = order[:1 + (U + group - 1) // group].cpu().numpy()
    return st, res


def oracle_segments(L, Rr, keys, agg):
    li, ri = R.coordinate_join(L.coords, Rr.coords, keys)
    oc = R.compute_output_coords(L.coords, Rr.coords, li, ri, agg)
    uc, perm, off, _ = R.segment_plan(oc)
    return li, uc, [(li[perm[off[u]:off[u + 1]]], ri[perm[off[u]:off[u + 1]]])
                    for u in range(len(uc))]


def xcd_chunks(ng):
    """The einsum's split of ng groups over the eight XCDs: XCD x runs
    positions [start_x, start_x + cnt_x) of the run order."""
    per, rem = divmod(ng, 8)
    out, st = [], 0
    for x in range(8):
        c = per + (1 if x < rem else 0)
        out.append((st, st + c))
        st += c
    return out


def snake_order(lens, gpr):
    """Runs ranked longest first (counts above 255 tie, ties by run index),
    dealt to XCDs 0-7, 7-0, 0-7, ...; XCD 0's runs first, each XCD's in rank
    order, each run's gpr groups in order."""
    nr = len(lens)
    ranked = sorted(range(nr), key=lambda r: (-min(lens[r], 255), r))
    xcd_runs = [[] for _ in range(8)]
    for p, r in enumerate(ranked):
        q = p % 8
        xcd_runs[7 - q if (p // 8) % 2 else q].append(r)
    return [r * gpr + k for x in range(8) for r in xcd_runs[x] for k in range(gpr)]


def check_run_order(order, segs, NK, group):
    """The dense plan's run order (order[0] is its header).  Where every
    run holds whole groups and the XCDs' equal shares of consecutive groups
    would leave one share's pair total more than 5% above the mean: the snake
    deal, each XCD's groups longest first, XCD pair totals within one run's
    weight of each other.  Otherwise no order: a header of 0, which the
    einsum ignores (groups run in plan order)."""
    ng = (len(segs) + group - 1) // group
    if NK % group:
        assert order[0] == 0
        return
    gpr = NK // group
    lens = [len(segs[r * NK][0]) for r in range(len(segs) // NK)]
    natural = [sum(group * lens[g // gpr] for g in range(a, b)) for a, b in xcd_chunks(ng)]
    if max(natural) * 8 * 100 <= sum(natural) * 105:
        assert order[0] == 0
        return
    assert order[0] == ng
    order = order[1:]
    npt.assert_array_equal(order, snake_order(lens, gpr))
    if len(lens) % 8:
        return
    # whole runs on every XCD: each XCD's share falls in non-increasing run
    # weights, and the shares' totals differ by at most one run's weight
    weight = [group * lens[g // gpr] for g in order]
    loads = []
    for a, b in xcd_chunks(len(order)):
        w = weight[a:b]
        assert all(x >= y for x, y in zip(w, w[1:]))
        loads.append(sum(w))
    assert max(loads) - min(loads) <= NK * max(lens)


def workloads():
    w3 = G.workload_order3(n=256, l=64, density=0.05)
    yield "blocksparse_1k", G.workload_blocksparse_1k()
    yield "blocksparse_128", G.workload_blocksparse_16k(seed=2, m=2048, n=1024, density=0.1)
    yield "banded", G.workload_batched_banded(b=2, n=1024)
    yield "order3", w3
    # a lhs whose join dims are its last two, against a 3-D dense rhs
    rng = np.random.default_rng(3)
    lc = np.array(sorted({(int(a), int(b), int(c)) for a, b, c in
                          rng.integers(0, (6, 5, 4), size=(60, 3))}), np.int32)
    L = R.Rel(lc, rng.standard_normal((len(lc), 2, 3, 4)).astype(np.float32), (12, 15, 16),
              (2, 3, 4))
    rc = np.stack(np.unravel_index(np.arange(5 * 4 * 3), (5, 4, 3)), 1).astype(np.int32)
    Rr = R.Rel(rc, rng.standard_normal((len(rc), 3, 4, 2)).astype(np.float32), (15, 16, 6),
               (3, 4, 2))
    yield "two_key", dict(lhs=L, rhs=Rr, join_keys=[(1, 0), (2, 1)], agg_keys=[(0, 0), (1, 2)],
                          kernel_string="ajk,jkb->ab", dtype="fp32")


@pytest.mark.parametrize("idx", range(5))
def test_dense_plan_matches_oracle_segments(gpu, idx):
    """Output coordinates and, segment by segment, the pairs in the
    reference's accumulation order, bit-exact; with a run order, a
    permutation of the live groups behind its header."""
    name, w = list(workloads())[idx]
    note("dense plan vs oracle", name)
    L, Rr, keys, agg = w["lhs"], w["rhs"], w["join_keys"], w["agg_keys"]
    li_o, uc, segs = oracle_segments(L, Rr, keys, agg)
    for group in (0, 2, 4):
        st, res = run_plan(L, Rr, keys, agg, group=group)
        assert st == _lib.EJ_OK and res["counts"][1] == 0, (name, st)
        assert res["counts"][4] == len(li_o) and res["counts"][0] == len(uc) == res["dev_u"]
        npt.assert_array_equal(res["coords"], uc)
        assert res["off"][-1] == len(li_o)
        for u, (sl, sr) in enumerate(segs):
            a, b = res["off"][u], res["off"][u + 1]
            npt.assert_array_equal(res["li"][a:b], sl, err_msg=f"{name} segment {u}")
            npt.assert_array_equal(res["ri"][a:b], sr, err_msg=f"{name} segment {u}")
        if group:
            assert res["written"] == 1
            check_run_order(res["order"], segs, int(np.prod(grid(Rr)[len(keys):])), group)


@pytest.mark.parametrize("idx", range(5))
def test_dense_step_bitwise_equals_general_plan(gpu, idx, monkeypatch):
    """execute_sparse on the dense plan against the general plan: the same
    coordinates and bitwise the same values (same pairs, same order, same
    kernel), default and fp32 output; both within tolerance of the oracle."""
    name, w = list(workloads())[idx]
    note("dense step vs general", name)
    statuses = []
    real = _device.run_dense_step

    def spy(*a, **k):
        st, res = real(*a, **k)
        statuses.append(st)
        return st, res

    monkeypatch.setattr(_device, "run_dense_step", spy)
    lhs, rhs = dev_rel(w["lhs"], w["dtype"]), dev_rel(w["rhs"], w["dtype"])
    args = (lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    want = R.execute_sparse(w["lhs"], w["rhs"], w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    for out_dtype in (None, torch.float32):
        sd._pair_hints.clear()
        sd._steps.clear()
        dense = [ej.execute_sparse(*args, out_dtype=out_dtype) for _ in range(2)]
        assert statuses[-2:] == ["ok", "ok"]
        with monkeypatch.context() as m:
            m.setattr(sd, "_dense_step", lambda *a, **k: None)
            m.setattr(sd, "_row_step", lambda *a, **k: None)
            sd._steps.clear()
            general = ej.execute_sparse(*args, out_dtype=out_dtype)
            sd._steps.clear()
        for d in dense:
            assert torch.equal(d.coords, general.coords)
            bits = torch.int16 if d.values.dtype == torch.bfloat16 else torch.int32
            assert torch.equal(d.values.view(bits), general.values.view(bits))
        npt.assert_array_equal(dense[0].coords.cpu().numpy(), want.coords)
        tol = 1e-2 if w["dtype"] == "bf16" and out_dtype is None else 1e-5
        assert R.rel_l2(dense[0].values.float().cpu().numpy(), want.values) <= tol


@pytest.mark.parametrize("dt", [torch.float64, torch.float16], ids=["f64", "f16"])
def test_dense_step_other_float_dtypes(gpu, dt, monkeypatch):
    """float64 and float16 relations through the dense step (operands in
    fp32, results in the reference's dtype: float32 for float64 tiles,
    float16 for float16 tiles): bitwise the exact path's result, the
    oracle's coordinates, values within tolerance of float64 math."""
    name, w = list(workloads())[0]
    note("dense step dtype", name, dt)
    L, Rr = w["lhs"], w["rhs"]
    keys, agg, ks = w["join_keys"], w["agg_keys"], w["kernel_string"]
    vals = lambda r: torch.from_numpy(np.ascontiguousarray(r.values, dtype=np.float64)).cuda().to(dt)
    lhs = SparseTensorRelation(torch.from_numpy(L.coords).cuda(), vals(L), L.shape, L.tile_shape)
    rhs = SparseTensorRelation(torch.from_numpy(Rr.coords).cuda(), vals(Rr), Rr.shape,
                               Rr.tile_shape)
    statuses = []
    real = _device.run_dense_step
    monkeypatch.setattr(_device, "run_dense_step",
                        lambda *a, **k: statuses.append(1) or real(*a, **k))
    sd._pair_hints.clear()
    sd._steps.clear()
    res = [ej.execute_sparse(lhs, rhs, keys, ks, agg) for _ in range(3)]
    assert statuses
    want_dt = torch.float32 if dt == torch.float64 else torch.float16
    for r in res:
        assert r.values.dtype == want_dt
        assert torch.equal(r.coords, res[0].coords) and torch.equal(r.values, res[0].values)
    with monkeypatch.context() as m:
        m.setattr(sd, "_dense_step", lambda *a, **k: None)
        m.setattr(sd, "_row_step", lambda *a, **k: None)
        sd._steps.clear()
        general = ej.execute_sparse(lhs, rhs, keys, ks, agg, fused=True)
        sd._steps.clear()
    assert torch.equal(general.values, res[0].values)
    Lh = R.Rel(L.coords, vals(L).double().cpu().numpy(), L.shape, L.tile_shape)
    Rh = R.Rel(Rr.coords, vals(Rr).double().cpu().numpy(), Rr.shape, Rr.tile_shape)
    want = R.execute_sparse(Lh, Rh, keys, ks, agg, precision="fp64")
    npt.assert_array_equal(res[1].coords.cpu().numpy(), want.coords)
    tol = 1e-5 if dt == torch.float64 else 2e-3
    assert R.rel_l2(res[1].values.double().cpu().numpy(), want.values) <= tol


def _shuffled(r: R.Rel, seed: int) -> R.Rel:
    p = np.random.default_rng(seed).permutation(len(r.coords))
    return R.Rel(r.coords[p], r.values[p], r.shape, r.tile_shape)


def _cases():
    w = G.workload_blocksparse_1k(n=512, tile=32, density=0.2)
    L, Rr = w["lhs"], w["rhs"]
    yield "lhs unsorted", w, _shuffled(L, 1), Rr, None
    yield "rhs out of grid order", w, L, _shuffled(Rr, 2), None
    dup = R.Rel(np.concatenate([L.coords[:5], L.coords[4:]]),
                np.concatenate([L.values[:5], L.values[4:]]), L.shape, L.tile_shape)
    yield "lhs duplicate coordinates", w, dup, Rr, None
    yield "lhs shape understates rows", w, L, Rr, (256, 512)
    # a join value beyond the rhs grid: those lhs tiles meet no rhs tile
    wide = R.Rel(np.concatenate([L.coords, [[15, 17]]]).astype(np.int32),
                 np.concatenate([L.values, L.values[:1]]), (512, 576), L.tile_shape)
    yield "lhs join value beyond the rhs grid", w, wide, Rr, None
    # more runs (9000) than the plan keeps
    n = 9000
    lr = R.Rel(np.stack([np.arange(n), np.zeros(n, int)], 1).astype(np.int32),
               np.ones((n, 1, 1), np.float32), (n, 1), (1, 1))
    rr = R.Rel(np.array([[0, 0], [0, 1]], np.int32), np.full((2, 1, 1), 2.0, np.float32),
               (1, 2), (1, 1))
    yield "9000 runs", dict(w, lhs=lr, rhs=rr), lr, rr, None


@pytest.mark.parametrize("case", range(6))
def test_dense_plan_misses_fall_back(gpu, case, monkeypatch):
    """Data that breaks the dense structure: the plan reports the miss
    (counts[1] = 1, no segments on the device), execute_sparse answers with
    the general plan (the oracle's results), and later calls on the same
    coordinates skip the dense plan."""
    name, w, L, Rr, lshape = list(_cases())[case]
    note("dense miss", name)
    st, res = run_plan(L, Rr, w["join_keys"], w["agg_keys"], lshape=lshape)
    assert st == _lib.EJ_OK and res["counts"][1] == 1 and res["dev_u"] == 0, name
    statuses = []
    real = _device.run_dense_step

    def spy(*a, **k):
        st, r = real(*a, **k)
        statuses.append(st)
        return st, r

    monkeypatch.setattr(_device, "run_dense_step", spy)
    sd._pair_hints.clear()
    sd._steps.clear()
    lhs = dev_rel(L, shape=lshape)
    rhs = dev_rel(Rr)
    want = R.execute_sparse(L, Rr, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            output_shape=None if lshape is None else
                            (lshape[0], Rr.shape[1]), precision="fp64")
    for _ in range(2):
        got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
        npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
        assert R.rel_l2(got.values.float().cpu().numpy(), want.values) <= 1e-5
    assert statuses == ["miss"]


def test_dense_plan_at_its_lhs_limit(gpu):
    """16384 lhs tiles (every tile of a 64 x 256 grid of 1 x 1 tiles)
    against a dense 256 x 8 rhs: 131,072 pairs over 64 plan blocks, 512
    segments; one tile more is refused on the host."""
    note("dense plan at 16384 lhs tiles")
    rng = np.random.default_rng(8)
    lc = np.stack(np.unravel_index(np.arange(64 * 256), (64, 256)), 1).astype(np.int32)
    rc = np.stack(np.unravel_index(np.arange(256 * 8), (256, 8)), 1).astype(np.int32)
    L = R.Rel(lc, rng.standard_normal((len(lc), 1, 1)).astype(np.float32), (64, 256), (1, 1))
    Rr = R.Rel(rc, rng.standard_normal((len(rc), 1, 1)).astype(np.float32), (256, 8), (1, 1))
    keys, agg = [(1, 0)], [(0, 0), (1, 1)]
    li_o, uc, segs = oracle_segments(L, Rr, keys, agg)
    st, res = run_plan(L, Rr, keys, agg, group=4)
    assert st == _lib.EJ_OK and res["counts"][1] == 0 and res["counts"][4] == 131072
    # a wrong rhs row near the end (checked by one of the last plan blocks)
    # and, separately, two lhs rows out of order: each is reported as a miss
    bad_r = R.Rel(Rr.coords.copy(), Rr.values, Rr.shape, Rr.tile_shape)
    bad_r.coords[2000] = bad_r.coords[2001]
    st, miss = run_plan(L, bad_r, keys, agg, group=4)
    assert st == _lib.EJ_OK and miss["counts"][1] == 1 and miss["dev_u"] == 0
    bad_l = R.Rel(L.coords.copy(), L.values, L.shape, L.tile_shape)
    bad_l.coords[[9000, 9001]] = bad_l.coords[[9001, 9000]]
    st, miss = run_plan(bad_l, Rr, keys, agg)
    assert st == _lib.EJ_OK and miss["counts"][1] == 1 and miss["dev_u"] == 0
    st, again = run_plan(L, Rr, keys, agg, group=4)  # the counters were left ready
    assert st == _lib.EJ_OK and again["counts"] == res["counts"]
    big = R.Rel(np.stack(np.unravel_index(np.arange(16385), (16385, 1)), 1).astype(np.int32),
                np.ones((16385, 1, 1), np.float32), (16385, 1), (1, 1))
    one = R.Rel(np.array([[0, 0]], np.int32), np.ones((1, 1, 1), np.float32), (1, 1), (1, 1))
    assert run_plan(big, one, keys, agg)[0] == _lib.EJ_E_UNSUPPORTED
    npt.assert_array_equal(res["coords"], uc)
    for u in range(0, len(uc), 37):
        a, b = res["off"][u], res["off"][u + 1]
        npt.assert_array_equal(res["li"][a:b], segs[u][0])
        npt.assert_array_equal(res["ri"][a:b], segs[u][1])
    got = ej.execute_sparse(dev_rel(L), dev_rel(Rr), keys, "ij,jk->ik", agg)
    want = R.execute_sparse(L, Rr, keys, "ij,jk->ik", agg, precision="fp64")
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    assert R.rel_l2(got.values.cpu().numpy(), want.values) <= 1e-5


def test_dense_plan_tall_rhs(gpu):
    """Three lhs tiles against a dense 4096 x 2 rhs: one plan block checks
    all 8192 rhs rows (eight per thread); a wrong row at either end is a
    miss, and the plan matches the oracle's."""
    note("dense plan, tall rhs")
    rng = np.random.default_rng(9)
    lc = np.array([[0, 5], [0, 4000], [2, 17]], np.int32)
    rc = np.stack(np.unravel_index(np.arange(4096 * 2), (4096, 2)), 1).astype(np.int32)
    L = R.Rel(lc, rng.standard_normal((3, 2, 2)).astype(np.float32), (6, 8192), (2, 2))
    Rr = R.Rel(rc, rng.standard_normal((len(rc), 2, 2)).astype(np.float32), (8192, 4), (2, 2))
    keys, agg = [(1, 0)], [(0, 0), (1, 1)]
    li_o, uc, segs = oracle_segments(L, Rr, keys, agg)
    st, res = run_plan(L, Rr, keys, agg, group=2)
    assert st == _lib.EJ_OK and res["counts"][1] == 0 and res["counts"][4] == 6
    npt.assert_array_equal(res["coords"], uc)
    for u in range(len(uc)):
        a, b = res["off"][u], res["off"][u + 1]
        npt.assert_array_equal(res["li"][a:b], segs[u][0])
        npt.assert_array_equal(res["ri"][a:b], segs[u][1])
    for row in (0, 8191):
        bad_r = R.Rel(Rr.coords.copy(), Rr.values, Rr.shape, Rr.tile_shape)
        bad_r.coords[row, 1] ^= 1
        st, miss = run_plan(L, bad_r, keys, agg, group=2)
        assert st == _lib.EJ_OK and miss["counts"][1] == 1 and miss["dev_u"] == 0


def test_dense_run_order_balances_xcds(gpu):
    """The headline's 128 runs of Binomial(128, 0.05) lhs tiles against 32
    free rhs tiles, groups of 2: the snake deal leaves the XCDs' pair totals
    within 3% of their mean (16 whole runs each), where equal shares of
    consecutive runs differ by 13%."""
    note("dense run order balance")
    w = G.workload_blocksparse_16k(values=False)
    L = R.Rel(w["lhs"].coords, np.zeros((len(w["lhs"].coords), 1, 1), np.float32),
              (128, 128), (1, 1))
    rc = np.stack(np.unravel_index(np.arange(128 * 32), (128, 32)), 1).astype(np.int32)
    Rr = R.Rel(rc, np.zeros((len(rc), 1, 1), np.float32), (128, 32), (1, 1))
    keys, agg = [(1, 0)], [(0, 0), (1, 1)]
    li_o, uc, segs = oracle_segments(L, Rr, keys, agg)
    st, res = run_plan(L, Rr, keys, agg, group=2)
    assert st == _lib.EJ_OK and res["counts"][0] == 4096
    order = res["order"][1:]
    check_run_order(res["order"], segs, 32, 2)
    lens = np.bincount(L.coords[:, 0], minlength=128)
    loads = [sum(2 * lens[g // 16] for g in order[a:b]) for a, b in xcd_chunks(2048)]
    assert max(loads) / np.mean(loads) < 1.03
    naive = [2 * 16 * lens[16 * x:16 * x + 16].sum() for x in range(8)]
    assert max(naive) / np.mean(naive) > 1.10


def test_dense_steps_on_two_streams(gpu):
    """Two dense steps of different sizes queued from one thread on two
    streams, back to back without a wait between them: each stream's plan
    has its own device counters, so both results equal the same steps run
    alone on one stream, bitwise."""
    note("dense steps on two streams")
    wa = G.workload_blocksparse_16k(seed=4, m=2048, n=1024, density=0.2)
    wb = G.workload_blocksparse_1k(n=512, tile=32, density=0.1)
    runs = []
    for w in (wa, wb):
        lhs, rhs = dev_rel(w["lhs"], w["dtype"]), dev_rel(w["rhs"], w["dtype"])
        runs.append((lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"]))
    alone = [ej.execute_sparse(*r) for r in runs]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            a = ej.execute_sparse(*runs[0])
        with torch.cuda.stream(s2):
            b = ej.execute_sparse(*runs[1])
        torch.cuda.synchronize()
        for got, want in ((a, alone[0]), (b, alone[1])):
            assert torch.equal(got.coords, want.coords)
            bits = torch.int16 if got.values.dtype == torch.bfloat16 else torch.int32
            assert torch.equal(got.values.view(bits), want.values.view(bits))
