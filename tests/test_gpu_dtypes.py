"""GPU parity for the reference's value dtypes and coordinate ranges.

The reference accepts integer and boolean tile values (kernel_einsum hands
them to jnp.array / jnp.einsum, sparse_dispatch.py:125, and segment_sum keeps
the values' numpy dtype, :164-169) and any integer coordinates (its joins and
segment sums are dict-based, :65-80, :156-161).  These tests run those cases
through the HIP path and compare with the oracle: integer and boolean results
bit-exact and of the reference's dtype, float64 / float16 segment sums bit-exact
(the same sequential additions), floating einsums within the usual tolerance,
coordinates bit-exact.
"""

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import reference_path as R

import einjax_amd as ej
from einjax_amd import SparseTensorRelation
from einjax_amd.kernels import coordinate_join_hash, coordinate_join_sorted

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


# ---------------------------------------------------------------------------
# the reference's own edge cases (tests/test_rigorous.py:938-970)

def test_reference_kernel_einsum_single_pair_int_rhs(gpu):
    note("kernel_einsum eye(2) float64 x int64 tile (test_rigorous.py:938-945)")
    lhs = np.eye(2).reshape(1, 2, 2)
    rhs = np.array([[[1, 2], [3, 4]]])
    result = ej.kernel_einsum(lhs, rhs, np.array([0]), np.array([0]), "ij,jk->ik")
    assert result.dtype == np.float32  # jnp: float32 with int32 -> float32
    npt.assert_array_almost_equal(result[0], [[1, 2], [3, 4]])


def test_reference_segment_sum_int_single_entry(gpu):
    note("segment_sum of one int64 tile (test_rigorous.py:958-963)")
    values = np.array([[[1, 2], [3, 4]]])
    coords = np.array([[0, 0]])
    unique_coords, agg = ej.segment_sum(values, coords)
    assert agg.shape == (1, 2, 2)
    assert agg.dtype == values.dtype
    npt.assert_array_equal(agg[0], [[1, 2], [3, 4]])
    npt.assert_array_equal(unique_coords, [[0, 0]])


def test_reference_segment_sum_three_entries_same_coord(gpu):
    note("segment_sum of three float64 ones tiles (test_rigorous.py:965-970)")
    values = np.ones((3, 2, 2))
    coords = np.array([[0, 0], [0, 0], [0, 0]])
    _, agg = ej.segment_sum(values, coords)
    assert agg.shape == (1, 2, 2) and agg.dtype == np.float64
    npt.assert_array_equal(agg[0], np.ones((2, 2)) * 3)


# ---------------------------------------------------------------------------
# integer and boolean einsums

PAIRS = [(np.int32, np.int32), (np.int64, np.int64), (np.int8, np.int8), (np.uint8, np.int8),
         (np.int16, np.int32), (np.bool_, np.bool_), (np.bool_, np.int8), (np.uint32, np.uint32)]
SPECS = [("ij,jk->ik", (6, 5), (5, 7)), ("ij,ij->ij", (4, 6), (4, 6)), ("i,i->", (9,), (9,)),
         ("ij,kj->ik", (3, 8), (5, 8)), ("ijk,kl->ijl", (2, 3, 4), (4, 5))]


def _rand_int(rng, dt, shape):
    if dt == np.bool_:
        return rng.random(shape) < 0.4
    info = np.iinfo(dt)
    return rng.integers(max(info.min, -2 ** 40), min(info.max, 2 ** 40), size=shape,
                        endpoint=True).astype(dt)


@pytest.mark.parametrize("dts", PAIRS, ids=lambda d: f"{np.dtype(d[0]).name}-{np.dtype(d[1]).name}")
@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s[0])
def test_integer_kernel_einsum_bit_exact(gpu, dts, spec):
    ks, lt, rt = spec
    note("integer kernel_einsum", ks, dts)
    rng = np.random.default_rng(7)
    L = _rand_int(rng, dts[0], (5, *lt))
    Rt = _rand_int(rng, dts[1], (4, *rt))
    li = rng.integers(0, 5, 23)
    ri = rng.integers(0, 4, 23)
    got = ej.kernel_einsum(L, Rt, li, ri, ks)
    want = R.kernel_einsum_typed(L, Rt, li, ri, ks)
    assert got.dtype == want.dtype
    npt.assert_array_equal(got, want)


def test_integer_kernel_einsum_device_tensors(gpu):
    note("integer kernel_einsum on device int64 tensors")
    rng = np.random.default_rng(8)
    L = rng.integers(-2 ** 33, 2 ** 33, (6, 8, 8))
    Rt = rng.integers(-2 ** 33, 2 ** 33, (6, 8, 8))
    li, ri = rng.integers(0, 6, 40), rng.integers(0, 6, 40)
    got = ej.kernel_einsum(torch.from_numpy(L).cuda(), torch.from_numpy(Rt).cuda(),
                           torch.from_numpy(li).cuda(), torch.from_numpy(ri).cuda(), "ij,jk->ik")
    assert got.is_cuda and got.dtype == torch.int32
    npt.assert_array_equal(got.cpu().numpy(), R.kernel_einsum_typed(L, Rt, li, ri, "ij,jk->ik"))


@pytest.mark.parametrize("dts", [(np.float32, np.int64), (np.int32, np.float64),
                                 (np.float16, np.int8), (np.float16, np.float16)],
                         ids=lambda d: f"{np.dtype(d[0]).name}-{np.dtype(d[1]).name}")
def test_mixed_and_float16_kernel_einsum(gpu, dts):
    note("mixed / float16 kernel_einsum", dts)
    rng = np.random.default_rng(9)

    def vals(dt, shape):
        if np.dtype(dt).kind == "f":
            return rng.standard_normal(shape).astype(dt)
        return rng.integers(-50, 50, shape).astype(dt)

    L, Rt = vals(dts[0], (4, 16, 16)), vals(dts[1], (3, 16, 16))
    li, ri = rng.integers(0, 4, 10), rng.integers(0, 3, 10)
    got = ej.kernel_einsum(L, Rt, li, ri, "ij,jk->ik")
    want = R.kernel_einsum_typed(L, Rt, li, ri, "ij,jk->ik")
    assert got.dtype == want.dtype
    truth = R.kernel_einsum(L.astype(np.float64), Rt.astype(np.float64), li, ri, "ij,jk->ik",
                            precision="fp64")
    tol = 1e-2 if want.dtype == np.float16 else 1e-5
    assert R.rel_l2(got.astype(np.float64), truth) <= tol


def test_integer_execute_sparse_bit_exact(gpu):
    note("execute_sparse on int32 relations, fused and unfused")
    rng = np.random.default_rng(10)
    nl, nr, t = 40, 30, 8
    lc = np.unique(rng.integers(0, 8, (nl, 2)), axis=0).astype(np.int32)
    rc = np.unique(rng.integers(0, 8, (nr, 2)), axis=0).astype(np.int32)
    lv = rng.integers(-2 ** 31, 2 ** 31 - 1, (len(lc), t, t)).astype(np.int32)
    rv = rng.integers(-2 ** 31, 2 ** 31 - 1, (len(rc), t, t)).astype(np.int32)
    lhs = SparseTensorRelation(lc, lv, (64, 64), (t, t))
    rhs = SparseTensorRelation(rc, rv, (64, 64), (t, t))
    jk, ak = [(1, 0)], [(0, 0), (1, 1)]
    li, ri = R.coordinate_join(lc, rc, jk)
    tiles = R.kernel_einsum_typed(lv, rv, li, ri, "ij,jk->ik")
    want_c, want_v = R.segment_sum(tiles, R.compute_output_coords(lc, rc, li, ri, ak))
    for fused in (True, False):
        got = ej.execute_sparse(lhs, rhs, jk, "ij,jk->ik", ak, fused=fused)
        npt.assert_array_equal(got.coords, want_c)
        assert got.values.dtype == np.int32
        npt.assert_array_equal(got.values, want_v)
    dl = SparseTensorRelation(torch.from_numpy(lc).cuda(), torch.from_numpy(lv).cuda(),
                              (64, 64), (t, t))
    dr = SparseTensorRelation(torch.from_numpy(rc).cuda(), torch.from_numpy(rv).cuda(),
                              (64, 64), (t, t))
    got = ej.execute_sparse(dl, dr, jk, "ij,jk->ik", ak)
    assert got.values.dtype == torch.int32
    npt.assert_array_equal(got.values.cpu().numpy(), want_v)


# ---------------------------------------------------------------------------
# segment sums in the values' dtype

@pytest.mark.parametrize("dt", [np.float64, np.float32, np.float16, np.int64, np.int32, np.int8,
                                np.uint8, np.uint32, np.uint64, np.bool_],
                         ids=lambda d: np.dtype(d).name)
def test_segment_sum_dtypes_bit_exact(gpu, dt):
    note("segment_sum", np.dtype(dt).name)
    rng = np.random.default_rng(11)
    P = 300
    if np.dtype(dt).kind == "f":
        v = (rng.standard_normal((P, 3, 5)) * 10.0 ** rng.integers(-3, 4, (P, 1, 1))).astype(dt)
    else:
        v = _rand_int(rng, dt, (P, 3, 5))
    oc = rng.integers(-3, 4, (P, 2)).astype(np.int32)  # negative coordinates too
    want_c, want_v = R.segment_sum(v, oc)
    got_c, got_v = ej.segment_sum(v, oc)
    npt.assert_array_equal(got_c, want_c)
    assert got_v.dtype == want_v.dtype
    npt.assert_array_equal(got_v, want_v)


def test_segment_sum_device_int64_and_bool(gpu):
    note("segment_sum on device int64 and bool tensors")
    rng = np.random.default_rng(12)
    oc = rng.integers(0, 5, (100, 1)).astype(np.int32)
    for v in (rng.integers(-2 ** 62, 2 ** 62, (100, 4)), rng.random((100, 4)) < 0.1):
        want_c, want_v = R.segment_sum(v, oc)
        got_c, got_v = ej.segment_sum(torch.from_numpy(v).cuda(), torch.from_numpy(oc).cuda())
        assert got_v.is_cuda
        npt.assert_array_equal(got_c.cpu().numpy(), want_c)
        npt.assert_array_equal(got_v.cpu().numpy(), want_v)


# ---------------------------------------------------------------------------
# negative coordinates

def test_negative_coordinates_join_and_execute(gpu):
    note("negative tile coordinates: joins, execute_sparse")
    rng = np.random.default_rng(13)
    lc = np.unique(rng.integers(-6, 6, (60, 2)), axis=0).astype(np.int32)
    rc = np.unique(rng.integers(-5, 7, (50, 2)), axis=0).astype(np.int32)
    t = 4
    lv = rng.standard_normal((len(lc), t, t)).astype(np.float32)
    rv = rng.standard_normal((len(rc), t, t)).astype(np.float32)
    jk, ak = [(1, 0)], [(0, 0), (1, 1)]
    want_l, want_r = R.coordinate_join(lc, rc, jk)
    lhs = SparseTensorRelation(lc, lv, (48, 48), (t, t))
    rhs = SparseTensorRelation(rc, rv, (48, 48), (t, t))
    got_l, got_r = ej.coordinate_join(lhs, rhs, jk)
    npt.assert_array_equal(got_l, want_l)
    npt.assert_array_equal(got_r, want_r)
    for fn, ref in ((coordinate_join_hash, R.coordinate_join_hash),
                    (coordinate_join_sorted, R.coordinate_join_sorted)):
        a, b = fn(lc, rc, [(1, 0)])
        wa, wb = ref(lc, rc, [(1, 0)])
        npt.assert_array_equal(a, wa)
        npt.assert_array_equal(b, wb)
    want = R.execute_sparse(R.Rel(lc, lv, (48, 48), (t, t)), R.Rel(rc, rv, (48, 48), (t, t)),
                            jk, "ij,jk->ik", ak, precision="fp64")
    for fused in (True, False):
        got = ej.execute_sparse(lhs, rhs, jk, "ij,jk->ik", ak, fused=fused)
        npt.assert_array_equal(got.coords, want.coords)
        assert R.rel_l2(got.values, want.values) <= 1e-5
    dl = SparseTensorRelation(torch.from_numpy(lc).cuda(), torch.from_numpy(lv).cuda(),
                              (48, 48), (t, t))
    dr = SparseTensorRelation(torch.from_numpy(rc).cuda(), torch.from_numpy(rv).cuda(),
                              (48, 48), (t, t))
    for _ in range(2):  # the second call takes the queued path's fallbacks
        got = ej.execute_sparse(dl, dr, jk, "ij,jk->ik", ak)
        npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
        assert R.rel_l2(got.values.cpu().numpy(), want.values) <= 1e-5
