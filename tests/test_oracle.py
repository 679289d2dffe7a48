"""Pins the CPU oracle (oracle/reference_path.py) before it is trusted.

Each check is a known answer from the reference's own tests, a golden vector
written by the reference's code (tests/golden/make_golden.py), a brute-force
result on tiny inputs, a closed form, or a library routine.  The checks are
chosen so that a plausible mistake (wrong pair order, transposed operand,
dropped term, wrong rounding) fails at least one of them.
"""

from pathlib import Path

import numpy as np
import numpy.testing as npt
import pytest

from oracle import generators as G
from oracle import reference_path as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "join_order.npz"


def rel(dense, tile):
    return R.dense_to_relation(np.asarray(dense, dtype=np.float64), tile)


# ---------------------------------------------------------------------------
# to_relation (reference tests/test_sparse.py:216-291)

def test_to_relation_identity_tiling():
    data = np.array([[1.0, 0.0], [0.0, 2.0]])
    r = rel(data, (2, 2))
    npt.assert_array_equal(r.coords, [[0, 0]])
    npt.assert_array_equal(r.values[0], data)


def test_to_relation_diagonal():
    r = rel(np.diag([1.0, 2.0, 3.0, 4.0]), (2, 2))
    npt.assert_array_equal(r.coords, [[0, 0], [1, 1]])
    npt.assert_array_equal(r.values[0], [[1, 0], [0, 2]])
    npt.assert_array_equal(r.values[1], [[3, 0], [0, 4]])


def test_to_relation_skips_empty_and_roundtrips():
    d = np.zeros((4, 4))
    d[0, 0] = 1.0
    r = rel(d, (2, 2))
    npt.assert_array_equal(r.coords, [[0, 0]])
    data = np.array([[1.0, 0, 0, 2], [0, 3, 0, 0], [0, 0, 4, 0], [5, 0, 0, 6]])
    npt.assert_array_equal(R.relation_to_dense(rel(data, (2, 2))), data)


def test_to_relation_errors_and_empty():
    with pytest.raises(ValueError):
        rel(np.eye(3), (2, 2))
    r = rel(np.zeros((4, 4)), (2, 2))
    assert r.coords.shape == (0, 2) and r.values.shape == (0, 2, 2)


def test_to_relation_3d():
    d = np.zeros((4, 4, 4))
    d[0, 0, 0] = 1.0
    d[3, 3, 3] = 2.0
    r = rel(d, (2, 2, 2))
    npt.assert_array_equal(r.coords, [[0, 0, 0], [1, 1, 1]])
    npt.assert_array_equal(R.relation_to_dense(r), d)


def test_to_relation_brute_force():
    rng = np.random.default_rng(3)
    d = rng.standard_normal((12, 18)) * (rng.random((12, 18)) < 0.05)
    r = rel(d, (3, 6))
    tiles = [(i, j) for i in range(4) for j in range(3)
             if np.any(d[3 * i:3 * i + 3, 6 * j:6 * j + 6] != 0)]
    npt.assert_array_equal(r.coords, np.array(tiles).reshape(-1, 2))
    npt.assert_array_equal(R.relation_to_dense(r), d)


def test_extract_coo_known_answers():
    # reference tests/test_sparse.py:318-355
    idx, vals, shape = R.extract_coo(np.array([[1.0, 0.0], [0.0, 2.0]]))
    assert shape == (2, 2) and idx.dtype == np.int32 and vals.dtype == np.float64
    npt.assert_array_equal(idx, [[0, 0], [1, 1]])
    npt.assert_array_equal(vals, [1.0, 2.0])
    idx, vals, shape = R.extract_coo(np.zeros((3, 3)))
    assert shape == (3, 3) and idx.shape == (0, 2) and len(vals) == 0
    idx, vals, shape = R.extract_coo(np.array([0.0, 1.0, 0.0, 3.0]))
    assert shape == (4,) and len(vals) == 2
    import scipy.sparse as sp

    idx, vals, shape = R.extract_coo(sp.csr_matrix(np.array([[1.0, 0.0], [0.0, 2.0]])))
    assert shape == (2, 2) and len(vals) == 2


def test_extract_coo_row_major_brute_force():
    rng = np.random.default_rng(5)
    d = rng.standard_normal((5, 7, 3)) * (rng.random((5, 7, 3)) < 0.3)
    d[0, 0, 0] = np.nan  # NaN != 0: kept
    d[1, 1, 1] = -0.0    # -0.0 == 0: dropped
    idx, vals, _ = R.extract_coo(d)
    want = [(i, j, k) for i in range(5) for j in range(7) for k in range(3)
            if not (d[i, j, k] == 0)]
    npt.assert_array_equal(idx, np.array(want))
    npt.assert_array_equal(vals, np.array([d[w] for w in want]))


def test_to_relation_from_coo_repeats_keep_last_entry():
    # A COO list with repeated elements and explicit zeros: the tiles equal a
    # sequential write of the nonzero entries in list order (the reference's
    # to_dense_array loop, tensor/sparse.py:228-230, restricted to nonzeros).
    rng = np.random.default_rng(9)
    n = 400
    idx = rng.integers(0, 12, size=(n, 2)).astype(np.int32)
    vals = rng.standard_normal(n)
    vals[rng.random(n) < 0.2] = 0.0
    r = R.to_relation(idx, vals, (12, 12), (4, 3))
    want = np.zeros((12, 12))
    for (i, j), v in zip(idx, vals):
        if v != 0:
            want[i, j] = v
    npt.assert_array_equal(R.relation_to_dense(r), want)
    occupied = {(int(i) // 4, int(j) // 3) for (i, j), v in zip(idx, vals) if v != 0}
    npt.assert_array_equal(r.coords, np.array(sorted(occupied)))


# ---------------------------------------------------------------------------
# tile shapes and statistics (reference tests/test_sparse.py:135-214,
# tests/test_dense.py:77-112, tests/test_rigorous.py:367-400)

def test_all_tile_shapes():
    assert R.divisors(12) == [1, 2, 3, 4, 6, 12]
    assert len(R.all_tile_shapes((3, 4, 5))) == 12   # test_dense.py:41
    assert R.all_tile_shapes((3, 3)) == [(1, 1), (1, 3), (3, 1), (3, 3)]
    assert R.all_tile_shapes((1, 1)) == [(1, 1)]     # test_rigorous.py:370-374
    with pytest.raises(ValueError):
        R.divisors(0)


def metrics(data, shapes=None):
    idx, vals, shape = R.extract_coo(np.asarray(data, dtype=np.float64))
    return R.sparsity_metrics(idx, vals, shapes or R.all_tile_shapes(shape))


def test_sparsity_metrics_known_answers():
    m = metrics(np.array([[1.0, 0.0], [0.0, 2.0]]))
    assert m[(2, 2)][0] == 1
    m = metrics(np.diag([1.0, 2.0, 3.0]))
    assert m[(1, 1)][0] == 3
    m = metrics(np.diag([1.0, 2.0, 3.0, 4.0]))
    assert m[(2, 2)] == (2, (2, 2))
    d = np.zeros((4, 4))
    d[0, 0], d[0, 3], d[1, 1] = 1.0, 2.0, 3.0
    assert metrics(d)[(2, 2)] == (2, (1, 2))
    assert metrics(np.zeros((3, 3)))[(1, 1)] == (0, (0, 0))
    m = metrics(np.array([0.0, 1.0, 0.0, 3.0, 0.0, 0.0]))
    assert m[(1,)][0] == 2 and m[(2,)][0] == 2 and m[(3,)][0] == 2
    m = metrics(np.arange(1, 65).reshape(4, 4, 4).astype(float))
    assert m[(2, 2, 2)][0] == 8
    m = metrics(np.array([[1.0, 2, 0], [3.0, 4, 0], [5.0, 0, 0]]))
    assert {ts: (n, vc) for ts, (n, vc) in m.items()} == {
        (1, 1): (5, (3, 2)), (1, 3): (3, (3, 1)), (3, 1): (2, (1, 2)), (3, 3): (1, (1, 1))}
    d = np.zeros((100, 100))
    d[0, 0] = 1.0
    m = metrics(d, [(1, 1), (100, 100)])
    assert m[(1, 1)][0] == 1 and m[(100, 100)][0] == 1
    assert metrics(np.ones((4, 4)), [(1, 1)])[(1, 1)][0] == 16
    m = metrics(np.eye(4))
    assert (m[(1, 1)][0], m[(1, 4)][0], m[(4, 1)][0], m[(2, 2)][0]) == (4, 4, 4, 2)


def block_any(d, ts):
    """Occupancy grid of tile shape ts by reducing the dense blocks."""
    grid = tuple(n // t for n, t in zip(d.shape, ts))
    inter = []
    for g, t in zip(grid, ts):
        inter += [g, t]
    return (d.reshape(inter) != 0).any(axis=tuple(range(1, 2 * d.ndim, 2)))


@pytest.mark.parametrize("shape,p", [((12, 18), 0.05), ((8, 6, 10), 0.02), ((30,), 0.2),
                                     ((7, 4), 0.0)])
def test_sparsity_metrics_brute_force(shape, p):
    rng = np.random.default_rng(sum(shape))
    d = rng.standard_normal(shape) * (rng.random(shape) < p)
    m = metrics(d)
    for ts, (n, vc) in m.items():
        occ = block_any(d, ts)
        assert n == int(occ.sum()), ts
        for l in range(d.ndim):
            other = tuple(a for a in range(d.ndim) if a != l)
            assert vc[l] == int(occ.any(axis=other).sum()), (ts, l)
    assert m[(1,) * d.ndim][0] == np.count_nonzero(d)


# ---------------------------------------------------------------------------
# joins

def test_join_counts_reference_cases():
    # tests/test_sparse_dispatch.py:46-129
    A = np.zeros((4, 4)); A[0, 0] = 1.0; A[0, 2] = 2.0
    B = np.zeros((4, 4)); B[0, 0] = 3.0; B[2, 0] = 4.0
    li, _ = R.coordinate_join(rel(A, (2, 2)).coords, rel(B, (2, 2)).coords, [(1, 0)])
    assert len(li) == 2
    li, _ = R.coordinate_join(rel(np.eye(2), (1, 1)).coords, rel(np.eye(2), (1, 1)).coords, [])
    assert len(li) == 4
    A = np.zeros((4, 4)); A[0, 0] = 1.0; A[2, 0] = 2.0
    B = np.zeros((4, 4)); B[0, 0] = 3.0
    li, _ = R.coordinate_join(rel(A, (2, 2)).coords, rel(B, (2, 2)).coords, [(1, 0)])
    assert len(li) == 2
    # tests/test_pallas.py:235-338
    lc = np.array([[0, 0], [0, 1], [1, 0]], np.int32)
    rc = np.array([[0, 0], [1, 0]], np.int32)
    assert len(R.coordinate_join_hash(lc, rc, [(1, 0)])[0]) == 3
    assert len(R.coordinate_join_hash(np.array([[0], [1]]), np.array([[0], [1], [2]]), [])[0]) == 6
    assert len(R.coordinate_join_sorted(np.array([[0, 0], [1, 0]]), np.array([[0, 0], [0, 1]]),
                                        [(1, 0)])[0]) == 4
    e = np.zeros((0, 2), np.int32)
    assert len(R.coordinate_join_hash(e, e, [(1, 0)])[0]) == 0
    assert len(R.coordinate_join_sorted(e, e, [(1, 0)])[0]) == 0


def _brute(lc, rc, keys):
    return {(i, j) for i in range(len(lc)) for j in range(len(rc))
            if all(lc[i, a] == rc[j, b] for a, b in keys)}


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_join_match_set_brute_force(seed):
    rng = np.random.default_rng(seed)
    lc = rng.integers(0, 4, size=(40, 3)).astype(np.int32)
    rc = rng.integers(0, 4, size=(30, 3)).astype(np.int32)
    for keys in ([(1, 0)], [(0, 2), (2, 1)], [(0, 0), (1, 1), (2, 2)]):
        want = _brute(lc, rc, keys)
        for fn in (R.coordinate_join, R.coordinate_join_sorted):
            li, ri = fn(lc, rc, keys)
            assert set(zip(li.tolist(), ri.tolist())) == want
            assert len(li) == len(want)


def test_join_order_closed_forms():
    rng = np.random.default_rng(5)
    lc = rng.integers(0, 5, size=(60, 2)).astype(np.int32)
    rc = rng.integers(0, 5, size=(50, 2)).astype(np.int32)
    li, ri = R.coordinate_join(lc, rc, [(1, 0)])
    order = np.lexsort((li, ri))  # rhs major, lhs minor
    npt.assert_array_equal(order, np.arange(len(li)))
    sl, sr = R.coordinate_join_sorted(lc, rc, [(1, 0)])
    key = lc[sl, 1]
    lrank = np.argsort(np.lexsort((np.arange(60), lc[:, 1])))[sl]
    rrank = np.argsort(np.lexsort((np.arange(50), rc[:, 0])))[sr]
    npt.assert_array_equal(np.lexsort((rrank, lrank, key)), np.arange(len(sl)))


def test_join_order_golden_vectors():
    g = np.load(GOLDEN)
    for name in g["names"]:
        lc, rc = g[f"{name}__lhs"], g[f"{name}__rhs"]
        keys = [tuple(k) for k in g[f"{name}__keys"].tolist()]
        hl, hr = R.coordinate_join_hash(lc, rc, keys)
        npt.assert_array_equal(hl, g[f"{name}__hash_lhs"], err_msg=name)
        npt.assert_array_equal(hr, g[f"{name}__hash_rhs"], err_msg=name)
        cl, cr = R.coordinate_join(lc, rc, keys)
        npt.assert_array_equal(cl, g[f"{name}__hash_lhs"], err_msg=name)
        npt.assert_array_equal(cr, g[f"{name}__hash_rhs"], err_msg=name)
        sl, sr = R.coordinate_join_sorted(lc, rc, keys)
        npt.assert_array_equal(sl, g[f"{name}__sorted_lhs"], err_msg=name)
        npt.assert_array_equal(sr, g[f"{name}__sorted_rhs"], err_msg=name)


def test_golden_vectors_distinguish_orders():
    """The order checks have teeth: the two orders differ on the fixtures,
    so an implementation emitting the wrong one fails."""
    g = np.load(GOLDEN)
    differs = [n for n in g["names"]
               if not np.array_equal(g[f"{n}__hash_lhs"], g[f"{n}__sorted_lhs"])]
    assert len(differs) >= 4


# ---------------------------------------------------------------------------
# tile einsum (tests/test_sparse_dispatch.py:137-196)

def test_kernel_einsum_known_answers():
    lv = np.array([[[1.0, 0], [0, 1]], [[2.0, 0], [0, 2]]])
    rv = np.array([[[3.0, 0], [0, 3]], [[4.0, 0], [0, 4]]])
    out = R.kernel_einsum(lv, rv, np.array([0, 1]), np.array([0, 1]), "ij,jk->ik")
    npt.assert_allclose(out[0], 3 * np.eye(2), atol=1e-6)
    npt.assert_allclose(out[1], 8 * np.eye(2), atol=1e-6)
    out = R.kernel_einsum(np.array([[1.0, 2.0]]), np.array([[3.0, 4.0]]), [0], [0], "i,j->ij")
    npt.assert_allclose(out[0], [[3, 4], [6, 8]], atol=1e-6)
    out = R.kernel_einsum(np.array([[1.0, 2, 3]]), np.array([[4.0, 5, 6]]), [0], [0], "i,i->")
    assert out.shape == (1,) and abs(out[0] - 32.0) < 1e-6
    out = R.kernel_einsum(np.zeros((2, 3, 3)), np.zeros((2, 3, 3)), np.array([], np.int64),
                          np.array([], np.int64), "ij,jk->ik")
    assert out.shape == (0, 3, 3)


@pytest.mark.parametrize("spec,ls,rs", [
    ("ij,jk->ik", (5, 7), (7, 3)), ("bij,bjk->bik", (2, 4, 5), (2, 5, 3)),
    ("ijk,kl->ijl", (3, 4, 5), (5, 6)), ("ij,kj->ik", (4, 5), (3, 5)),
    ("ji,jk->ik", (5, 4), (5, 3)), ("ii,ij->j", (4, 4), (4, 3)), ("ij,ij->ij", (3, 4), (3, 4)),
])
def test_batched_einsum_matches_numpy(spec, ls, rs):
    rng = np.random.default_rng(1)
    L = rng.standard_normal((6, *ls))
    Rm = rng.standard_normal((6, *rs))
    npt.assert_allclose(R.batched_einsum(R.add_batch_dim(spec), L, Rm),
                        np.einsum(R.add_batch_dim(spec), L, Rm), rtol=1e-12, atol=1e-12)
    # a transposed operand gives a different answer (the check can fail)
    if spec == "ij,jk->ik":
        bad = np.einsum("zij,zkj->zik", L[:, :, :3], Rm[:, :3, :3])
        good = R.batched_einsum("zij,zjk->zik", L[:, :, :3], Rm[:, :3, :3])
        assert not np.allclose(bad, good)


def test_batch_dim_and_output_tile_shape():
    assert R.add_batch_dim("ij,jk->ik") == "zij,zjk->zik"
    assert R.add_batch_dim("i,j->ij") == "zi,zj->zij"
    assert R.add_batch_dim("i,i->") == "zi,zi->z"
    with pytest.raises(ValueError):
        R.add_batch_dim("ij,jk")
    assert R.infer_output_tile_shape("ij,jk->ik", (2, 3), (3, 4)) == (2, 4)
    assert R.infer_output_tile_shape("i,j->ij", (3,), (4,)) == (3, 4)
    assert R.infer_output_tile_shape("i,i->", (5,), (5,)) == ()
    assert R.infer_output_tile_shape("ii,ij->j", (3, 3), (3, 4)) == (4,)


def test_output_coords_known_answer():
    # tests/test_sparse_dispatch.py:474-501
    lc = np.array([[0, 0], [1, 0]], np.int32)
    rc = np.array([[0, 0], [0, 1]], np.int32)
    oc = R.compute_output_coords(lc, rc, np.array([0, 0, 1, 1]), np.array([0, 1, 0, 1]),
                                 [(0, 0), (1, 1)])
    assert oc.shape == (4, 2)
    npt.assert_array_equal(oc[0], [0, 0])
    npt.assert_array_equal(oc[1], [0, 1])
    assert R.compute_output_coords(lc, rc, [], [], [(0, 0), (1, 1)]).shape == (0, 2)


# ---------------------------------------------------------------------------
# segment sum (tests/test_sparse_dispatch.py:204-252)

def test_segment_sum_known_answers():
    v = np.array([[[1.0, 2.0], [3.0, 4.0]]])
    c, a = R.segment_sum(v, np.array([[0, 0]], np.int32))
    assert c.shape == (1, 2)
    npt.assert_allclose(a, v)
    v = np.array([[[1.0, 0], [0, 1]], [[2.0, 0], [0, 2]]])
    c, a = R.segment_sum(v, np.array([[0, 0], [0, 0]], np.int32))
    assert c.shape[0] == 1
    npt.assert_allclose(a[0], 3 * np.eye(2))
    c, a = R.segment_sum(np.array([[[1.0]], [[2.0]], [[3.0]]]),
                         np.array([[0, 0], [0, 0], [1, 0]], np.int32))
    assert c.shape[0] == 2 and a[0, 0, 0] == 3 and a[1, 0, 0] == 3
    c, a = R.segment_sum(np.array([[[1.0]], [[2.0]], [[3.0]]]),
                         np.array([[2, 0], [0, 0], [1, 0]], np.int32))
    assert np.all(c[:-1] <= c[1:])
    c, a = R.segment_sum(np.zeros((0, 2, 2)), np.zeros((0, 2), np.int32))
    assert c.shape[0] == 0 and a.shape[0] == 0


def test_segment_sum_and_plan_brute_force():
    rng = np.random.default_rng(11)
    oc = rng.integers(0, 5, size=(300, 2)).astype(np.int32)
    v = rng.standard_normal((300, 3, 2))
    c, a = R.segment_sum(v, oc)
    uc, perm, off, seg = R.segment_plan(oc)
    npt.assert_array_equal(c, uc)
    keys = sorted({tuple(x) for x in oc.tolist()})
    npt.assert_array_equal(uc, np.array(keys))
    for u, k in enumerate(keys):
        members = [i for i in range(300) if tuple(oc[i]) == k]
        npt.assert_array_equal(perm[off[u]:off[u + 1]], members)  # pair order inside
        npt.assert_allclose(a[u], v[members].sum(0), rtol=1e-12)
        assert np.all(seg[members] == u)


# ---------------------------------------------------------------------------
# end to end (tests/test_sparse_dispatch.py:263-426, tests/test_pallas.py:53-224)

def _dense_of(r):
    return R.relation_to_dense(r)


@pytest.mark.parametrize("case", ["identity", "diagonal", "tiled", "empty", "inferred"])
def test_execute_sparse_matmul_cases(case):
    if case == "identity":
        A, B, t = np.array([[1.0, 2], [3, 4]]), np.eye(2), (1, 1)
    elif case == "diagonal":
        A, B, t = np.diag([1.0, 2, 3, 4]), np.diag([5.0, 6, 7, 8]), (1, 1)
    elif case == "tiled":
        A = np.array([[1.0, 2, 0, 0], [3, 4, 0, 0], [0, 0, 5, 6], [0, 0, 7, 8]])
        B, t = np.eye(4), (2, 2)
    elif case == "empty":
        A = np.zeros((4, 4)); A[0, 0] = 1
        B = np.zeros((4, 4)); B[2, 2] = 1
        t = (2, 2)
    else:
        A, B, t = np.diag([1.0, 2]), np.diag([3.0, 4]), (1, 1)
    kw = {} if case == "inferred" else dict(output_shape=A.shape[:1] + B.shape[1:],
                                            output_tile_shape=t)
    out = R.execute_sparse(rel(A, t), rel(B, t), [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], **kw)
    npt.assert_allclose(_dense_of(out), A @ B, atol=1e-6)
    bs = R.block_sparse_matmul_generic(rel(A, t), rel(B, t))
    npt.assert_allclose(_dense_of(bs), A @ B, atol=1e-6)


def test_execute_sparse_outer_and_elementwise():
    a = np.array([1.0, 0, 3])
    b = np.array([0.0, 2, 4])
    out = R.execute_sparse(rel(a.reshape(3, 1), (1, 1)), rel(b.reshape(1, 3), (1, 1)), [],
                           "ij,kl->ij", [(0, 0), (1, 1)], (3, 3), (1, 1))
    npt.assert_allclose(_dense_of(out), np.outer(a, b), atol=1e-6)
    A, B = np.diag([1.0, 2, 3]), np.diag([4.0, 5, 6])
    out = R.execute_sparse(rel(A, (1, 1)), rel(B, (1, 1)), [(0, 0), (1, 1)], "ij,ij->ij",
                           [(0, 0), (0, 1)], (3, 3), (1, 1))
    npt.assert_allclose(_dense_of(out), A * B, atol=1e-6)


def test_block_sparse_matmul_raw_and_validation():
    A = np.array([[1.0, 0, 2, 0], [0, 3, 0, 4], [5, 0, 6, 0]])
    B = np.array([[1.0, 0], [0, 2], [3, 0], [0, 4]])
    la, rb = rel(A, (1, 1)), rel(B, (1, 1))
    out = R.block_sparse_matmul(la.coords, la.values, rb.coords, rb.values, (1, 1, 1), A.shape,
                                B.shape)
    npt.assert_allclose(_dense_of(out), A @ B, atol=1e-6)
    bad = R.Rel(np.array([[0, 0, 0]], np.int32), np.ones((1, 1, 1, 1)), (1, 1, 1), (1, 1, 1))
    with pytest.raises(ValueError):
        R.block_sparse_matmul_generic(la, bad)


def test_random_blocksparse_end_to_end_fp64():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((64, 96)) * np.kron(rng.random((8, 6)) < 0.3, np.ones((8, 16)))
    B = rng.standard_normal((96, 40)) * np.kron(rng.random((6, 5)) < 0.5, np.ones((16, 8)))
    out = R.execute_sparse(rel(A, (8, 16)), rel(B, (16, 8)), [(1, 0)], "ij,jk->ik",
                           [(0, 0), (1, 1)], precision="fp64")
    npt.assert_allclose(_dense_of(out), A @ B, rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------------------
# bf16 rounding against torch's conversion

def test_bf16_round_matches_torch():
    import torch

    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32),
                        np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, 0.0, 65504.0,
                                  1e-40, np.inf, -np.inf], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    npt.assert_array_equal(R.bf16_round(x), want)
    npt.assert_array_equal(R.bf16_from_bits(R.bf16_bits(want)), want)


# ---------------------------------------------------------------------------
# workload generators: sizes fixed by the generation protocol

@pytest.mark.parametrize("name,n_l,n_r,P", [
    ("blocksparse_1k", 102, 1024, 3264),
    ("blocksparse_16k_bf16", 819, 4096, 26208),
    ("order3", 1311, 1024, 20976),
])
def test_generator_sizes(name, n_l, n_r, P):
    w = G.WORKLOADS[name]()
    assert w["lhs"].coords.shape[0] == n_l and w["rhs"].coords.shape[0] == n_r
    li, ri = R.coordinate_join(w["lhs"].coords, w["rhs"].coords, w["join_keys"])
    assert len(li) == P
    c = w["lhs"].coords
    assert np.all(np.diff(np.ravel_multi_index(c.T, [s // t for s, t in zip(
        w["lhs"].shape, w["lhs"].tile_shape)])) > 0)  # lexicographic, distinct


# ---------------------------------------------------------------------------
# backward (reference autodiff/custom_vjp.py:31-62, :254-275;
# tests/test_autodiff.py)

def test_reverse_einsum_string_known_answers():
    assert R.reverse_einsum_string("ij,jk->ik") == ("ik,jk->ij", "ij,ik->jk")
    assert R.reverse_einsum_string("i,j->ij") == ("ij,j->i", "i,ij->j")
    assert R.reverse_einsum_string("i,i->") == (",i->i", "i,->i")
    assert R.reverse_einsum_string("bij,bjk->bik") == ("bik,bjk->bij", "bij,bik->bjk")
    with pytest.raises(ValueError):
        R.reverse_einsum_string("ij,jk")


def test_pair_einsum_vjp_known_answers():
    # tests/test_autodiff.py:160-224: loss = sum(A @ B) with one 2x2 tile each:
    # dL/dA = ones @ B^T, dL/dB = A^T @ ones.
    A = np.array([[1.0, 2.0], [3.0, 4.0]])
    B = np.array([[5.0, 6.0], [7.0, 8.0]])
    g = np.ones((1, 2, 2))
    gl, gr = R.pair_einsum_vjp(A[None], B[None], [0], [0], "ij,jk->ik", g)
    npt.assert_array_equal(gl[0], np.ones((2, 2)) @ B.T)
    npt.assert_array_equal(gr[0], A.T @ np.ones((2, 2)))
    # :335-373: an lhs tile matched twice accumulates both partners' terms.
    A = np.zeros((4, 4)); A[0, 0], A[0, 2] = 1.0, 2.0
    B = np.zeros((4, 4)); B[0, 0], B[2, 0] = 3.0, 4.0
    lhs, rhs = R.dense_to_relation(A, (2, 2)), R.dense_to_relation(B, (2, 2))
    li, ri = R.coordinate_join(lhs.coords, rhs.coords, [(1, 0)])
    P = len(li)
    gl, _ = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik", np.ones((P, 2, 2)))
    want = np.zeros_like(lhs.values)
    for p in range(P):
        want[li[p]] += np.ones((2, 2)) @ rhs.values[ri[p]].T
    npt.assert_array_equal(gl, want)
    # :441-476 outer product "ij,kl->ijkl", (1, 1) tiles: dL/da = sum of b
    a, b = np.array([[[1.0]], [[2.0]]]), np.array([[[3.0]], [[4.0]]])
    li, ri = np.repeat(np.arange(2), 2), np.tile(np.arange(2), 2)
    gl, gr = R.pair_einsum_vjp(a, b, li, ri, "ij,kl->ijkl", np.ones((4, 1, 1, 1, 1)))
    npt.assert_array_equal(gl.reshape(-1), [7.0, 7.0])
    npt.assert_array_equal(gr.reshape(-1), [3.0, 3.0])


@pytest.mark.parametrize("spec,lt,rt", [("ij,jk->ik", (3, 4), (4, 2)),
                                        ("ij,kj->ik", (2, 3), (4, 3)),
                                        ("bij,bjk->bik", (1, 2, 3), (1, 3, 2)),
                                        ("ij,kl->ijkl", (2, 1), (1, 2)),
                                        ("i,i->", (5,), (5,)),
                                        ("ij,ij->ij", (2, 3), (2, 3)),
                                        ("ijk,kl->ijl", (2, 2, 3), (3, 2))])
def test_pair_einsum_vjp_finite_differences(spec, lt, rt):
    """f(L, R) = sum_p <W_p, out_p> is linear in each operand, so central
    differences in float64 give its gradient up to rounding."""
    rng = np.random.default_rng(len(spec))
    nl, nr, P = 4, 3, 9
    L, Rv = rng.standard_normal((nl, *lt)), rng.standard_normal((nr, *rt))
    li, ri = rng.integers(0, nl, P), rng.integers(0, nr, P)
    li[0] = li[1]  # a tile in several pairs
    out_shape = R.kernel_einsum(L, Rv, li, ri, spec, precision="fp64").shape
    W = rng.standard_normal(out_shape)

    def f(L_, R_):
        return float(np.sum(W * R.kernel_einsum(L_, R_, li, ri, spec, precision="fp64")))

    gl, gr = R.pair_einsum_vjp(L, Rv, li, ri, spec, W)
    eps = 1e-3
    for X, G, which in ((L, gl, 0), (Rv, gr, 1)):
        fd = np.zeros_like(X)
        for idx in np.ndindex(*X.shape):
            Xp, Xm = X.copy(), X.copy()
            Xp[idx] += eps
            Xm[idx] -= eps
            fp = f(Xp, Rv) if which == 0 else f(L, Xp)
            fm = f(Xm, Rv) if which == 0 else f(L, Xm)
            fd[idx] = (fp - fm) / (2 * eps)
        npt.assert_allclose(G, fd, rtol=1e-9, atol=1e-9)
    # tiles in no pair get zero gradient
    unused = np.setdiff1d(np.arange(nl), li)
    assert np.all(gl[unused] == 0)


# ---------------------------------------------------------------------------
# kernel_einsum with the reference's dtypes (jnp.array / jnp.einsum with 64-bit
# types off, sparse_dispatch.py:125) and segment_sum in the values' dtype

def test_kernel_einsum_typed_reference_single_pair():
    # tests/test_rigorous.py:938-945: float64 identity with an int64 tile
    lhs = np.eye(2).reshape(1, 2, 2)
    rhs = np.array([[[1, 2], [3, 4]]])
    out = R.kernel_einsum_typed(lhs, rhs, np.array([0]), np.array([0]), "ij,jk->ik")
    assert out.dtype == np.float32
    npt.assert_array_equal(out[0], [[1, 2], [3, 4]])


@pytest.mark.parametrize("a,b,want", [
    (np.int64, np.int64, np.int32), (np.int8, np.int8, np.int8), (np.uint8, np.int8, np.int16),
    (np.int32, np.float64, np.float32), (np.uint32, np.int32, np.int32),
    (np.bool_, np.bool_, np.bool_), (np.bool_, np.int8, np.int8), (np.float16, np.int8, np.float16),
    (np.float16, np.float32, np.float32), (np.uint64, np.uint8, np.uint32),
    (np.float64, np.float64, np.float32)])
def test_jnp_einsum_dtype_table(a, b, want):
    # JAX's promotion lattice with 64-bit types canonicalised to 32 bits
    assert R.jnp_einsum_dtype(a, b) == np.dtype(want)


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.int8, np.uint32])
def test_kernel_einsum_typed_wraps_like_fixed_width_ints(dt):
    # brute force in Python integers, reduced mod 2^bits of the result type
    rng = np.random.default_rng(3)
    info = np.iinfo(dt)
    lo, hi = max(info.min, -2 ** 31), min(info.max, 2 ** 31 - 1)
    L = rng.integers(lo, hi, size=(3, 3, 4), endpoint=True).astype(dt)
    Rt = rng.integers(lo, hi, size=(2, 4, 2), endpoint=True).astype(dt)
    li, ri = np.array([0, 2, 1]), np.array([1, 0, 1])
    out = R.kernel_einsum_typed(L, Rt, li, ri, "ij,jk->ik")
    res = R.jnp_einsum_dtype(dt, dt)
    assert out.dtype == res
    bits = np.iinfo(res).bits
    for p in range(3):
        a = [[int(x) for x in row] for row in L[li[p]]]
        b = [[int(x) for x in row] for row in Rt[ri[p]]]
        if dt in (np.int64, np.uint64):  # jnp.array truncates 64-bit ints to 32 bits first
            a = [[x % 2 ** 32 - (2 ** 32 if dt == np.int64 and x % 2 ** 32 >= 2 ** 31 else 0)
                  for x in row] for row in a]
            b = [[x % 2 ** 32 - (2 ** 32 if dt == np.int64 and x % 2 ** 32 >= 2 ** 31 else 0)
                  for x in row] for row in b]
        for i in range(3):
            for k in range(2):
                v = sum(a[i][j] * b[j][k] for j in range(4)) % 2 ** bits
                got = int(out[p, i, k]) % 2 ** bits
                assert got == v


def test_kernel_einsum_typed_bool_is_or_of_and():
    rng = np.random.default_rng(4)
    L = rng.random((2, 3, 5)) < 0.3
    Rt = rng.random((2, 5, 4)) < 0.3
    out = R.kernel_einsum_typed(L, Rt, np.array([0, 1]), np.array([1, 0]), "ij,jk->ik")
    assert out.dtype == np.bool_
    for p, (a, b) in enumerate(((0, 1), (1, 0))):
        want = [[any(L[a, i, j] and Rt[b, j, k] for j in range(5)) for k in range(4)]
                for i in range(3)]
        npt.assert_array_equal(out[p], want)


def test_segment_sum_keeps_integer_dtype_and_wraps():
    # tests/test_rigorous.py:958-963 (ints, single entry) and wrapping as numpy adds int8
    coords, agg = R.segment_sum(np.array([[[1, 2], [3, 4]]]), np.array([[0, 0]]))
    assert agg.dtype == np.array([1]).dtype
    npt.assert_array_equal(agg[0], [[1, 2], [3, 4]])
    v = np.array([[100], [100], [-7]], dtype=np.int8)
    _, agg = R.segment_sum(v, np.array([[0], [0], [1]]))
    assert agg.dtype == np.int8
    npt.assert_array_equal(agg[:, 0], [np.int8(-56), -7])  # 200 mod 256 = -56
