"""GPU parity of relation construction: COO ingest, COO tiling and the
per-tile-shape statistics, against the oracle.

Indices, tile coordinates and statistics must be bit-exact; tile values are
the oracle's float64 values rounded to the tile dtype, bit for bit.
"""

from math import prod

import numpy as np
import numpy.testing as npt
import pytest
import scipy.sparse as sp
import torch

from oracle import generators as G
from oracle import reference_path as R

from einjax_amd import SparseTensor, SparseTensorRelation
from einjax_amd import _device as D

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


def sparse_array(rng, shape, p):
    d = rng.standard_normal(shape) * (rng.random(shape) < p)
    return d


def to_device(d64: np.ndarray, dtype: str) -> tuple[torch.Tensor, np.ndarray]:
    """Device tensor of the given dtype and the float64 values it holds."""
    if dtype == "f64":
        return torch.from_numpy(d64).cuda(), d64
    f = d64.astype(np.float32)
    if dtype == "bf16":
        f = R.bf16_round(f)
        return torch.from_numpy(f).cuda().to(torch.bfloat16), f.astype(np.float64)
    return torch.from_numpy(f).cuda(), f.astype(np.float64)


def stats_dict(tile_shapes, nt, vc):
    return {ts: (n, v) for ts, n, v in zip(tile_shapes, nt, vc)}


# ---------------------------------------------------------------------------
# dense -> COO (reference: _extract_coo, tensor/sparse.py:234-270)

@pytest.mark.parametrize("dtype", ["f64", "f32", "bf16"])
@pytest.mark.parametrize("shape,p", [((64, 96), 0.1), ((5, 7, 33), 0.3), ((1001,), 0.5),
                                     ((3, 2, 4, 2, 5), 0.9), ((16, 16), 0.0)])
def test_extract_coo_parity(gpu, dtype, shape, p):
    note("extract_coo", dtype, shape, p)
    rng = np.random.default_rng(prod(shape))
    d = sparse_array(rng, shape, p)
    if d.size > 10:
        d.flat[7] = np.nan   # nonzero
        d.flat[9] = -0.0     # zero
    t, d64 = to_device(d, dtype)
    idx, vals = D.extract_coo(t)
    want_idx, want_vals, _ = R.extract_coo(d64)
    npt.assert_array_equal(idx.cpu().numpy(), want_idx)
    assert idx.dtype == torch.int32 and vals.dtype == torch.float64
    npt.assert_array_equal(vals.cpu().numpy(), want_vals)  # NaN == NaN here
    assert D.count_nonzero(t) == len(want_vals)


def test_extract_coo_unaligned_and_public_api(gpu):
    note("extract_coo unaligned")
    rng = np.random.default_rng(2)
    base = torch.from_numpy(sparse_array(rng, (4097,), 0.4).astype(np.float32)).cuda()
    t = base[1:]  # 4-byte offset: the 16-byte vector loads are off
    assert t.data_ptr() % 16 != 0
    idx, vals = D.extract_coo(t)
    want_idx, want_vals, _ = R.extract_coo(t.cpu().numpy().astype(np.float64))
    npt.assert_array_equal(idx.cpu().numpy(), want_idx)
    npt.assert_array_equal(vals.cpu().numpy(), want_vals)
    # the module-level _extract_coo answers in the input's residency
    from einjax_amd.tensor.sparse import _extract_coo

    d = np.array([[1.0, 0.0], [0.0, 2.0]])
    hi, hv, hs = _extract_coo(d)
    assert isinstance(hi, np.ndarray) and hi.dtype == np.int32 and hs == (2, 2)
    npt.assert_array_equal(hi, [[0, 0], [1, 1]])
    npt.assert_array_equal(hv, [1.0, 2.0])
    di, dv, _ = _extract_coo(torch.from_numpy(d).cuda())
    assert di.is_cuda and dv.is_cuda
    t = SparseTensor("s", np.diag([1.0, 2.0, 3.0]))
    assert t.nnz == 3
    npt.assert_array_equal(t._indices, [[0, 0], [1, 1], [2, 2]])
    npt.assert_array_equal(t._values, [1.0, 2.0, 3.0])


# ---------------------------------------------------------------------------
# COO -> tiles (reference: to_relation, tensor/sparse.py:160-219)

@pytest.mark.parametrize("dtype", ["f64", "f32", "bf16"])
@pytest.mark.parametrize("shape,tile,n", [((48, 60), (8, 12), 700), ((12, 10, 16), (3, 5, 4), 900),
                                          ((96,), (16,), 50), ((64, 64), (64, 64), 30),
                                          ((20, 30), (1, 1), 300)])
def test_bucket_coo_parity(gpu, dtype, shape, tile, n):
    note("bucket_coo", dtype, shape, tile, n)
    rng = np.random.default_rng(n + len(shape))
    idx = np.stack([rng.integers(0, s, size=n) for s in shape], axis=1).astype(np.int32)
    vals = rng.standard_normal(n)
    vals[rng.random(n) < 0.15] = 0.0          # explicit zeros are dropped
    k = min(20, n // 4)
    idx[n // 2:n // 2 + k] = idx[:k]          # repeated elements: the last nonzero wins
    vals[3] = np.nan
    vals[5] = -0.0
    vals[7] = 1e-300                          # kept by float64 tiles only
    if dtype == "f64":
        v64 = vals
        tv = torch.from_numpy(vals).cuda()
    else:
        f = vals.astype(np.float32)
        if dtype == "bf16":
            f = R.bf16_round(f)
        v64 = f.astype(np.float64)
        tv = torch.from_numpy(f).cuda()
        if dtype == "bf16":
            tv = tv.to(torch.bfloat16)
    coords, tiles = D.bucket_coo(torch.from_numpy(idx).cuda(), tv, shape, tile)
    want = R.to_relation(idx, v64, shape, tile)
    npt.assert_array_equal(coords.cpu().numpy(), want.coords)
    if dtype == "f64":  # float64 tiles, bit-exact: the reference's dtype
        got = tiles.cpu().numpy()
        npt.assert_array_equal(got, want.values)
    else:
        got = tiles.float().cpu().numpy()
        npt.assert_array_equal(got, want.values.astype(np.float32))
    assert not np.any(np.signbit(got[got == 0]))
    assert tiles.dtype == {"f64": torch.float64, "f32": torch.float32,
                           "bf16": torch.bfloat16}[dtype]


def test_bucket_coo_sorted_input_and_errors(gpu):
    note("bucket_coo edges")
    # one entry, entries all zero, index out of range
    idx = torch.tensor([[3, 5]], dtype=torch.int32).cuda()
    c, t = D.bucket_coo(idx, torch.tensor([2.5], dtype=torch.float64).cuda(), (8, 8), (4, 4))
    npt.assert_array_equal(c.cpu().numpy(), [[0, 1]])
    assert t[0, 3, 1].item() == 2.5 and t.abs().sum().item() == 2.5
    c, t = D.bucket_coo(idx, torch.zeros(1, dtype=torch.float64).cuda(), (8, 8), (4, 4))
    assert c.shape == (0, 2) and t.shape == (0, 4, 4)
    bad = torch.tensor([[3, 8]], dtype=torch.int32).cuda()
    with pytest.raises(ValueError):
        D.bucket_coo(bad, torch.ones(1, dtype=torch.float64).cuda(), (8, 8), (4, 4))
    # a zero entry outside the shape is dropped like every zero entry
    c, t = D.bucket_coo(bad, torch.zeros(1, dtype=torch.float64).cuda(), (8, 8), (4, 4))
    assert c.shape == (0, 2)


def test_scipy_to_relation_without_densifying(gpu):
    note("scipy to_relation")
    rng = np.random.default_rng(11)
    m = sp.random(300, 420, density=0.01, random_state=12, format="coo")
    # a repeated entry and an explicit zero, which scipy keeps in COO form
    row = np.concatenate([m.row, m.row[:5], [7]])
    col = np.concatenate([m.col, m.col[:5], [9]])
    data = np.concatenate([m.data, rng.standard_normal(5), [0.0]])
    coo = sp.coo_matrix((data, (row, col)), shape=(300, 420))
    for mat in (coo, sp.csr_matrix(sp.random(64, 48, density=0.05, random_state=3))):
        t = SparseTensor("m", mat)
        want_idx, want_vals, shape = R.extract_coo(mat)
        assert t.nnz == len(want_vals) and t.shape == shape
        rel = t.to_relation((4, 6) if shape == (64, 48) else (10, 20))
        want = R.to_relation(want_idx, want_vals, shape, rel.tile_shape)
        assert isinstance(rel.coords, np.ndarray)
        npt.assert_array_equal(rel.coords, want.coords)
        assert rel.values.dtype == np.float64
        npt.assert_array_equal(rel.values, want.values)
        npt.assert_array_equal(t.to_dense_array(), R.relation_to_dense(want))


# ---------------------------------------------------------------------------
# statistics (reference: _compute_sparsity_metrics, tensor/sparse.py:124-158)

# (3, 65536): last-dimension chains of 16 power-of-two levels, longer than one
# counting pass; (4, 96, 32): chains from every (a, b, 1) map and odd factors;
# (64, 16384), (4, 16, 16384), (8, 32768), (6, 16384): map rows of whole
# 16384-bit chunks, so runs of row poolings are banded (one and two chunks per
# row, a leading dimension with its own pools, a row count with a factor 3);
# (8, 64, 2048), (2, 32, 512), (64, 256): rows of 2048, 512 and 256 bits,
# banded inside a chunk.
STAT_SHAPES = [((12, 18), 0.05), ((8, 6, 10), 0.02), ((30,), 0.2), ((7, 4), 0.3),
               ((64, 48), 0.002), ((2, 3, 4, 5), 0.1), ((16, 16), 0.0), ((1, 1), 1.0),
               ((3, 65536), 0.0005), ((4, 96, 32), 0.01), ((64, 16384), 0.0005),
               ((4, 16, 16384), 0.0003), ((8, 32768), 0.0002), ((6, 16384), 0.001),
               ((8, 64, 2048), 0.0003), ((2, 32, 512), 0.002), ((64, 256), 0.01)]


@pytest.mark.parametrize("dtype", ["f64", "f32", "bf16"])
@pytest.mark.parametrize("shape,p", STAT_SHAPES)
def test_scheme_stats_dense_parity(gpu, dtype, shape, p):
    note("stats dense", dtype, shape, p)
    rng = np.random.default_rng(7 * prod(shape))
    d = sparse_array(rng, shape, p)
    t, d64 = to_device(d, dtype)
    shapes = R.all_tile_shapes(shape)
    nt, vc = D.scheme_stats(shapes, shape, dense=t)
    idx, vals, _ = R.extract_coo(d64)
    assert stats_dict(shapes, nt, vc) == R.sparsity_metrics(idx, vals, shapes)


@pytest.mark.parametrize("cap", [0, 40, 8, 1])
@pytest.mark.parametrize("shape,n", [((12, 18), 40), ((8, 6, 10), 60), ((30,), 9),
                                     ((64, 48), 500), ((131072,), 300)])
def test_scheme_stats_coo_parity(gpu, cap, shape, n):
    """bitmap_cap moves tile shapes between the map path and the sort path;
    the counts must not change."""
    note("stats coo", cap, shape, n)
    rng = np.random.default_rng(n)
    idx = np.stack([rng.integers(0, s, size=n) for s in shape], axis=1).astype(np.int32)
    vals = rng.standard_normal(n)
    vals[rng.random(n) < 0.2] = 0.0
    idx[-5:] = idx[:5]
    shapes = R.all_tile_shapes(shape)
    nt, vc = D.scheme_stats(shapes, shape, indices=torch.from_numpy(idx).cuda(),
                            values=torch.from_numpy(vals).cuda(), bitmap_cap=cap)
    assert stats_dict(shapes, nt, vc) == R.sparsity_metrics(idx, vals, shapes)


def test_scheme_stats_subset_and_range_error(gpu):
    note("stats subset")
    rng = np.random.default_rng(1)
    d = sparse_array(rng, (24, 36), 0.05)
    shapes = [(24, 1), (3, 4), (1, 36), (8, 9)]  # any subset, any order
    nt, vc = D.scheme_stats(shapes, (24, 36), dense=torch.from_numpy(d).cuda())
    idx, vals, _ = R.extract_coo(d)
    assert stats_dict(shapes, nt, vc) == R.sparsity_metrics(idx, vals, shapes)
    bad = torch.tensor([[1, 36]], dtype=torch.int32).cuda()
    with pytest.raises(ValueError):
        D.scheme_stats([(1, 1)], (24, 36), indices=bad,
                       values=torch.ones(1, dtype=torch.float64).cuda())


def test_sparse_tensor_schemes_known_answers(gpu):
    """The reference's own expectations (tests/test_sparse.py:135-214,
    tests/test_dense.py:77-112, tests/test_rigorous.py:367-400), through
    SparseTensor.schemes on the GPU."""
    note("schemes known answers")
    assert SparseTensor("s", np.array([[1.0, 0.0], [0.0, 2.0]])).schemes[(2, 2)].num_tuples == 1
    assert SparseTensor("s", np.diag([1.0, 2.0, 3.0])).schemes[(1, 1)].num_tuples == 3
    s = SparseTensor("d", np.diag([1.0, 2.0, 3.0, 4.0])).schemes[(2, 2)]
    assert (s.num_tuples, s.value_count) == (2, (2, 2))
    d = np.zeros((4, 4))
    d[0, 0], d[0, 3], d[1, 1] = 1.0, 2.0, 3.0
    s = SparseTensor("r", d).schemes[(2, 2)]
    assert (s.num_tuples, s.value_count) == (2, (1, 2))
    assert SparseTensor("z", np.zeros((3, 3))).schemes[(1, 1)].num_tuples == 0
    v = SparseTensor("v", np.array([0.0, 1.0, 0.0, 3.0, 0.0, 0.0])).schemes
    assert (v[(1,)].num_tuples, v[(2,)].num_tuples, v[(3,)].num_tuples) == (2, 2, 2)
    a = SparseTensor("a", np.arange(1, 65).reshape(4, 4, 4).astype(float))
    assert a.schemes[(2, 2, 2)].num_tuples == 8
    m = SparseTensor("a", np.array([[1.0, 2, 0], [3.0, 4, 0], [5.0, 0, 0]])).schemes
    assert len(m) == 4
    got = {ts: (s.num_tuples, s.value_count) for ts, s in m.items()}
    assert got == {(1, 1): (5, (3, 2)), (1, 3): (3, (3, 1)), (3, 1): (2, (1, 2)),
                   (3, 3): (1, (1, 1))}
    d = np.zeros((100, 100))
    d[0, 0] = 1.0
    big = SparseTensor("t", d).schemes
    assert big[(1, 1)].num_tuples == 1 and big[(100, 100)].num_tuples == 1
    assert SparseTensor("t", np.ones((4, 4))).schemes[(1, 1)].num_tuples == 16
    e = SparseTensor("t", np.eye(4)).schemes
    assert [e[ts].num_tuples for ts in [(1, 1), (1, 4), (4, 1), (2, 2)]] == [4, 4, 4, 2]
    c = SparseTensor("c", sp.csr_matrix(np.eye(4)))
    assert c.nnz == 4 and c.schemes[(2, 2)].num_tuples == 2


def blocksparse_closed_form(coords, block, ts):
    """Statistics of a block-sparse tensor whose chosen blocks are entirely
    nonzero, for tile extents that divide or are multiples of the block."""
    nd = coords.shape[1]
    coarse = np.array([max(1, t // block[d]) for d, t in enumerate(ts)])
    per = [block[d] // t if t < block[d] else 1 for d, t in enumerate(ts)]
    cc = coords // coarse
    n = len(np.unique(cc, axis=0)) * prod(per)
    vc = tuple(len(np.unique(cc[:, d])) * per[d] for d in range(nd))
    return n, vc


def test_scheme_stats_blocksparse_16k_all_tile_shapes(gpu):
    """The 16384 x 16384 bf16 operand with 5% of its 128 x 128 tiles nonzero,
    all 225 tile shapes, against the closed form of a block-sparse tensor;
    nnz and the COO of the same tensor against the tile list."""
    w = G.workload_blocksparse_16k(values=False)
    coords = w["lhs"].coords
    note("stats blocksparse 16k", len(coords), "tiles")
    tiles = torch.rand((len(coords), 128, 128), device="cuda", dtype=torch.float32) + 0.5
    rel = SparseTensorRelation(torch.from_numpy(coords).cuda(), tiles.to(torch.bfloat16),
                               (16384, 16384), (128, 128))
    dense = rel.to_dense()
    shapes = R.all_tile_shapes((16384, 16384))
    assert len(shapes) == 225
    nt, vc = D.scheme_stats(shapes, (16384, 16384), dense=dense)
    for ts, n, v in zip(shapes, nt, vc):
        assert (n, v) == blocksparse_closed_form(coords, (128, 128), ts), ts
    assert D.count_nonzero(dense) == len(coords) * 128 * 128
    # the dense -> COO -> tiles path gives back the tile list
    idx, vals = D.extract_coo(dense)
    assert idx.shape == (len(coords) * 16384, 2)
    c2, t2 = D.bucket_coo(idx, vals, (16384, 16384), (128, 128))
    npt.assert_array_equal(c2.cpu().numpy(), coords)
    assert torch.equal(t2, tiles.to(torch.bfloat16).float())


def test_scheme_stats_order3_all_tile_shapes(gpu):
    """The 2048^3 fp32 order-3 operand with 0.5% of its 32^3 tiles nonzero
    (34.4 GB dense), all 1,728 tile shapes (every extent a power of two, so
    each divides or is a multiple of 32), against the closed form of a
    block-sparse tensor: the map, pooling and banded counting kernels at
    their full size."""
    w = G.workload_order3(values=False)
    coords = w["lhs"].coords
    note("stats order-3 2048^3", len(coords), "tiles")
    tiles = torch.rand((len(coords), 32, 32, 32), device="cuda", dtype=torch.float32) + 0.5
    rel = SparseTensorRelation(torch.from_numpy(coords).cuda(), tiles, (2048, 2048, 2048),
                               (32, 32, 32))
    dense = rel.to_dense()
    del tiles, rel
    shapes = R.all_tile_shapes((2048, 2048, 2048))
    assert len(shapes) == 1728
    nt, vc = D.scheme_stats(shapes, (2048, 2048, 2048), dense=dense)
    for ts, n, v in zip(shapes, nt, vc):
        assert (n, v) == blocksparse_closed_form(coords, (32, 32, 32), ts), ts
    assert D.count_nonzero(dense) == len(coords) * 32 ** 3
    del dense
    torch.cuda.empty_cache()
