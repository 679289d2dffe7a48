"""Tile-shape selection over statistics counted on the GPU, registry
dispatch onto the GPU kernels and the api's relation einsum.

The reference's tests/test_tiling.py cases run through SparseTensor /
DenseTensor.schemes (GPU statistics) and must give the reference's answers;
on random tensors the product's ranking and selection must equal the
oracle's (oracle/selection.py over the oracle's sparsity_metrics).
"""

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R
from oracle import selection as S

import einjax_amd as ej
from einjax_amd import DenseTensor, SparseTensor, SparseTensorRelation

pytestmark = pytest.mark.gpu

DIAG = np.diag([1.0, 2.0, 3.0, 4.0])


def note(*a):
    print("[case]", *a, flush=True)


def test_tiling_reference_cases_gpu_stats(gpu):
    """tests/test_tiling.py:33-160, :270-510 with the statistics of
    SparseTensor / DenseTensor counted on the GPU."""
    note("tiling reference cases")
    t = SparseTensor("s", DIAG)
    assert len(ej.prune_infeasible_schemes(t.schemes, num_devices=1)) == len(t.schemes)
    pruned = ej.prune_infeasible_schemes(t.schemes, num_devices=1, max_tile_bytes=4, dtype_size=4)
    assert pruned and all(s.tile_size == 1 for s in pruned.values())
    assert len(ej.prune_infeasible_schemes(t.schemes, 1, max_tile_bytes=1_000_000)) == 9
    assert len(ej.prune_infeasible_schemes(t.schemes, 1, max_tile_bytes=0)) == 0
    ranked = ej.rank_schemes_by_sparsity(t.schemes, t.shape)
    first = ej.sparsity_ratio(ranked[0].num_tuples, t.shape, ranked[0].tile_shape)
    assert all(ej.sparsity_ratio(s.num_tuples, t.shape, s.tile_shape) >= first
               for s in ranked[1:])
    assert ranked[0].tile_shape == (1, 1)
    assert len(ej.rank_schemes_by_sparsity(SparseTensor("s", np.diag([1.0, 2.0])).schemes,
                                           (2, 2))) == 4
    best = ej.select_best_sparse_tiling(t.schemes, t.shape)
    assert isinstance(best, ej.TilingScheme) and best.tile_shape == (1, 1)
    assert ej.select_best_sparse_tiling(t.schemes, t.shape, max_tile_bytes=0) is None
    best = ej.select_best_sparse_tiling(t.schemes, t.shape, max_tile_bytes=16, dtype_size=4)
    assert best is not None and best.tile_size * 4 <= 16
    assert ej.prepare_sparse_tiling(t).tile_shape == (1, 1)
    best = ej.prepare_sparse_tiling(t, max_tile_bytes=4, dtype_size=4)
    assert best is not None and best.tile_size * 4 <= 4
    assert ej.prepare_sparse_tiling(SparseTensor("v", np.array([0.0, 1, 0, 3, 0, 0]))) is not None
    d = DenseTensor("d", np.ones((4, 4)))
    ranked = ej.rank_schemes_by_sparsity(d.schemes, d.shape)
    assert all(a.tile_size >= b.tile_size for a, b in zip(ranked, ranked[1:]))
    assert ej.prepare_sparse_tiling(d).tile_shape == (4, 4)
    d8 = DenseTensor("d", np.ones((8, 8)))
    assert len(ej.filter_schemes_by_device_count(d8.schemes, 1)) == len(d8.schemes)
    f = ej.filter_schemes_by_device_count(d8.schemes, num_devices=8)
    assert {(8, 8), (1, 8), (1, 1)} <= set(f) and not {(2, 8), (4, 8), (8, 4)} & set(f)
    f = ej.filter_schemes_by_device_count(DenseTensor("d", np.ones((16, 16))).schemes, 8)
    assert (4, 4) in f and (8, 8) not in f
    f = ej.filter_schemes_by_sharding(t.schemes, num_devices=4, min_sharded_dims=1)
    assert (4, 4) not in f


@pytest.mark.parametrize("seed", range(6))
def test_selection_on_gpu_stats_matches_oracle(gpu, seed):
    note("selection vs oracle", seed)
    rng = np.random.default_rng(200 + seed)
    shape = [(24, 36), (8, 12, 10), (60,), (32, 48), (6, 10, 14), (64, 64)][seed]
    d = rng.standard_normal(shape) * (rng.random(shape) < [0.01, 0.05, 0.2, 0.5][seed % 4])
    tensor = SparseTensor("x", torch.from_numpy(d).float().cuda()) if seed % 2 else \
        SparseTensor("x", d)
    idx, vals, _ = R.extract_coo(d.astype(np.float32) if seed % 2 else d)
    osch = S.schemes_from_metrics(R.sparsity_metrics(idx, vals, R.all_tile_shapes(shape)))
    assert [s.tile_shape for s in osch] == list(tensor.schemes)
    assert [s.num_tuples for s in osch] == [s.num_tuples for s in tensor.schemes.values()]
    for limit in (None, 256, 32, 4, 0):
        want = [s.tile_shape for s in S.rank_schemes_by_sparsity(
            S.prune_infeasible_schemes(osch, 1, limit), shape)]
        got = [s.tile_shape for s in ej.rank_schemes_by_sparsity(
            ej.prune_infeasible_schemes(tensor.schemes, 1, limit), shape)]
        assert got == want, limit
        ob = S.select_best_sparse_tiling(osch, shape, max_tile_bytes=limit)
        pb = ej.prepare_sparse_tiling(tensor, max_tile_bytes=limit)
        assert (pb is None) == (ob is None)
        if ob is not None:
            assert pb.tile_shape == ob.tile_shape


def test_registry_dispatch_runs_gpu_kernels(gpu):
    """Kernels looked up in the registry run the GPU path and match the oracle."""
    note("registry dispatch")
    w = G.workload_blocksparse_1k(n=512, tile=32, density=0.2)
    want = R.execute_sparse(w["lhs"], w["rhs"], w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    reg = ej.KernelRegistry()
    lhs = SparseTensorRelation(w["lhs"].coords, w["lhs"].values, w["lhs"].shape,
                               w["lhs"].tile_shape)
    rhs = SparseTensorRelation(w["rhs"].coords, w["rhs"].values, w["rhs"].shape,
                               w["rhs"].tile_shape)
    out = reg.lookup("ij,jk->ik", sparsity="sparse")(lhs, rhs)
    npt.assert_array_equal(out.coords, want.coords)
    assert R.rel_l2(out.values, want.values) <= 1e-5
    out = reg.lookup("ij,jk->ik", backend="gpu:mi355x", sparsity="sparse")(lhs, rhs)
    npt.assert_array_equal(out.coords, want.coords)
    fn = reg.lookup("ijk,kl->ijl", sparsity="sparse")
    w3 = G.workload_order3(n=256, l=64, density=0.05)
    got = fn(SparseTensorRelation(*w3["lhs"]), SparseTensorRelation(*w3["rhs"]), w3["join_keys"], w3["kernel_string"],
             w3["agg_keys"])
    want3 = R.execute_sparse(w3["lhs"], w3["rhs"], w3["join_keys"], w3["kernel_string"],
                             w3["agg_keys"], precision="fp64")
    npt.assert_array_equal(got.coords, want3.coords)
    assert R.rel_l2(got.values, want3.values) <= 1e-5
    with pytest.raises(NotImplementedError):
        reg.lookup("ij,jk->ik", sparsity="dense")()


@pytest.mark.parametrize("name", ["blocksparse_1k", "order3_small", "banded_small", "zipf_small"])
def test_api_einsum_relations(gpu, name):
    """einsum on relations: join keys and output coordinates derived from
    the labels, same result as the oracle's execute_sparse with the keys the
    workload names."""
    note("api einsum", name)
    if name == "blocksparse_1k":
        w = G.workload_blocksparse_1k(n=512)
    elif name == "order3_small":
        w = G.workload_order3(n=256, l=64, density=0.05)
    elif name == "banded_small":
        w = G.workload_batched_banded(b=2, n=512)
    else:
        w = G.workload_sparse_sparse_zipf(n=2048)
    want = R.execute_sparse(w["lhs"], w["rhs"], w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    tdt = torch.bfloat16 if w["dtype"] == "bf16" else torch.float32
    dev = [SparseTensorRelation(torch.from_numpy(r.coords).cuda(),
                                torch.from_numpy(r.values).cuda().to(tdt), r.shape, r.tile_shape)
           for r in (w["lhs"], w["rhs"])]
    got = ej.einsum(w["kernel_string"], *dev)
    assert got.is_device
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    tol = 1e-2 if w["dtype"] == "bf16" else 1e-5
    assert R.rel_l2(got.values.float().cpu().numpy(), want.values) <= tol
    host = ej.einsum(w["kernel_string"], SparseTensorRelation(*w["lhs"]),
                     SparseTensorRelation(*w["rhs"]), out_dtype=torch.float32)
    npt.assert_array_equal(host.coords, want.coords)
    assert R.rel_l2(host.values, want.values) <= tol
    with pytest.raises(NotImplementedError):
        ej.einsum(w["kernel_string"], *dev, num_devices=2)
