"""Host-side selection rules on the CPU: tile-shape selection (reference:
tensor/tiling.py), the kernel registry (kernels/registry.py) and the
api's shape analysis (api.py, core/notation.py).

The oracle's restatements (oracle/selection.py) are pinned first by the
reference's own known answers (tests/test_tiling.py, tests/test_pallas.py:
346-525) and by invariants of the ranking; the product is then compared
with the oracle over every tile shape of random tensors and over a grid of
registry queries.  Statistics that need the GPU (SparseTensor.schemes) are
exercised in test_gpu_selection.py; here schemes carry statistics from the
oracle's sparsity_metrics, or the full-grid counts of a dense tensor.
"""

import itertools
from math import prod

import numpy as np
import pytest

from oracle import reference_path as R
from oracle import selection as S

import einjax_amd as ej
from einjax_amd.kernels import registry as REG
from einjax_amd.tensor import tiling as T


def oracle_schemes(dense: np.ndarray) -> list:
    idx, vals, shape = R.extract_coo(dense)
    return S.schemes_from_metrics(R.sparsity_metrics(idx, vals, R.all_tile_shapes(shape)))


def product_schemes(dense: np.ndarray) -> dict:
    """Product TilingSchemes carrying the oracle's statistics."""
    out = {}
    for s in oracle_schemes(dense):
        sch = T.TilingScheme(None, dense.shape, s.tile_shape)
        sch.num_tuples = s.num_tuples
        out[s.tile_shape] = sch
    return out


def full_grid_schemes(shape) -> dict:
    """Schemes of a tensor with every element nonzero: every tile occupied."""
    return {ts: T.TilingScheme(None, shape, ts) for ts in T.enumerate_tile_shapes(shape)}


DIAG = np.diag([1.0, 2.0, 3.0, 4.0])

# ---------------------------------------------------------------------------
# oracle pinning: tile-shape selection


def test_oracle_selection_known_answers():
    """tests/test_tiling.py:33-160, :440-489."""
    sch = oracle_schemes(DIAG)
    assert len(sch) == 9
    # no pruning without a memory limit; a 4-byte limit keeps only (1,1)
    assert S.prune_infeasible_schemes(sch) == sch
    assert [s.tile_shape for s in S.prune_infeasible_schemes(sch, max_tile_bytes=4)] == [(1, 1)]
    assert S.prune_infeasible_schemes(sch, max_tile_bytes=1_000_000) == sch
    assert S.prune_infeasible_schemes(sch, max_tile_bytes=0) == []
    # diagonal: (1,1) is 4/16 = 0.25, the lowest ratio
    ranked = S.rank_schemes_by_sparsity(sch, DIAG.shape)
    assert ranked[0].tile_shape == (1, 1)
    assert S.select_best_sparse_tiling(sch, DIAG.shape).tile_shape == (1, 1)
    assert S.select_best_sparse_tiling(sch, DIAG.shape, max_tile_bytes=0) is None
    best = S.select_best_sparse_tiling(sch, DIAG.shape, max_tile_bytes=16, dtype_size=4)
    assert best.tile_size * 4 <= 16
    best = S.select_best_sparse_tiling(sch, DIAG.shape, max_tile_bytes=4, dtype_size=4)
    assert best.tile_size * 4 <= 4
    # all ones: every ratio is 1.0, ties go to the larger tile, (4,4) first
    ones = oracle_schemes(np.ones((4, 4)))
    ranked = S.rank_schemes_by_sparsity(ones, (4, 4))
    assert ranked[0].tile_shape == (4, 4)
    assert all(a.tile_size >= b.tile_size for a, b in zip(ranked, ranked[1:]))
    # 1-D sparse vector gives a scheme
    v = np.array([0.0, 1.0, 0.0, 3.0, 0.0, 0.0])
    assert S.select_best_sparse_tiling(oracle_schemes(v), v.shape) is not None
    assert S.sparsity_ratio(4, (4, 4), (1, 1)) == 0.25
    assert S.sparsity_ratio(1, (4, 4), (4, 4)) == 1.0


@pytest.mark.parametrize("seed", range(6))
def test_oracle_rank_invariants(seed):
    """The ranking is a permutation of the schemes, ordered by ratio
    ascending and, at equal ratio, by tile size descending, with equal keys
    left in enumeration order (a stable sort); the selection is its head."""
    rng = np.random.default_rng(seed)
    shape = [(12, 18), (8, 8, 6), (30,), (16, 24)][seed % 4]
    d = rng.standard_normal(shape) * (rng.random(shape) < [0.02, 0.1, 0.3][seed % 3])
    sch = oracle_schemes(d)
    ranked = S.rank_schemes_by_sparsity(sch, shape)
    assert sorted(map(tuple, ranked)) == sorted(map(tuple, sch))
    pos = {s.tile_shape: i for i, s in enumerate(sch)}
    for a, b in zip(ranked, ranked[1:]):
        ka = (S.sparsity_ratio(a.num_tuples, shape, a.tile_shape), -a.tile_size)
        kb = (S.sparsity_ratio(b.num_tuples, shape, b.tile_shape), -b.tile_size)
        assert ka < kb or (ka == kb and pos[a.tile_shape] < pos[b.tile_shape])
    # brute force: the minimum over every tile shape of (occupied fraction,
    # -tile size), occupancy counted by reducing the dense blocks
    best = None
    for ts in R.all_tile_shapes(shape):
        grid = tuple(s // t for s, t in zip(shape, ts))
        blocks = np.abs(d).reshape([x for g, t in zip(grid, ts) for x in (g, t)])
        occ = blocks.max(axis=tuple(range(1, 2 * len(shape), 2))) != 0
        key = (occ.sum() / occ.size, -prod(ts))
        if best is None or key < best[0]:
            best = (key, ts)
    assert S.select_best_sparse_tiling(sch, shape).tile_shape == best[1]


# ---------------------------------------------------------------------------
# oracle pinning: registry


def test_oracle_registry_known_answers():
    """tests/test_pallas.py:346-525."""
    E = S.BUILTINS
    assert S.lookup(E, "ij,jk->ik", "cpu", "sparse").name == "generic_sparse_matmul"
    assert S.lookup(E, "ij,jk->ik", "cpu", "dense").name == "generic_dense_einsum"
    assert S.lookup(E, "ij,kj->ik", "cpu", "sparse").name == "generic_sparse_einsum"
    assert S.lookup(E, "ij,jk->ik", "cpu", "unknown_mode") is None
    for b in ("gpu", "tpu", "cpu"):
        assert S.lookup(E, "ij,jk->ik", b, "sparse") is not None
    custom = E + [S.Entry("custom_sparse_matmul", "ij,jk->ik", "generic", "sparse", 10)]
    assert S.lookup(custom, "ij,jk->ik", "cpu", "sparse").name == "custom_sparse_matmul"
    mine = E + [S.Entry("my_custom", "ijk,jkl->il", "generic", "sparse", 5)]
    assert S.lookup(mine, "ijk,jkl->il", "cpu", "sparse").name == "my_custom"
    assert len(S.list_kernels(E)) >= 3
    assert len(S.list_kernels(E, sparsity="sparse")) >= 2
    assert len(S.list_kernels(E, sparsity="dense")) >= 1
    assert S.pattern_matches("ij,jk->ik", "ij,jk->ik") and S.pattern_matches("*", "anything")
    assert not S.pattern_matches("ij,jk->ik", "ij,kj->ik")
    assert all(S.backend_matches("generic", b) for b in ("gpu", "tpu", "cpu"))
    assert S.backend_matches("gpu", "gpu") and S.backend_matches("gpu", "gpu:triton")
    assert not S.backend_matches("gpu", "tpu")
    assert S.sparsity_matches("any", "dense") and S.sparsity_matches("any", "sparse")
    assert S.sparsity_matches("sparse", "sparse") and not S.sparsity_matches("sparse", "dense")
    # equal priorities: the earlier registration wins (stable sort)
    tie = E + [S.Entry("late", "ij,jk->ik", "generic", "sparse", 0)]
    assert S.lookup(tie, "ij,jk->ik", "cpu", "sparse").name == "generic_sparse_matmul"


# ---------------------------------------------------------------------------
# product tile-shape selection against the oracle


@pytest.mark.parametrize("seed", range(8))
def test_tiling_selection_matches_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    shape = [(12, 18), (8, 8, 6), (30,), (16, 24), (6, 10), (4, 6, 4, 2), (36,), (20, 20)][seed]
    d = rng.standard_normal(shape) * (rng.random(shape) < [0.02, 0.1, 0.3, 0.6][seed % 4])
    osch = oracle_schemes(d)
    psch = product_schemes(d)
    assert list(psch) == [s.tile_shape for s in osch]  # same enumeration order
    for limit, dsz in [(None, 4), (64, 4), (16, 8), (0, 4), (4, 4)]:
        want = [s.tile_shape for s in S.rank_schemes_by_sparsity(
            S.prune_infeasible_schemes(osch, 1, limit, dsz), shape)]
        got = [s.tile_shape for s in T.rank_schemes_by_sparsity(
            T.prune_infeasible_schemes(psch, 1, limit, dsz), shape)]
        assert got == want
        ob = S.select_best_sparse_tiling(osch, shape, max_tile_bytes=limit, dtype_size=dsz)
        pb = T.select_best_sparse_tiling(psch, shape, max_tile_bytes=limit, dtype_size=dsz)
        assert (pb is None) == (ob is None)
        if ob is not None:
            assert pb.tile_shape == ob.tile_shape and pb.num_tuples == ob.num_tuples
            assert isinstance(pb, T.TilingScheme)


def test_tiling_reference_cases_on_host_schemes():
    """tests/test_tiling.py cases whose statistics need no GPU: a fully
    dense tensor occupies every tile, as TilingScheme's defaults say."""
    # tie-break by tile size, coarsest tiling for a dense tensor (:99-109, :469-480)
    sch = full_grid_schemes((4, 4))
    ranked = T.rank_schemes_by_sparsity(sch, (4, 4))
    assert all(a.tile_size >= b.tile_size for a, b in zip(ranked, ranked[1:]))
    assert T.select_best_sparse_tiling(sch, (4, 4)).tile_shape == (4, 4)
    # partition specs (:168-202)
    assert T.get_sparse_partition_spec(T.TilingScheme(None, (4, 4), (2, 2))) == ("x", "y")
    assert T.get_sparse_partition_spec(T.TilingScheme(None, (4, 4), (4, 4))) == (None, None)
    assert T.get_sparse_partition_spec(T.TilingScheme(None, (4, 4), (2, 4))) == ("x", None)
    assert T.get_sparse_partition_spec(T.TilingScheme(None, (4, 4), (2, 2)),
                                       mesh_axis_names=("a", "b")) == ("a", "b")
    # memory (:210-262)
    assert T.compute_tile_memory((2, 2), dtype_size=4) == 24
    assert T.compute_tile_memory((2, 2), dtype_size=4, include_coords=False) == 16
    assert T.compute_tile_memory((2, 3, 4), dtype_size=4) == 108
    assert T.compute_tile_memory((1, 1), dtype_size=4) == 12
    s = T.TilingScheme(None, (4, 4), (2, 2))
    s.num_tuples = 3
    assert T.compute_relation_memory(s, dtype_size=4) == 72
    s.num_tuples = 0
    assert T.compute_relation_memory(s) == 0
    s = T.TilingScheme(None, (4, 4), (4, 4))
    s.num_tuples = 1
    assert T.compute_relation_memory(s, dtype_size=4) == 72
    # device-count filter (:328-435)
    s8 = full_grid_schemes((8, 8))
    assert len(T.filter_schemes_by_device_count(s8, num_devices=1)) == len(s8)
    f = T.filter_schemes_by_device_count(s8, num_devices=8)
    assert (8, 8) in f and (1, 8) in f and (1, 1) in f
    assert (2, 8) not in f and (4, 8) not in f and (8, 4) not in f
    s16 = full_grid_schemes((16, 16))
    f = T.filter_schemes_by_device_count(s16, num_devices=8)
    assert (4, 4) in f and (8, 8) not in f

    def upper_tiles(sch):
        cases = sch.get_case_assignments()
        return prod(a // t for a, t, c in zip(sch.shape, sch.tile_shape, cases)
                    if c == T.CaseAssignment.UPPER)

    for sch in f.values():
        if any(c == T.CaseAssignment.UPPER for c in sch.get_case_assignments()):
            assert upper_tiles(sch) >= 8 and upper_tiles(sch) % 8 == 0
    for sch in T.filter_schemes_by_device_count(s16, 8, min_tiles_per_device=2).values():
        if any(c == T.CaseAssignment.UPPER for c in sch.get_case_assignments()):
            assert upper_tiles(sch) >= 16
    for sch in T.filter_schemes_by_device_count(full_grid_schemes((12, 12)), 8).values():
        if any(c == T.CaseAssignment.UPPER for c in sch.get_case_assignments()):
            assert upper_tiles(sch) % 8 == 0
    # sharding filter on a diagonal's schemes (:270-322)
    sd = product_schemes(DIAG)
    f = T.filter_schemes_by_sharding(sd, num_devices=4, min_sharded_dims=1)
    assert (4, 4) not in f
    for sch in T.filter_schemes_by_sharding(sd, num_devices=4, max_sharded_dims=1).values():
        assert sum(c == T.CaseAssignment.UPPER for c in sch.get_case_assignments()) <= 1
    for sch in T.filter_schemes_by_sharding(sd, num_devices=2, min_sharded_dims=1).values():
        assert upper_tiles(sch) <= 2
    sd2 = product_schemes(np.diag([1.0, 2.0]))
    assert len(T.filter_schemes_by_sharding(sd2, num_devices=1)) == len(sd2)


def test_tiling_names_exported():
    """tests/test_tiling.py:516-544."""
    for name in ("prune_infeasible_schemes", "rank_schemes_by_sparsity",
                 "select_best_sparse_tiling", "get_sparse_partition_spec", "compute_tile_memory",
                 "compute_relation_memory", "filter_schemes_by_sharding",
                 "filter_schemes_by_device_count", "prepare_sparse_tiling"):
        assert getattr(ej, name) is getattr(ej.tensor, name)


# ---------------------------------------------------------------------------
# product registry: the reference's tests, then the oracle over a query grid


def test_registry_reference_cases():
    """tests/test_pallas.py:346-525."""
    reg = ej.KernelRegistry()
    assert reg.lookup("ij,jk->ik", backend="cpu", sparsity="sparse") is \
        ej.block_sparse_matmul_generic
    assert reg.lookup("ij,jk->ik", backend="cpu", sparsity="dense") is REG.execute_dense_einsum
    assert reg.lookup("ij,kj->ik", backend="cpu", sparsity="sparse") is ej.execute_sparse
    with pytest.raises(ValueError):
        reg.lookup("ij,jk->ik", backend="cpu", sparsity="unknown_mode")
    for b in ("gpu", "tpu", "cpu"):
        assert reg.lookup("ij,jk->ik", backend=b, sparsity="sparse") is not None

    def custom_matmul(*a, **k):
        pass

    reg.register(ej.KernelInfo("custom_sparse_matmul", "ij,jk->ik", "generic", "sparse", 10,
                               custom_matmul))
    assert reg.lookup("ij,jk->ik", backend="cpu", sparsity="sparse") is custom_matmul
    reg = ej.KernelRegistry()

    def my_kernel(*a, **k):
        return "custom_result"

    reg.register(ej.KernelInfo("my_custom", "ijk,jkl->il", "generic", "sparse", 5, my_kernel))
    assert reg.lookup("ijk,jkl->il", backend="cpu", sparsity="sparse") is my_kernel
    reg = ej.KernelRegistry()
    assert len(reg.list_kernels()) >= 3
    assert len(reg.list_kernels(sparsity="sparse")) >= 2
    assert len(reg.list_kernels(sparsity="dense")) >= 1
    info = reg.lookup_info("ij,jk->ik", backend="cpu", sparsity="sparse")
    assert isinstance(info, ej.KernelInfo)
    assert info.pattern == "ij,jk->ik" and info.name == "generic_sparse_matmul"
    with pytest.raises(ValueError):
        reg.lookup_info("ij,jk->ik", backend="cpu", sparsity="nonexistent")
    assert REG._pattern_matches("ij,jk->ik", "ij,jk->ik") and REG._pattern_matches("*", "x")
    assert not REG._pattern_matches("ij,jk->ik", "ij,kj->ik")
    assert all(REG._backend_matches("generic", b) for b in ("gpu", "tpu", "cpu"))
    assert REG._backend_matches("gpu", "gpu") and REG._backend_matches("gpu", "gpu:triton")
    assert not REG._backend_matches("gpu", "tpu")
    assert REG._sparsity_matches("any", "dense") and REG._sparsity_matches("any", "sparse")
    assert REG._sparsity_matches("sparse", "sparse")
    assert not REG._sparsity_matches("sparse", "dense")
    assert REG._detect_backend() in ("gpu", "tpu", "cpu")
    from einjax_amd.kernels import (KernelInfo, KernelRegistry, block_sparse_matmul,  # noqa: F401
                                    block_sparse_matmul_generic, coordinate_join_hash,
                                    coordinate_join_sorted)


EXTRA = [S.Entry("custom_gpu_matmul", "ij,jk->ik", "gpu", "sparse", 3),
         S.Entry("any_star", "*", "generic", "any", -5),
         S.Entry("late_tie", "ij,jk->ik", "generic", "sparse", 0),
         S.Entry("triton_batch", "bij,bjk->bik", "gpu:triton", "sparse", 7),
         S.Entry("tpu_dense", "*", "tpu", "dense", 2)]


def test_registry_matches_oracle_on_query_grid():
    patterns = ["ij,jk->ik", "ij,kj->ik", "bij,bjk->bik", "ijk,kl->ijl", "*", "x"]
    backends = ["cpu", "gpu", "tpu", "gpu:triton", "generic", "gpu:mi355x"]
    sparsities = ["sparse", "dense", "any", "other"]
    for n_extra in range(len(EXTRA) + 1):
        entries = S.BUILTINS + EXTRA[:n_extra]
        reg = ej.KernelRegistry()
        fns = {e.name: (lambda *a, _n=e.name: _n) for e in EXTRA}
        for e in EXTRA[:n_extra]:
            reg.register(ej.KernelInfo(e.name, e.pattern, e.backend, e.sparsity, e.priority,
                                       fns[e.name]))
        assert [k.name for k in reg.list_kernels()] == [e.name for e in entries]
        for p, b, s in itertools.product(patterns, backends, sparsities):
            want = S.lookup(entries, p, b, s)
            if want is None:
                with pytest.raises(ValueError):
                    reg.lookup_info(p, b, s)
            else:
                assert reg.lookup_info(p, b, s).name == want.name, (p, b, s)
        for p, b, s in itertools.product(patterns + [None], backends + [None],
                                         sparsities + [None]):
            assert [k.name for k in reg.list_kernels(p, b, s)] == \
                [e.name for e in S.list_kernels(entries, p, b, s)]


# ---------------------------------------------------------------------------
# api: shape analysis and the relation einsum plan


def test_analyze_reference_cases():
    """tests/test_execution.py:181-230, tests/test_api.py:414-425."""
    r = ej.analyze("ij,jk->ik", np.ones((3, 4)), np.ones((4, 5)))
    assert isinstance(r, ej.AnalysisResult)
    assert r.einsum_string == "ij,jk->ik" and r.input_shapes == [(3, 4), (4, 5)]
    assert r.output_shape == (3, 5) and r.contracted_indices == ["j"]
    assert r.free_indices == ["i", "k"] and r.label_dimensions == {"i": 3, "j": 4, "k": 5}
    r = ej.analyze("ij,jk", np.ones((3, 4)), np.ones((4, 5)))
    assert r.einsum_string == "ij,jk->ik" and r.output_shape == (3, 5)
    r = ej.analyze("ii->", np.ones((4, 4)))
    assert r.output_shape == () and r.contracted_indices == ["i"] and r.free_indices == []
    r = ej.analyze("ij->ji", np.ones((3, 4)))
    assert r.output_shape == (4, 3) and r.contracted_indices == [] and r.free_indices == ["i", "j"]
    s = repr(ej.analyze("ij,jk->ik", np.ones((2, 3)), np.ones((3, 4))))
    assert "ij,jk->ik" in s and "contracted" in s
    # relations are analysed by their logical shapes
    rel = ej.SparseTensorRelation(np.zeros((0, 2), np.int32), np.zeros((0, 2, 2)), (4, 6), (2, 2))
    assert ej.analyze("ij,jk->ik", rel, np.ones((6, 8))).output_shape == (4, 8)


def test_notation_reference_cases():
    """tests/test_notation.py:55-170."""
    assert ej.normalize_notation("ij,jk") == "ij,jk->ik"
    assert ej.normalize_notation("ii") == "ii->"
    assert ej.normalize_notation("ij") == "ij->ij"
    assert ej.normalize_notation("ij,jk,kl") == "ij,jk,kl->il"
    assert ej.normalize_notation("ij,jk->ik") == "ij,jk->ik"
    assert ej.normalize_notation("ij,ij") == "ij,ij->"
    assert ej.get_label_dimensions("ij,jk->ik", [(3, 4), (4, 5)]) == {"i": 3, "j": 4, "k": 5}
    with pytest.raises(ValueError):
        ej.get_label_dimensions("ij,jk->ik", [(3, 4), (5, 6)])
    ej.validate_inputs("ij,jk->ik", [(3, 4), (4, 5)])
    for spec, shapes in [("ij,jk->ik", [(3, 4)]), ("ij,jk->ik", [(3, 4), (5, 6)]),
                         ("ij,jk->iz", [(3, 4), (4, 5)]), ("ij,jk->ik", [(3, 4, 1), (4, 5)]),
                         ("iJ,Jk->ik", [(3, 4), (4, 5)])]:
        with pytest.raises(ValueError):
            ej.validate_inputs(spec, shapes)


def test_relation_einsum_plan():
    """Join keys and output coordinates derived from the labels equal the
    ones the reference's own callers pass for these strings
    (tests/test_sparse_dispatch.py:263-426, tests/test_pallas.py:53-224)."""
    from einjax_amd.api import relation_einsum_plan as plan

    assert plan("ij,jk->ik", (2, 2), (2, 2)) == ([(1, 0)], [(0, 0), (1, 1)])
    assert plan("bij,bjk->bik", (1, 4, 4), (1, 4, 4)) == ([(0, 0), (2, 1)],
                                                          [(0, 0), (0, 1), (1, 2)])
    assert plan("ijk,kl->ijl", (2, 2, 2), (2, 2)) == ([(2, 0)], [(0, 0), (0, 1), (1, 1)])
    assert plan("ij,ij->ij", (1, 1), (1, 1)) == ([(0, 0), (1, 1)], [(0, 0), (0, 1)])
    assert plan("i,j->ij", (1,), (1,)) == ([], [(0, 0), (1, 0)])
    assert plan("ij,jk", (2, 3), (3, 5)) == ([(1, 0)], [(0, 0), (1, 1)])
    with pytest.raises(ValueError):
        plan("ij,jk->ik", (2, 3), (2, 5))
    with pytest.raises(NotImplementedError):
        plan("ii,ij->j", (2, 2), (2, 2))
    with pytest.raises(NotImplementedError):
        ej.einsum("ij,jk->ik", np.ones((2, 2)), np.ones((2, 2)))
