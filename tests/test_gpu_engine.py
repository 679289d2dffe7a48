"""The execution engine on the GPU (reference: execution/engine.py:113-487).

The reference's engine tests (tests/test_execution.py:355-510) restated with
tile relations as operands: each binary step runs through execute_sparse,
intermediates stay device relations, and the chained result matches the
oracle's chain of execute_sparse calls (coordinates bit-exact, values within
the fp32 / bf16 tolerance of float64 math).
"""

from types import SimpleNamespace

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R

from einjax_amd import SparseTensorRelation, TilingScheme
from einjax_amd.execution.engine import ContractionPlan, ContractionStep, ExecutionEngine

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


def dev_rel(r: R.Rel, dtype=torch.float32):
    return SparseTensorRelation(torch.from_numpy(np.ascontiguousarray(r.coords)).cuda(),
                                torch.from_numpy(np.ascontiguousarray(r.values, np.float32))
                                .cuda().to(dtype), r.shape, r.tile_shape)


def dense(rel: SparseTensorRelation) -> np.ndarray:
    return rel.to_dense().float().cpu().numpy()


def block_sparse(rng, shape, tile, density):
    grid = (shape[0] // tile, shape[1] // tile)
    mask = rng.random(grid) < density
    d = rng.standard_normal(shape) * np.kron(mask, np.ones((tile, tile)))
    return R.dense_to_relation(d, (tile, tile))


def test_reference_matmul_plan_schemes_sequence(gpu):
    note("engine: identity x arange through plan, schemes and sequence")
    a = R.dense_to_relation(np.eye(4), (2, 2))
    b = R.dense_to_relation(np.arange(16, dtype=np.float64).reshape(4, 4) + 1, (2, 2))
    want = np.eye(4) @ (np.arange(16).reshape(4, 4) + 1)
    eng = ExecutionEngine()
    plan = ContractionPlan("ij,jk->ik", [ContractionStep(0, "ij,jk->ik", (0, 1))])
    out = eng.execute_plan(plan, [dev_rel(a), dev_rel(b)])
    assert out.is_device and out.shape == (4, 4)
    npt.assert_allclose(dense(out), want, rtol=1e-6)
    sa = TilingScheme(SimpleNamespace(name="A"), (4, 4), (2, 2))
    sb = TilingScheme(SimpleNamespace(name="B"), (4, 4), (2, 2))
    so = TilingScheme(SimpleNamespace(name="result"), (4, 4), (2, 2))
    so.source = (sa, sb)
    out = eng.execute_schemes(so, data={"A": dev_rel(a), "B": dev_rel(b)},
                              formulas={"result": "ij,jk->ik"})
    npt.assert_allclose(dense(out), want, rtol=1e-6)
    out = eng.execute_sequence([sa, sb, so], [dev_rel(a), dev_rel(b)], ["ij,jk->ik"])
    npt.assert_allclose(dense(out), want, rtol=1e-6)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_three_operand_block_sparse_chain(gpu, dtype):
    """(A B) C over 32x32 tiles: the plan consumes A and B, appends T, then
    contracts T with C; against the oracle's chain in float64."""
    note("engine: three-operand block-sparse chain", dtype)
    rng = np.random.default_rng(21)
    A = block_sparse(rng, (256, 384), 32, 0.15)
    B = block_sparse(rng, (384, 512), 32, 0.25)
    C = block_sparse(rng, (512, 160), 32, 0.35)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":  # the oracle sees the values the GPU sees
        A, B, C = (R.Rel(r.coords, R.bf16_round(r.values.astype(np.float32)), r.shape,
                         r.tile_shape) for r in (A, B, C))
    plan = ContractionPlan("ij,jk,kl->il", [ContractionStep(0, "ij,jk->ik", (0, 1)),
                                            ContractionStep(1, "ik,kl->il", (1, 0))])
    out = ExecutionEngine().execute_plan(plan, [dev_rel(A, tdt), dev_rel(B, tdt), dev_rel(C, tdt)])
    assert out.is_device and out.values.dtype == tdt
    T = R.execute_sparse(A, B, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], precision="fp64")
    if dtype == "bf16":  # the intermediate is a bf16 relation on the GPU
        T = R.Rel(T.coords, R.bf16_round(T.values.astype(np.float32)), T.shape, T.tile_shape)
    want = R.execute_sparse(T, C, [(1, 0)], "ik,kl->il", [(0, 0), (1, 1)], precision="fp64")
    npt.assert_array_equal(out.coords.cpu().numpy(), want.coords)
    assert out.shape == (256, 160) and out.tile_shape == (32, 32)
    tol = 1e-2 if dtype == "bf16" else 1e-5
    assert R.rel_l2(out.values.float().cpu().numpy(), want.values) <= tol
    # and the dense product of the three operands
    full = R.relation_to_dense(A) @ R.relation_to_dense(B) @ R.relation_to_dense(C)
    assert R.rel_l2(dense(out), full) <= (2e-2 if dtype == "bf16" else 1e-5)


def test_sequence_chain_with_shared_source(gpu):
    """A scheme sequence whose last step reads an input twice removed:
    T1 = A B, T2 = T1 C; sources found by identity among earlier schemes."""
    note("engine: execute_sequence chain")
    w = G.workload_blocksparse_1k(n=256, tile=32, density=0.2)
    A, B = w["lhs"], w["rhs"]
    rng = np.random.default_rng(5)
    C = block_sparse(rng, (256, 96), 32, 0.5)
    mk = lambda n, shape: TilingScheme(SimpleNamespace(name=n), shape, (32, 32))
    sa, sb, sc = mk("A", A.shape), mk("B", B.shape), mk("C", C.shape)
    t1, t2 = mk("T1", (256, 256)), mk("T2", (256, 96))
    t1.source = (sa, sb)
    t2.source = (t1, sc)
    out = ExecutionEngine().execute_sequence([sa, sb, sc, t1, t2],
                                             [dev_rel(A), dev_rel(B), dev_rel(C)],
                                             ["ij,jk->ik", "ik,kl->il"])
    T = R.execute_sparse(A, B, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], precision="fp64")
    want = R.execute_sparse(T, C, [(1, 0)], "ik,kl->il", [(0, 0), (1, 1)], precision="fp64")
    npt.assert_array_equal(out.coords.cpu().numpy(), want.coords)
    assert R.rel_l2(out.values.cpu().numpy(), want.values) <= 1e-5
