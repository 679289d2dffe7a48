"""The execution engine's host logic (reference: execution/engine.py), restated
from the reference's tests/test_execution.py:228-530: the dependency graph and
Kahn ordering of scheme DAGs, and the errors raised before any step runs."""

from types import SimpleNamespace

import pytest

from einjax_amd import TilingScheme
from einjax_amd.execution.engine import (ContractionPlan, ContractionStep, ExecutionEngine,
                                         build_dependency_graph, topological_sort)


def scheme(name, shape=(4, 4), tile=(4, 4)):
    return TilingScheme(SimpleNamespace(name=name), shape, tile)


def test_single_node_no_deps():
    s = scheme("A")
    graph = build_dependency_graph(s)
    assert len(graph) == 1
    assert not graph[id(s)][1] and not graph[id(s)][2]


def test_binary_contraction_edges():
    sa, sb, out = scheme("A"), scheme("B"), scheme("C")
    out.source = (sa, sb)
    graph = build_dependency_graph(out)
    assert len(graph) == 3
    assert len(graph[id(out)][1]) == 2 and not graph[id(out)][2]
    for src in (sa, sb):
        assert not graph[id(src)][1] and len(graph[id(src)][2]) == 1


def test_topological_orders():
    s = scheme("A")
    assert topological_sort(s) == [s]
    sa, sb, sc, st1, st2 = (scheme(n) for n in ("A", "B", "C", "T1", "T2"))
    st1.source = (sa, sb)
    st2.source = (st1, sc)
    ordered = topological_sort(st2)
    assert len(ordered) == 5 and ordered[-1] is st2
    assert len({id(x) for x in ordered}) == 5
    assert ordered.index(st1) < ordered.index(st2)
    assert ordered.index(sa) < ordered.index(st1) and ordered.index(sb) < ordered.index(st1)


def test_cycle_detected():
    a, b = scheme("A"), scheme("B")
    a.source = (b,)
    b.source = (a,)
    with pytest.raises(RuntimeError, match="Cycle"):
        topological_sort(a)


def test_errors_before_any_step():
    sa, sb, out = scheme("A"), scheme("B"), scheme("result")
    out.source = (sa, sb)
    eng = ExecutionEngine()
    with pytest.raises(ValueError):  # missing formula
        eng.execute_schemes(out, data={"A": object(), "B": object()}, formulas={})
    with pytest.raises(ValueError):  # missing input
        eng.execute_schemes(out, data={"A": object()}, formulas={"result": "ij,jk->ik"})
    with pytest.raises(ValueError):  # formula count
        eng.execute_sequence([sa, sb, out], [object(), object()], ["ij,jk->ik", "extra"])


def test_dense_steps_and_meshes_raise():
    plan = ContractionPlan("ij,jk->ik", [ContractionStep(0, "ij,jk->ik", (0, 1))])
    with pytest.raises(NotImplementedError, match="dense"):
        ExecutionEngine().execute_plan(plan, [[[1.0]], [[1.0]]])
    mesh = SimpleNamespace(devices=SimpleNamespace(size=8), axis_names=("x",))
    with pytest.raises(NotImplementedError, match="one process per GPU"):
        ExecutionEngine(mesh=mesh)
