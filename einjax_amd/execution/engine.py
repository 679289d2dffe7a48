"""Execution of contraction sequences over tile relations (reference:
execution/engine.py).

The reference's engine orders a DAG of tiling schemes (Kahn's algorithm) and
runs every binary step as a dense, optionally sharded, jnp einsum.  This
engine keeps that interface (``build_dependency_graph``, ``topological_sort``,
``ExecutionEngine.execute_plan`` / ``execute_schemes`` / ``execute_sequence``,
with the reference's arguments and control flow) and runs each binary step
whose two operands are ``SparseTensorRelation``s through ``execute_sparse``:
the join keys and output coordinates come from the step's labels, and an
intermediate stays a device-resident relation for the next step (no host
round trip between steps).  A step with a dense operand raises
NotImplementedError (the dense path is not part of this library), and so
does a mesh of more than one device (one process drives one GPU).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from ..tensor.sparse import SparseTensorRelation
from ..tensor.tiling import TilingScheme

__all__ = ["build_dependency_graph", "topological_sort", "ContractionStep", "ContractionPlan",
           "ExecutionEngine"]


def build_dependency_graph(root_scheme) -> dict:
    """{id(scheme): (scheme, incoming ids, outgoing ids)} over the schemes
    reachable from root_scheme through ``source`` (reference:
    execution/engine.py:27-60).  Each scheme's sources are expanded once:
    the graph of a DAG is the reference's, and a cycle ends the walk (the
    reference re-queues every source and never ends on one), so that
    topological_sort reports it."""
    graph: dict = {}
    todo = [root_scheme]
    expanded = set()
    while todo:
        scheme = todo.pop(0)
        sid = id(scheme)
        graph.setdefault(sid, (scheme, set(), set()))
        if sid in expanded:
            continue
        expanded.add(sid)
        for src in scheme.source:
            todo.append(src)
            graph.setdefault(id(src), (src, set(), set()))
            graph[id(src)][2].add(sid)
            graph[sid][1].add(id(src))
    return graph


def topological_sort(root_scheme) -> list:
    """Schemes in dependency order, inputs first and root last (Kahn's
    algorithm, taking the first ready node in insertion order as the
    reference does, execution/engine.py:63-110); RuntimeError on a cycle."""
    graph = {sid: (s, set(i), set(o)) for sid, (s, i, o) in build_dependency_graph(root_scheme).items()}
    ordered = []
    while graph:
        ready = next((sid for sid, (_, inc, _) in graph.items() if not inc), None)
        if ready is None:
            raise RuntimeError("Cycle detected in dependency graph")
        scheme, _, out = graph.pop(ready)
        for o in out:
            if o in graph:
                graph[o][1].discard(ready)
        ordered.append(scheme)
    return ordered


@dataclass
class ContractionStep:
    """One binary step of a contraction plan (fields of the reference's
    optimizer/contraction_path.py:31-56; the engine reads ``formula``,
    ``input_indices`` and ``best_scheme``)."""

    step_index: int
    formula: str
    input_indices: tuple
    lhs_labels: str = ""
    rhs_labels: str = ""
    output_labels: str = ""
    output_tensor: Any = None
    reduction_info: Any = None
    best_scheme: Any = None


@dataclass
class ContractionPlan:
    """A sequence of binary steps over a working list of operands, each step
    consuming input_indices and appending its result (reference:
    optimizer/contraction_path.py:59-74)."""

    einsum_string: str
    steps: list
    total_cost: float = 0.0
    tiling_schemes: list = field(default_factory=list)


def _devices(mesh) -> int:
    if mesh is None:
        return 1
    devs = getattr(mesh, "devices", None)
    if devs is None:
        return 1
    size = getattr(devs, "size", None)
    return int(size) if size is not None else len(devs)


class ExecutionEngine:
    """Runs contraction plans and scheme DAGs step by step (reference:
    execution/engine.py:113-487).  Every step is a binary sparse einsum on
    the GPU; intermediates stay device relations.  ``step_options`` (an
    extension): keyword arguments for every step's execute_sparse call,
    e.g. ``fused`` or ``out_dtype``."""

    def __init__(self, mesh: Any = None, cost_config: Any = None,
                 mesh_axis_names: tuple | None = None, **step_options):
        if _devices(mesh) > 1:
            raise NotImplementedError("multi-device execution is not part of this library: "
                                      "run one process per GPU")
        self.mesh = mesh
        self.cost_config = cost_config
        if mesh is not None and mesh_axis_names is None:
            self.mesh_axis_names = tuple(getattr(mesh, "axis_names", ("x", "y", "z", "w")))
        else:
            self.mesh_axis_names = mesh_axis_names or ("x", "y", "z", "w")
        self.step_options = step_options

    def _execute_einsum(self, formula: str, source_arrays: list, source_schemes=None,
                        output_scheme=None):
        """One binary step: execute_sparse with join keys and output
        coordinates from the formula's labels (the reference runs a dense
        einsum here, engine.py:194-230)."""
        from ..api import relation_einsum_plan
        from .sparse_dispatch import execute_sparse

        if len(source_arrays) != 2:
            raise NotImplementedError(f"steps are binary einsums, got {len(source_arrays)} "
                                      f"operands for '{formula}'")
        lhs, rhs = source_arrays
        if not (isinstance(lhs, SparseTensorRelation) and isinstance(rhs, SparseTensorRelation)):
            raise NotImplementedError("dense einsum steps are not part of einjax_amd; the "
                                      "engine runs steps whose operands are SparseTensorRelation")
        join, agg = relation_einsum_plan(formula, lhs.tile_shape, rhs.tile_shape)
        return execute_sparse(lhs, rhs, join, formula, agg, **self.step_options)

    def execute_plan(self, plan, operands: list, gather_output: bool = False):
        """Runs plan.steps in order over a working list that starts as the
        operands; each step removes its inputs and appends its result
        (reference: engine.py:264-324).  Returns the last result.
        gather_output has nothing to gather on one device."""
        intermediates = list(operands)
        for step in plan.steps:
            idx = tuple(step.input_indices)
            result = self._execute_einsum(step.formula, [intermediates[idx[0]],
                                                         intermediates[idx[1]]])
            for i in sorted(idx, reverse=True):
                del intermediates[i]
            intermediates.append(result)
        return intermediates[-1]

    def execute_schemes(self, root_scheme, data: dict, formulas: dict,
                        gather_output: bool = False):
        """Runs the DAG under root_scheme in topological order: a scheme
        whose node name is in data is an input, every other one is computed
        from its source schemes with formulas[name] (reference:
        engine.py:326-409)."""
        ordered = topological_sort(root_scheme)
        results = dict(data)
        for scheme in ordered:
            name = scheme.node.name
            if name in results:
                continue
            formula = formulas.get(name)
            if formula is None:
                raise ValueError(f"No formula provided for non-input node '{name}'")
            srcs = []
            for src in scheme.source:
                if src.node.name not in results:
                    raise ValueError(f"Missing intermediate result for '{src.node.name}'")
                srcs.append(results[src.node.name])
            results[name] = self._execute_einsum(formula, srcs, list(scheme.source), scheme)
        return results[ordered[-1].node.name]

    def execute_sequence(self, schemes: list, operands: list, formulas: list,
                         gather_output: bool = False):
        """Runs an ordered scheme list: the first len(operands) schemes are
        the inputs, each later scheme is computed, with the next formula, from
        its source schemes, found by identity among the schemes before it
        (reference: engine.py:411-487).  ValueError when the formulas do not
        match the computed schemes in number."""
        n_in = len(operands)
        n_compute = len(schemes) - n_in
        if len(formulas) != n_compute:
            raise ValueError(f"Expected {n_compute} formulas for {n_compute} compute steps, "
                             f"got {len(formulas)}")
        results = list(operands)
        for i, formula in enumerate(formulas):
            scheme = schemes[n_in + i]
            srcs = []
            for src in scheme.source:
                for j, s in enumerate(schemes):
                    if s is src and j < len(results):
                        srcs.append(results[j])
                        break
            results.append(self._execute_einsum(formula, srcs, list(scheme.source), scheme))
        return results[-1]
