"""User-facing entry points (reference: api.py:89-200, :323-397).

``analyze`` is the reference's shape analysis, unchanged in behaviour.
``einsum`` keeps the reference's signature; the reference's version is
dense only (it runs jnp.einsum, api.py:185-194).  This library implements
the tensor-relational sparse path, so ``einsum`` here is an extension: with
``SparseTensorRelation`` operands it derives the join keys and the output
tile coordinates from the labels and runs ``execute_sparse``
(execution/sparse_dispatch.py:226-297) on the GPU; dense operands raise
NotImplementedError, as the registry's dense entry does.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass
from typing import Any

import numpy as np

from .execution.sparse_dispatch import execute_sparse
from .tensor.sparse import SparseTensorRelation

__all__ = ["einsum", "analyze", "AnalysisResult", "normalize_notation", "validate_inputs",
           "get_label_dimensions", "relation_einsum_plan"]


def normalize_notation(einsum_string: str) -> str:
    """Explicit output labels, NumPy's implicit rule when "->" is absent: the
    labels that appear exactly once, sorted (reference: core/notation.py:74-98)."""
    if "->" in einsum_string:
        return einsum_string
    counts = Counter(einsum_string.replace(",", ""))
    return einsum_string + "->" + "".join(sorted(c for c in counts if counts[c] == 1))


def validate_inputs(einsum_string: str, shapes, names=None) -> None:
    """Operand count, lowercase labels, label-group rank, consistent extents
    and output labels drawn from the inputs; ValueError otherwise
    (reference: core/notation.py:101-181)."""
    names = names or [f"tensor_{i}" for i in range(len(shapes))]
    ins, _, out = einsum_string.partition("->")
    groups = ins.split(",")
    if len(groups) != len(shapes):
        raise ValueError(f"Number of input label groups ({len(groups)}) does not match "
                         f"number of tensors ({len(shapes)}): '{einsum_string}'")
    for ch in ins.replace(",", "") + out:
        if not ch.isalpha() or not ch.islower():
            raise ValueError(f"Invalid label character '{ch}' in '{einsum_string}': "
                             "labels must be lowercase alphabetic (a-z)")
    for i, (g, s) in enumerate(zip(groups, shapes)):
        if len(g) != len(s):
            raise ValueError(f"Label group '{g}' has {len(g)} indices but tensor '{names[i]}' "
                             f"(argument {i}) has {len(s)} dimensions (shape {tuple(s)})")
    seen: dict = {}
    for i, (g, s) in enumerate(zip(groups, shapes)):
        for lab, n in zip(g, s):
            if lab not in seen:
                seen[lab] = (n, names[i], i)
            elif seen[lab][0] != n:
                d0, n0, i0 = seen[lab]
                raise ValueError(f"Dimension mismatch for label '{lab}': tensor '{n0}' "
                                 f"(argument {i0}) has dimension {d0}, but tensor '{names[i]}' "
                                 f"(argument {i}) has dimension {n}")
    labels = set(ins.replace(",", ""))
    for ch in out:
        if ch not in labels:
            raise ValueError(f"Output label '{ch}' does not appear in any input: "
                             f"'{einsum_string}'. Output labels must be a subset of input "
                             f"labels {sorted(labels)}")


def get_label_dimensions(einsum_string: str, shapes) -> dict:
    """Label -> extent, first occurrence; ValueError on a mismatch
    (reference: core/notation.py:46-71)."""
    dims: dict = {}
    for g, s in zip(einsum_string.split("->")[0].split(","), shapes):
        for lab, n in zip(g, s):
            if lab not in dims:
                dims[lab] = n
            elif dims[lab] != n:
                raise ValueError(f"Dimension mismatch for label '{lab}': expected {dims[lab]}, "
                                 f"got {n}")
    return dims


@dataclass
class AnalysisResult:
    """Shape analysis of an einsum (reference: api.py:323-349)."""

    einsum_string: str
    input_shapes: list
    output_shape: tuple
    label_dimensions: dict
    contracted_indices: list
    free_indices: list

    def __repr__(self) -> str:
        contracted = ", ".join(self.contracted_indices) or "(none)"
        free = ", ".join(self.free_indices) or "(none)"
        return (f"AnalysisResult(\n  notation='{self.einsum_string}',\n"
                f"  input_shapes={self.input_shapes},\n  output_shape={self.output_shape},\n"
                f"  contracted_indices=[{contracted}],\n  free_indices=[{free}],\n"
                f"  label_dimensions={self.label_dimensions},\n)")


def _shape_of(op) -> tuple:
    if hasattr(op, "shape"):
        return tuple(int(s) for s in op.shape)
    return tuple(np.asarray(op).shape)


def analyze(einsum_string: str, *operands: Any) -> AnalysisResult:
    """Shapes, contracted and free labels of an einsum, without running it
    (reference: api.py:352-397).  Operands may be arrays, tensors or
    relations (only their shapes are read)."""
    einsum_string = normalize_notation(einsum_string)
    shapes = [_shape_of(op) for op in operands]
    validate_inputs(einsum_string, shapes)
    dims = get_label_dimensions(einsum_string, shapes)
    ins, out = einsum_string.split("->")
    in_labels = set(ins.replace(",", ""))
    return AnalysisResult(einsum_string=einsum_string, input_shapes=shapes,
                          output_shape=tuple(dims[c] for c in out),
                          label_dimensions=dims,
                          contracted_indices=sorted(in_labels - set(out)),
                          free_indices=sorted(set(out)))


def relation_einsum_plan(einsum_string: str, lhs_tile: tuple, rhs_tile: tuple) -> tuple:
    """(join_keys, agg_keys) of a two-operand einsum over tile relations.

    Every label the two operands share is a join key [(lhs_dim, rhs_dim)]:
    a pair of tiles contributes only where their coordinates agree on it.
    Each output label takes its tile coordinate from the lhs when the lhs
    carries it, else from the rhs.  The tile extents of a shared label must
    agree; a label repeated inside one operand has no tile-level join and
    raises NotImplementedError."""
    ins, out = normalize_notation(einsum_string).split("->")
    terms = ins.split(",")
    if len(terms) != 2:
        raise ValueError(f"the sparse einsum takes exactly two operands: '{einsum_string}'")
    a, b = terms
    for t in (a, b):
        if len(set(t)) != len(t):
            raise NotImplementedError(f"label repeated inside one operand ('{t}') has no "
                                      "tile-level join")
    join = []
    for i, lab in enumerate(a):
        j = b.find(lab)
        if j >= 0:
            if lhs_tile[i] != rhs_tile[j]:
                raise ValueError(f"label '{lab}' has tile extent {lhs_tile[i]} on the lhs and "
                                 f"{rhs_tile[j]} on the rhs")
            join.append((i, j))
    agg = [(0, a.index(c)) if c in a else (1, b.index(c)) for c in out]
    return join, agg


def einsum(einsum_string: str, *operands: Any, num_devices=None, mesh=None, mesh_shape=None,
           gather: bool = False, **kwargs):
    """Einstein summation (reference signature: api.py:89-200).

    Extension of the reference: two ``SparseTensorRelation`` operands run
    the sparse path, ``execute_sparse`` with join keys and output
    coordinates derived from the labels (``relation_einsum_plan``), and give
    a SparseTensorRelation.  Extra keyword arguments (``fused``,
    ``out_dtype``) go to ``execute_sparse``.  Dense operands raise
    NotImplementedError: the dense path is not part of this library.  One
    GPU only: ``num_devices`` / ``mesh`` / ``mesh_shape`` asking for more
    raise NotImplementedError; ``gather`` has no effect on one device."""
    einsum_string = normalize_notation(einsum_string)
    if not operands or not all(isinstance(op, SparseTensorRelation) for op in operands):
        raise NotImplementedError("dense einsum is not implemented by einjax_amd; pass "
                                  "SparseTensorRelation operands (SparseTensor.to_relation)")
    shapes = [op.shape for op in operands]
    validate_inputs(einsum_string, shapes)
    n_dev = num_devices
    if mesh is not None:
        n_dev = int(np.prod(getattr(mesh, "devices", np.empty(1)).shape))
    elif mesh_shape is not None:
        n_dev = int(np.prod(mesh_shape))
    if n_dev is not None and n_dev > 1:
        raise NotImplementedError("multi-device sparse execution is not part of this library: "
                                  "run one process per GPU")
    lhs, rhs = operands
    join, agg = relation_einsum_plan(einsum_string, lhs.tile_shape, rhs.tile_shape)
    return execute_sparse(lhs, rhs, join, einsum_string, agg, **kwargs)
