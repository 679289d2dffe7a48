"""Kernel dispatch registry (reference: kernels/registry.py).

Same matching rules and priorities as the reference (pattern "*" matches
anything, backend "generic" matches any backend and "gpu" matches
"gpu:<variant>", highest priority wins, ValueError when nothing matches).
The sparse builtins are this library's GPU kernels; a caller-registered
KernelInfo of higher priority replaces them, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

from ..execution.sparse_dispatch import execute_sparse
from .block_sparse import block_sparse_matmul_generic


@dataclass
class KernelInfo:
    """reference: registry.py:27-45."""

    name: str
    pattern: str
    backend: str
    sparsity: str
    priority: int
    kernel_fn: Callable[..., Any]


def execute_dense_einsum(*args, **kwargs):
    """Dense einsum entry of the registry.  The dense path (reference:
    execution/dense_kernels.py) is outside this library, which implements
    the tensor-relational sparse path only."""
    raise NotImplementedError("dense einsum is not implemented by einjax_amd; "
                              "use sparsity='sparse' relations")


class KernelRegistry:
    """reference: registry.py:48-223."""

    def __init__(self) -> None:
        self._kernels: list[KernelInfo] = []
        self._register_builtins()

    def _register_builtins(self) -> None:
        self.register(KernelInfo("generic_sparse_matmul", "ij,jk->ik", "generic", "sparse", 0,
                                 block_sparse_matmul_generic))
        self.register(KernelInfo("generic_sparse_einsum", "*", "generic", "sparse", -1,
                                 execute_sparse))
        self.register(KernelInfo("generic_dense_einsum", "*", "generic", "dense", 0,
                                 execute_dense_einsum))

    def register(self, kernel: KernelInfo) -> None:
        self._kernels.append(kernel)

    def lookup(self, pattern: str, backend: str | None = None, sparsity: str = "dense"):
        return self.lookup_info(pattern, backend, sparsity).kernel_fn

    def lookup_info(self, pattern: str, backend: str | None = None,
                    sparsity: str = "dense") -> KernelInfo:
        if backend is None:
            backend = _detect_backend()
        cands = self._find_candidates(pattern, backend, sparsity)
        if not cands:
            raise ValueError(f"No kernel found for pattern={pattern!r}, backend={backend!r}, "
                             f"sparsity={sparsity!r}")
        cands.sort(key=lambda k: k.priority, reverse=True)
        return cands[0]

    def list_kernels(self, pattern=None, backend=None, sparsity=None) -> list:
        out = list(self._kernels)
        if pattern is not None:
            out = [k for k in out if k.pattern == pattern or k.pattern == "*"]
        if backend is not None:
            out = [k for k in out if _backend_matches(k.backend, backend)]
        if sparsity is not None:
            out = [k for k in out if k.sparsity == sparsity or k.sparsity == "any"]
        return out

    def _find_candidates(self, pattern, backend, sparsity) -> list:
        return [k for k in self._kernels
                if _pattern_matches(k.pattern, pattern) and _backend_matches(k.backend, backend)
                and _sparsity_matches(k.sparsity, sparsity)]


def _detect_backend() -> str:
    """"gpu" when a ROCm GPU is visible, else "cpu" (reference:
    registry.py:226-242 reports JAX's platform; ROCm maps to "gpu")."""
    try:
        import torch

        if torch.cuda.is_available():
            return "gpu"
    except Exception:  # pragma: no cover
        pass
    return "cpu"


def _pattern_matches(registered: str, query: str) -> bool:
    return registered == "*" or registered == query


def _backend_matches(registered: str, query: str) -> bool:
    return registered == "generic" or registered == query or query.startswith(registered + ":")


def _sparsity_matches(registered: str, query: str) -> bool:
    return registered == "any" or registered == query
