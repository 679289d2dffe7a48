"""Differentiable sparse einsum (reference: autodiff/__init__.py).

Gradients flow through tile values only; coordinates and matched pair
indices are static structure.  The backward runs in libejhip.so
(ej_pair_einsum_vjp).
"""

from .custom_vjp import sparse_einsum, sparse_einsum_raw, sparse_einsum_raw_vjp

__all__ = ["sparse_einsum", "sparse_einsum_raw", "sparse_einsum_raw_vjp"]
