"""Differentiable sparse tile-pair einsum (reference: autodiff/custom_vjp.py).

The reference registers a jax.custom_vjp rule (custom_vjp.py:204-278).  JAX
is not part of this build: ``sparse_einsum_raw`` on GPU torch tensors is a
``torch.autograd.Function``, so ``torch.autograd.grad`` / ``.backward()``
take the place of ``jax.grad``, and its backward is one library call,
``ej_pair_einsum_vjp``.  ``sparse_einsum_raw_vjp`` exposes that backward
directly, for callers that drive their own differentiation (a JAX
custom_vjp rule binding the C entry point through its FFI, say).

Gradients are first order: the backward is a kernel call, not itself
differentiable.
"""

from __future__ import annotations

import numpy as np

from .. import _device
from ..execution.sparse_dispatch import (
    _add_batch_dim,
    _infer_output_tile_shape,
    execute_sparse,
    kernel_einsum,
)
from ..tensor.sparse import SparseTensorRelation, _is_torch


def _reverse_einsum_string(kernel_string: str) -> tuple[str, str]:
    """Einsum strings of the two gradients (reference: custom_vjp.py:31-62):
    for "A,B->C" the lhs gradient contracts the output cotangent with the rhs,
    "C,B->A", and the rhs gradient the lhs with the cotangent, "A,C->B".
    Raises ValueError without "->"."""
    if "->" not in kernel_string:
        raise ValueError(f"kernel_string must contain '->': {kernel_string}")
    operands, out = kernel_string.split("->")
    a, b = operands.split(",")[:2]
    return f"{out},{b}->{a}", f"{a},{out}->{b}"


def sparse_einsum(lhs: SparseTensorRelation, rhs: SparseTensorRelation, join_keys,
                  kernel_string: str, agg_keys, output_shape=None,
                  output_tile_shape=None) -> SparseTensorRelation:
    """Join, per-pair tile einsum and segment sum of two relations
    (reference: custom_vjp.py:124-201, whose forward is execute_sparse's)."""
    return execute_sparse(lhs, rhs, join_keys, kernel_string, agg_keys,
                          output_shape=output_shape, output_tile_shape=output_tile_shape)


def _torch_pair_einsum():
    import torch

    class _PairEinsum(torch.autograd.Function):
        """out[p] = einsum(kernel_string, lhs[li[p]], rhs[ri[p]]) in the values'
        dtype (float32, or bfloat16 for bfloat16 values)."""

        @staticmethod
        def forward(ctx, lhs_values, rhs_values, li, ri, kernel_string):
            ctx.kernel_string = kernel_string
            ctx.save_for_backward(lhs_values, rhs_values, li, ri)
            return kernel_einsum(lhs_values.detach(), rhs_values.detach(), li, ri, kernel_string)

        @staticmethod
        @torch.autograd.function.once_differentiable
        def backward(ctx, g):
            lhs_values, rhs_values, li, ri = ctx.saved_tensors
            gl, gr = sparse_einsum_raw_vjp(lhs_values, rhs_values, li, ri, ctx.kernel_string, g,
                                           need_lhs=ctx.needs_input_grad[0],
                                           need_rhs=ctx.needs_input_grad[1])
            return gl, gr, None, None, None

    return _PairEinsum


_PAIR_EINSUM = None


def sparse_einsum_raw(lhs_values, rhs_values, lhs_coords, rhs_coords, lhs_indices, rhs_indices,
                      kernel_string: str):
    """Per-pair tile einsum [P, *out_tile], differentiable in the tile values
    (reference: custom_vjp.py:204-278).  Coordinates and indices are static.

    GPU torch values give a GPU tensor of the values' dtype (float32, or
    bfloat16 for bfloat16 values, as the reference's jnp.einsum returns) that
    torch.autograd differentiates (gradients in the values' dtypes); host
    NumPy values give a NumPy result (no gradient tracking; use
    sparse_einsum_raw_vjp)."""
    global _PAIR_EINSUM
    _add_batch_dim(kernel_string)  # the reference's ValueError for a missing "->"
    if not (_is_torch(lhs_values) and _is_torch(rhs_values)):
        return kernel_einsum(lhs_values, rhs_values, lhs_indices, rhs_indices, kernel_string)
    import torch

    dev = _device.require_gpu()
    li = (lhs_indices if _is_torch(lhs_indices) else
          torch.from_numpy(np.asarray(lhs_indices, dtype=np.int64))).to(dev, torch.int64)
    ri = (rhs_indices if _is_torch(rhs_indices) else
          torch.from_numpy(np.asarray(rhs_indices, dtype=np.int64))).to(dev, torch.int64)
    if _PAIR_EINSUM is None:
        _PAIR_EINSUM = _torch_pair_einsum()
    return _PAIR_EINSUM.apply(lhs_values, rhs_values, li, ri, kernel_string)


def sparse_einsum_raw_vjp(lhs_values, rhs_values, lhs_indices, rhs_indices, kernel_string: str,
                          grad_out, need_lhs: bool = True, need_rhs: bool = True):
    """(grad_lhs, grad_rhs) of sparse_einsum_raw for the cotangent grad_out
    [P, *out_tile] (reference: the _bwd rule, custom_vjp.py:254-275): per-pair
    gradient einsums with the reversed strings, summed per operand tile in
    ascending pair order, in fp32.  Gradients have the values' shapes and
    dtypes; tiles no pair touches get zeros.  bfloat16 values with a bfloat16
    cotangent run the gradient einsums on bfloat16 operands (the reference's
    dtypes); any other cotangent is taken in float32.  Host inputs give host
    results."""
    import torch

    host = not (_is_torch(lhs_values) and lhs_values.is_cuda)
    dev = _device.require_gpu()

    def to_dev(x, dtype=None):
        t = x if _is_torch(x) else torch.from_numpy(np.ascontiguousarray(x))
        return t.to(device=dev, dtype=dtype or t.dtype).contiguous()

    lv, rv = to_dev(lhs_values), to_dev(rhs_values)
    out_dtypes = (lv.dtype, rv.dtype)
    if lv.dtype == torch.bfloat16 and rv.dtype == torch.bfloat16:
        pass
    else:
        lv, rv = lv.to(torch.float32), rv.to(torch.float32)
    li, ri = to_dev(lhs_indices, torch.int64), to_dev(rhs_indices, torch.int64)
    bf16 = lv.dtype == torch.bfloat16 and _is_torch(grad_out) and grad_out.dtype == torch.bfloat16
    g = to_dev(grad_out, None if bf16 else torch.float32)
    P = li.numel()
    out_tile = _infer_output_tile_shape(kernel_string, tuple(lv.shape[1:]), tuple(rv.shape[1:]))
    if tuple(g.shape) != (P, *out_tile):
        raise ValueError(f"grad_out has shape {tuple(g.shape)}, expected {(P, *out_tile)}")
    gl, gr = _device.pair_einsum_vjp(kernel_string, lv, rv, li, ri, g, need_lhs, need_rhs)
    gl = gl.to(out_dtypes[0]) if gl is not None else None
    gr = gr.to(out_dtypes[1]) if gr is not None else None
    if host:
        to_np = (lambda t: None if t is None else
                 (t.float() if t.dtype == torch.bfloat16 else t).cpu().numpy())
        return to_np(gl), to_np(gr)
    return gl, gr
