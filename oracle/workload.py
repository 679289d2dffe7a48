"""Algorithmic work per einsum, from sizes only (never from counters).

Test / bench infrastructure (see ``oracle/__init__.py``).  Definitions:
  F_gemm   = P * 2 * prod(all tile-einsum label extents)   (2*M*N*K per pair)
  B_join   = 8*(n_lhs + n_rhs) + 20*P   (packed keys read; int64 lhs, int64 rhs
                                          and int32 segment id written)
  B_gather = 2*P*(|tA| + |tB|)*e        (read the matched tiles, write the panel)
  B_segsum = 4*P*|tOut| + 4*U*|tOut| + 4*U*nd
  B_bucket = dense bytes read + T*|tile|*e + 4*nd*T
  B_fused  = compulsory bytes of the fused einsum: every distinct operand tile
             read once + the fp32 output tiles and their coordinates written.
"""

from __future__ import annotations

from math import prod


def label_extents(kernel_string: str, lhs_tile, rhs_tile) -> dict:
    ins, _ = kernel_string.split("->")
    a, b = ins.split(",")
    ext = {}
    for lab, e in zip(a, lhs_tile):
        ext[lab] = e
    for lab, e in zip(b, rhs_tile):
        ext[lab] = e
    return ext


def flops_gemm(kernel_string, lhs_tile, rhs_tile, n_pairs) -> float:
    return float(n_pairs) * 2.0 * prod(label_extents(kernel_string, lhs_tile, rhs_tile).values())


def bytes_join(n_lhs, n_rhs, n_pairs) -> float:
    return 8.0 * (n_lhs + n_rhs) + 20.0 * n_pairs


def bytes_gather(n_pairs, lhs_tile, rhs_tile, elem_bytes) -> float:
    return 2.0 * n_pairs * (prod(lhs_tile) + prod(rhs_tile)) * elem_bytes


def bytes_segsum(n_pairs, n_segments, out_tile, out_ndim, out_bytes=4) -> float:
    """Pair tiles read, output tiles and int32 coordinates written; out_bytes
    per value (4 fp32, 2 bf16: results keep the operands' dtype)."""
    t = prod(out_tile)
    return out_bytes * (float(n_pairs) * t + float(n_segments) * t) + 4.0 * n_segments * out_ndim


def bytes_bucket(dense_elems, n_tiles, tile, elem_bytes, ndim) -> float:
    return float(dense_elems) * elem_bytes + n_tiles * prod(tile) * elem_bytes + 4.0 * ndim * n_tiles


def bytes_fused(n_lhs_used, n_rhs_used, lhs_tile, rhs_tile, elem_bytes, n_segments, out_tile,
                out_ndim, out_bytes=4) -> float:
    """Every used operand tile read once, every output tile written once
    (out_bytes per value) plus its int32 coordinates."""
    return (float(n_lhs_used) * prod(lhs_tile) + float(n_rhs_used) * prod(rhs_tile)) * elem_bytes \
        + float(out_bytes) * n_segments * prod(out_tile) + 4.0 * n_segments * out_ndim
