"""ctypes binding of libejhip.so (declared in include/einjax_hip.h).

The library is the only compute path: if it is missing, or no GPU is
visible, every entry point raises instead of falling back.  PyTorch is used
for device memory and the current HIP stream only.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libejhip.so"
# A host-side test run may load the sanitized host-only build instead
# (einjax_amd/csrc/build.py --sanitize); nothing else sets this.
if os.environ.get("EINJAX_AMD_SANITIZED_LIB"):
    LIB_PATH = Path(os.environ["EINJAX_AMD_SANITIZED_LIB"])

EJ_OK = 0
EJ_E_INVAL = -1
EJ_E_CAPACITY = -2
EJ_E_HIP = -3
EJ_E_UNSUPPORTED = -4
EJ_E_RANGE = -5

EJ_F32 = 0
EJ_BF16 = 1
EJ_F64 = 2
EJ_I32 = 3
EJ_I64 = 4
EJ_F16 = 5

EJ_ORDER_PROBE = 0
EJ_ORDER_SORTED = 1

EJ_MAX_DIMS = 8
EJ_MAX_KEYS = 8
EJ_MAX_LABELS = 8

_i32, _i64, _sz, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
_P_i32 = ctypes.POINTER(ctypes.c_int32)
_P_i64 = ctypes.POINTER(ctypes.c_int64)
_P_sz = ctypes.POINTER(ctypes.c_size_t)


class EinsumDesc(ctypes.Structure):
    """Mirror of ej_einsum_desc."""

    _fields_ = [
        ("n_out", _i32), ("n_red", _i32),
        ("out_ext", _i64 * EJ_MAX_LABELS), ("out_a", _i64 * EJ_MAX_LABELS),
        ("out_b", _i64 * EJ_MAX_LABELS), ("red_ext", _i64 * EJ_MAX_LABELS),
        ("red_a", _i64 * EJ_MAX_LABELS), ("red_b", _i64 * EJ_MAX_LABELS),
        ("a_elems", _i64), ("b_elems", _i64), ("c_elems", _i64),
        ("is_gemm", _i32), ("seg_group", _i32),
        ("batch", _i64), ("m", _i64), ("n", _i64), ("k", _i64),
        ("a_sb", _i64), ("a_sm", _i64), ("a_sk", _i64),
        ("b_sb", _i64), ("b_sk", _i64), ("b_sn", _i64),
        ("c_sb", _i64), ("c_sm", _i64), ("c_sn", _i64),
        ("out_dtype", _i32), ("reserved", _i32),
    ]


# name -> (restype, argtypes); must match include/einjax_hip.h.
SIGNATURES = {
    "ej_version": (_i32, []),
    "ej_last_error": (ctypes.c_char_p, []),
    "ej_einsum_describe": (_i32, [ctypes.c_char_p, _P_i64, _i32, _P_i64, _i32,
                                  ctypes.POINTER(EinsumDesc)]),
    "ej_join_workspace_size": (_i32, [_i64, _i64, _i32, _P_sz]),
    "ej_join_count": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32, _P_i64, _i32,
                             _vp, _sz, _P_i64, _vp]),
    "ej_join_count_async": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32,
                                   _P_i64, _i32, _vp, _sz, _vp, _vp]),
    "ej_join_fill": (_i32, [_i64, _i64, _i32, _i32, _vp, _sz, _i64, _vp, _vp, _i64, _vp]),
    "ej_output_coords": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i64, _i32, _P_i32,
                                _P_i32, _vp, _vp]),
    "ej_segment_workspace_size": (_i32, [_i64, _P_sz]),
    "ej_segment_count": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i64, _i32, _P_i32,
                                _P_i32, _P_i64, _vp, _sz, _P_i64, _vp]),
    "ej_segment_fill": (_i32, [_i64, _i64, _i32, _P_i64, _vp, _sz, _vp, _vp, _vp, _vp, _i64,
                               _vp]),
    "ej_segment_count_async": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i64, _vp,
                                      _i32, _P_i32, _P_i32, _P_i64, _vp, _sz, _vp, _vp]),
    "ej_segment_fill_async": (_i32, [_i64, _i32, _P_i64, _vp, _sz, _vp, _vp, _vp, _vp, _i64,
                                     _vp]),
    "ej_gather_tiles": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "ej_pair_einsum": (_i32, [ctypes.POINTER(EinsumDesc), _i32, _vp, _vp, _i64, _i64, _vp, _vp,
                              _i64, _vp, _vp]),
    "ej_segment_einsum": (_i32, [ctypes.POINTER(EinsumDesc), _i32, _vp, _vp, _i64, _i64, _vp,
                                 _vp, _vp, _vp, _i64, _vp, _vp]),
    "ej_segment_einsum_async": (_i32, [ctypes.POINTER(EinsumDesc), _i32, _vp, _vp, _i64, _i64,
                                       _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp]),
    "ej_segment_einsum_group": (_i32, [ctypes.POINTER(EinsumDesc), _i32, _P_i32]),
    "ej_segment_sum": (_i32, [_vp, _i32, _i64, _vp, _vp, _i64, _vp, _vp]),
    "ej_bucket_workspace_size": (_i32, [_i32, _P_i64, _P_i64, _P_sz]),
    "ej_bucket_dense_count": (_i32, [_vp, _i32, _i32, _P_i64, _P_i64, _vp, _sz, _P_i64, _vp]),
    "ej_bucket_dense_fill": (_i32, [_vp, _i32, _i32, _P_i64, _P_i64, _vp, _sz, _i64, _vp, _vp,
                                    _i64, _vp]),
    "ej_relation_to_dense": (_i32, [_vp, _vp, _i64, _i32, _i32, _P_i64, _P_i64, _vp, _vp]),
    "ej_coords_range": (_i32, [_vp, _i64, _i32, _P_i32, _vp, _sz, _vp]),
    "ej_extract_coo_workspace_size": (_i32, [_i32, _P_i64, _i32, _P_sz]),
    "ej_extract_coo_count": (_i32, [_vp, _i32, _i32, _P_i64, _vp, _sz, _P_i64, _vp]),
    "ej_extract_coo_fill": (_i32, [_vp, _i32, _i32, _P_i64, _vp, _sz, _i64, _vp, _vp, _i64,
                                   _vp]),
    "ej_bucket_coo_workspace_size": (_i32, [_i64, _i32, _i32, _P_i64, _P_i64, _P_sz]),
    "ej_bucket_coo_count": (_i32, [_vp, _vp, _i32, _i64, _i32, _P_i64, _P_i64, _vp, _sz, _P_i64,
                                   _vp]),
    "ej_bucket_coo_fill": (_i32, [_vp, _vp, _i32, _i64, _i32, _P_i64, _P_i64, _vp, _sz, _i64,
                                  _vp, _vp, _i64, _vp]),
    "ej_scheme_stats_workspace_size": (_i32, [_i32, _P_i64, _i64, _P_i64, _i64, _i64, _P_sz]),
    "ej_scheme_stats_dense": (_i32, [_vp, _i32, _i32, _P_i64, _i64, _P_i64, _vp, _sz, _P_i64,
                                     _P_i64, _vp]),
    "ej_scheme_stats_coo": (_i32, [_vp, _vp, _i32, _i64, _i32, _P_i64, _i64, _P_i64, _i64, _vp,
                                   _sz, _P_i64, _P_i64, _vp]),
    "ej_pair_plan_async": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32, _P_i64,
                                  _i32, _P_i32, _P_i32, _P_i64, _i64, _vp, _sz, _vp, _sz, _vp,
                                  _vp, _vp, _vp, _vp, _i64, _i32, _vp, _P_i32, _vp, _i32, _vp]),
    "ej_pair_plan_async_noalloc": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32,
                                          _P_i64, _i32, _P_i32, _P_i32, _P_i64, _i64, _vp, _vp,
                                          _vp, _vp, _vp, _i64, _i32, _vp, _P_i32, _vp, _i32,
                                          _vp]),
    "ej_dense_plan_async": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32,
                                   _P_i64, _P_i64, _i32, _P_i32, _P_i32, _vp, _vp, _i64, _vp,
                                   _vp, _i64, _i32, _vp, _P_i32, _vp, _vp, _i32, _vp]),
    "ej_row_plan_async": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _i32, _P_i32, _P_i32, _P_i64,
                                 _P_i64, _i32, _P_i32, _P_i32, _vp, _vp, _i64, _vp, _vp, _i64,
                                 _vp, _sz, _vp, _vp, _i32, _vp]),
    "ej_row_plan_workspace_size": (_i32, [_i64, _i64, _i64, _P_sz]),
    "ej_host_alloc": (_i32, [_sz, ctypes.POINTER(_vp)]),
    "ej_host_free": (_i32, [_vp]),
    "ej_index_plan_workspace_size": (_i32, [_i64, _P_sz]),
    "ej_index_plan": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ej_pair_einsum_vjp_workspace_size": (_i32, [_i64, _i64, _i64, _i64, _i64, _i32, _i32,
                                                 _P_sz]),
    "ej_pair_einsum_vjp": (_i32, [ctypes.c_char_p, _P_i64, _i32, _P_i64, _i32, _i32, _vp, _i64,
                                  _vp, _i64, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _sz,
                                  _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads libejhip.so and declares every signature (no GPU needed)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m einjax_amd.csrc.build` "
                    "(the sparse-einsum path has no CPU fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


class CapacityError(RuntimeError):
    """An output buffer was smaller than the size the library counted."""


class RangeError(ValueError):
    """A coordinate lies outside the radix (grid extent) it was declared
    with (status EJ_E_RANGE)."""


def check(status: int, what: str) -> None:
    if status == EJ_OK:
        return
    msg = f"{what}: {load().ej_last_error().decode(errors='replace')}"
    if status == EJ_E_RANGE:
        raise RangeError(msg)
    if status == EJ_E_INVAL:
        raise ValueError(msg)
    if status == EJ_E_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status == EJ_E_CAPACITY:
        raise CapacityError(msg)
    raise RuntimeError(f"HIP error in {msg}")


def i32_array(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int32 * max(1, len(vals)))(*vals)


def i64_array(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(1, len(vals)))(*vals)
