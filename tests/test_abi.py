"""The C-ABI library: loads, exports every declared symbol, and its
host-only logic (kernel-string description, workspace sizing, argument
validation) behaves as documented.  No GPU work is launched here."""

import ctypes
import re
from pathlib import Path

import pytest

from einjax_amd import _lib
from einjax_amd._lib import EinsumDesc, i32_array, i64_array

HEADER = Path(__file__).resolve().parent.parent / "include" / "einjax_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(ej_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version():
    assert _lib.load().ej_version() == 14


def describe(spec, lt, rt):
    d = EinsumDesc()
    st = _lib.load().ej_einsum_describe(spec.encode(), i64_array(lt), len(lt), i64_array(rt),
                                        len(rt), ctypes.byref(d))
    return st, d


@pytest.mark.parametrize("spec,lt,rt,gemm", [
    ("ij,jk->ik", (128, 128), (128, 128), (1, 128, 128, 128, 0, 128, 1, 0, 128, 1, 0, 128, 1)),
    ("bij,bjk->bik", (1, 64, 64), (1, 64, 64), (1, 64, 64, 64, 0, 64, 1, 0, 64, 1, 0, 64, 1)),
    ("ijk,kl->ijl", (32, 32, 32), (32, 32), (1, 1024, 32, 32, 0, 32, 1, 0, 32, 1, 0, 32, 1)),
    ("ij,kj->ik", (32, 16), (64, 16), (1, 32, 64, 16, 0, 16, 1, 0, 1, 16, 0, 64, 1)),
    ("ji,jk->ik", (16, 32), (16, 64), (1, 32, 64, 16, 0, 1, 32, 0, 64, 1, 0, 64, 1)),
    ("bij,bjk->bik", (4, 32, 16), (4, 16, 8), (4, 32, 8, 16, 512, 16, 1, 128, 8, 1, 256, 8, 1)),
])
def test_describe_gemm_forms(spec, lt, rt, gemm):
    st, d = describe(spec, lt, rt)
    assert st == 0
    assert d.is_gemm == 1
    got = (d.batch, d.m, d.n, d.k, d.a_sb, d.a_sm, d.a_sk, d.b_sb, d.b_sk, d.b_sn, d.c_sb,
           d.c_sm, d.c_sn)
    assert got == gemm


@pytest.mark.parametrize("spec,lt,rt,n_out,n_red,c_elems,gemm", [
    ("i,j->ij", (3,), (4,), 2, 0, 12, 1),
    ("i,i->", (5,), (5,), 0, 1, 1, 1),
    ("ij,ij->ij", (3, 4), (3, 4), 2, 0, 12, 1),
    ("ii,ij->j", (3, 3), (3, 4), 1, 1, 4, 0),
    ("ij,kl->ij", (1, 1), (1, 1), 2, 2, 1, 0),
    ("ik,kj->ji", (4, 5), (5, 6), 2, 1, 24, 1),   # GEMM with a transposed output
    ("ijk,jl->il", (2, 3, 4), (3, 5), 2, 2, 10, 0),  # k contracted on one side only
])
def test_describe_general_forms(spec, lt, rt, n_out, n_red, c_elems, gemm):
    st, d = describe(spec, lt, rt)
    assert st == 0
    assert (d.n_out, d.n_red, d.c_elems, d.is_gemm) == (n_out, n_red, c_elems, gemm)
    if spec == "ik,kj->ji":
        assert (d.m, d.n, d.k, d.c_sm, d.c_sn) == (4, 6, 5, 1, 4)


@pytest.mark.parametrize("spec,lt,rt,status", [
    ("ij,jk", (2, 2), (2, 2), _lib.EJ_E_INVAL),          # no "->"
    ("ij,jk,kl->il", (2, 2), (2, 2), _lib.EJ_E_INVAL),   # three operands
    ("ij,jk->iq", (2, 2), (2, 2), _lib.EJ_E_INVAL),      # unknown output label
    ("ij,jk->ik", (2, 3), (4, 2), _lib.EJ_E_INVAL),      # extent mismatch
    ("ij,jk->ii", (2, 2), (2, 2), _lib.EJ_E_INVAL),      # repeated output label
    ("ij,jk->ik", (2, 2, 2), (2, 2), _lib.EJ_E_INVAL),   # rank mismatch
    ("...j,jk->...k", (2, 2), (2, 2), _lib.EJ_E_UNSUPPORTED),
])
def test_describe_errors(spec, lt, rt, status):
    st, _ = describe(spec, lt, rt)
    assert st == status
    assert _lib.load().ej_last_error()


def test_workspace_sizes_grow_with_input():
    lib = _lib.load()
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.ej_join_workspace_size(10, 10, 0, ctypes.byref(a)) == 0
    assert lib.ej_join_workspace_size(100000, 100000, 0, ctypes.byref(b)) == 0
    assert b.value > a.value > 0
    assert lib.ej_join_workspace_size(1, 1, 7, ctypes.byref(a)) == _lib.EJ_E_INVAL
    assert lib.ej_segment_workspace_size(1000, ctypes.byref(a)) == 0 and a.value > 8000
    assert lib.ej_bucket_workspace_size(2, i64_array([8, 8]), i64_array([2, 4]),
                                        ctypes.byref(a)) == 0
    assert lib.ej_bucket_workspace_size(2, i64_array([8, 8]), i64_array([3, 4]),
                                        ctypes.byref(a)) == _lib.EJ_E_INVAL


def test_join_count_host_paths():
    """Cross products and empty sides are sized on the host (no device work)."""
    lib = _lib.load()
    n = ctypes.c_int64(-1)
    st = lib.ej_join_count(None, 7, 2, None, 5, 2, 0, None, None, None, 0, None, 0,
                           ctypes.byref(n), None)
    assert st == 0 and n.value == 35
    st = lib.ej_join_count(None, 0, 2, None, 5, 2, 1, i32_array([1]), i32_array([0]),
                           i64_array([4]), 0, None, 0, ctypes.byref(n), None)
    assert st == 0 and n.value == 0
    # a key dim outside the coordinate rank is rejected before any device work
    st = lib.ej_join_count(None, 3, 2, None, 5, 2, 1, i32_array([2]), i32_array([0]),
                           i64_array([4]), 0, None, 0, ctypes.byref(n), None)
    assert st == _lib.EJ_E_INVAL


def test_fill_capacity_error():
    lib = _lib.load()
    st = lib.ej_join_fill(3, 4, 0, 0, None, 0, 12, None, None, 11, None)
    assert st == _lib.EJ_E_CAPACITY
    assert b"capacity" in lib.ej_last_error()
    st = lib.ej_segment_fill(10, 5, 2, i64_array([4, 4]), None, 0, None, None, None, None, 4,
                             None)
    assert st == _lib.EJ_E_CAPACITY


def test_key_space_overflow_is_unsupported():
    lib = _lib.load()
    n = ctypes.c_int64()
    big = i64_array([1 << 40, 1 << 40])
    # pointers are never dereferenced: the key-space check fails first
    fake = ctypes.c_void_p(16)
    st = lib.ej_join_count(fake, 1, 2, fake, 1, 2, 2, i32_array([0, 1]), i32_array([0, 1]), big,
                           0, None, 0, ctypes.byref(n), None)
    assert st == _lib.EJ_E_UNSUPPORTED


def test_coords_range_empty_is_host_only():
    lib = _lib.load()
    lo_hi = (ctypes.c_int32 * 4)()
    assert lib.ej_coords_range(None, 0, 2, lo_hi, None, 0, None) == 0
    assert list(lo_hi) == [0, -1, 0, -1]


def test_error_status_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.EJ_E_INVAL, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.EJ_E_UNSUPPORTED, "x")
    with pytest.raises(_lib.CapacityError):
        _lib.check(_lib.EJ_E_CAPACITY, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.EJ_E_HIP, "x")


def test_scheme_stats_workspace_and_validation():
    lib = _lib.load()
    shape = i64_array([16, 12])
    shapes = [(a, b) for a in (1, 2, 4, 8, 16) for b in (1, 2, 3, 4, 6, 12)]
    flat = i64_array([t for ts in shapes for t in ts])
    dense, coo_map, coo_sort = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.ej_scheme_stats_workspace_size(2, shape, len(shapes), flat, -1, 0,
                                              ctypes.byref(dense)) == 0
    # the finest occupancy map alone is 16 * 12 bytes
    assert dense.value >= 192
    assert lib.ej_scheme_stats_workspace_size(2, shape, len(shapes), flat, 1000, 0,
                                              ctypes.byref(coo_map)) == 0
    # a cap of 8 cells sends the finer tile shapes to the sort path: key buffers
    assert lib.ej_scheme_stats_workspace_size(2, shape, len(shapes), flat, 1000, 8,
                                              ctypes.byref(coo_sort)) == 0
    assert coo_sort.value > coo_map.value + 16 * 1000
    bad = i64_array([16, 5])
    assert lib.ej_scheme_stats_workspace_size(2, shape, 1, bad, -1, 0,
                                              ctypes.byref(dense)) == _lib.EJ_E_INVAL
    assert lib.ej_scheme_stats_workspace_size(2, i64_array([0, 4]), 1, i64_array([1, 1]), -1, 0,
                                              ctypes.byref(dense)) == _lib.EJ_E_INVAL


def test_scheme_stats_coo_without_entries_is_host_only():
    lib = _lib.load()
    nt = (ctypes.c_int64 * 2)(7, 7)
    vc = (ctypes.c_int64 * 4)(7, 7, 7, 7)
    st = lib.ej_scheme_stats_coo(None, None, _lib.EJ_F64, 0, 2, i64_array([4, 4]), 2,
                                 i64_array([1, 1, 2, 4]), 0, None, 0, nt, vc, None)
    assert st == 0 and list(nt) == [0, 0] and list(vc) == [0, 0, 0, 0]


def test_coo_calls_host_paths():
    lib = _lib.load()
    n = ctypes.c_int64(-1)
    a = ctypes.c_size_t()
    assert lib.ej_extract_coo_count(None, _lib.EJ_F32, 2, i64_array([0, 5]), None, 0,
                                    ctypes.byref(n), None) == 0 and n.value == 0
    assert lib.ej_extract_coo_count(None, 9, 2, i64_array([2, 5]), None, 0, ctypes.byref(n),
                                    None) == _lib.EJ_E_INVAL
    assert lib.ej_extract_coo_workspace_size(2, i64_array([1024, 1024]), _lib.EJ_BF16,
                                             ctypes.byref(a)) == 0 and a.value > 0
    n.value = -1
    assert lib.ej_bucket_coo_count(None, None, _lib.EJ_F64, 0, 2, i64_array([4, 4]),
                                   i64_array([2, 2]), None, 0, ctypes.byref(n), None) == 0
    assert n.value == 0
    assert lib.ej_bucket_coo_count(None, None, _lib.EJ_F64, 3, 2, i64_array([4, 4]),
                                   i64_array([3, 2]), None, 0, ctypes.byref(n),
                                   None) == _lib.EJ_E_INVAL
    sh, ts = i64_array([64, 64]), i64_array([4, 4])
    assert lib.ej_bucket_coo_workspace_size(1 << 31, _lib.EJ_F64, 2, sh, ts,
                                            ctypes.byref(a)) == _lib.EJ_E_INVAL
    # bf16 values: sorted path, workspace grows with the entries
    assert lib.ej_bucket_coo_workspace_size(1000, _lib.EJ_BF16, 2, sh, ts,
                                            ctypes.byref(a)) == 0 and a.value > 32000
    # fp32 tiles: occupancy-map path, workspace follows the 256-tile grid
    assert lib.ej_bucket_coo_workspace_size(1000, _lib.EJ_F64, 2, sh, ts,
                                            ctypes.byref(a)) == 0 and a.value < 8192
    assert lib.ej_bucket_coo_fill(None, None, _lib.EJ_F32, 10, 2, i64_array([4, 4]),
                                  i64_array([2, 2]), None, 0, 3, None, None, 2,
                                  None) == _lib.EJ_E_CAPACITY
    assert lib.ej_extract_coo_fill(None, _lib.EJ_F32, 2, i64_array([4, 4]), None, 0, 5, None,
                                   None, 4, None) == _lib.EJ_E_CAPACITY


def test_backward_host_validation():
    lib = _lib.load()
    a = ctypes.c_size_t()
    assert lib.ej_index_plan_workspace_size(1000, ctypes.byref(a)) == 0 and a.value > 16000
    F32, BF16 = _lib.EJ_F32, _lib.EJ_BF16
    assert lib.ej_pair_einsum_vjp_workspace_size(100, 10, 10, 64, 64, BF16, F32,
                                                 ctypes.byref(a)) == 0
    bf = a.value
    assert lib.ej_pair_einsum_vjp_workspace_size(100, 10, 10, 64, 64, F32, F32,
                                                 ctypes.byref(a)) == 0
    assert bf >= a.value + 4 * 64 * 20  # bf16 operands under an fp32 cotangent are widened
    assert lib.ej_pair_einsum_vjp_workspace_size(100, 10, 10, 64, 64, BF16, BF16,
                                                 ctypes.byref(a)) == 0
    assert a.value < bf  # a bf16 cotangent needs no widened operands
    # bf16 gradients need bf16 operands
    assert lib.ej_pair_einsum_vjp_workspace_size(100, 10, 10, 64, 64, F32, BF16,
                                                 ctypes.byref(a)) == _lib.EJ_E_INVAL
    t = i64_array([2, 2])
    fake = ctypes.c_void_p(16)
    # "ij,jk->k": the lhs gradient string "k,jk->ij" names i, found in no operand
    st = lib.ej_pair_einsum_vjp(b"ij,jk->k", t, 2, t, 2, F32, fake, 1, fake, 1, fake,
                                fake, 1, F32, fake, fake, None, None, 0, None)
    assert st == _lib.EJ_E_INVAL and b"gradient string" in lib.ej_last_error()
    st = lib.ej_pair_einsum_vjp(b"ij,jk", t, 2, t, 2, F32, fake, 1, fake, 1, fake,
                                fake, 1, F32, fake, fake, None, None, 0, None)
    assert st == _lib.EJ_E_INVAL
    st = lib.ej_pair_einsum_vjp(b"ij,jk->ik", t, 2, t, 2, F32, fake, 1, fake, 1, fake,
                                fake, 1, BF16, fake, fake, None, None, 0, None)
    assert st == _lib.EJ_E_INVAL and b"gradient dtype" in lib.ej_last_error()


def test_output_dtype_validation():
    """Descriptors start with fp32 outputs; bf16 outputs need bf16 operands
    (checked before any launch, so no GPU is needed)."""
    lib = _lib.load()
    st, d = describe("ij,jk->ik", (32, 32), (32, 32))
    assert st == 0 and d.out_dtype == _lib.EJ_F32
    d.out_dtype = _lib.EJ_BF16
    fake = ctypes.c_void_p(16)
    st = lib.ej_segment_einsum(ctypes.byref(d), _lib.EJ_F32, fake, fake, 1, 1, None, None, None,
                               fake, 0, fake, None)
    assert st == _lib.EJ_E_INVAL and b"output dtype" in lib.ej_last_error()
    assert lib.ej_segment_einsum(ctypes.byref(d), _lib.EJ_BF16, fake, fake, 1, 1, None, None,
                                 None, fake, 0, fake, None) == _lib.EJ_OK
    d.out_dtype = 7
    assert lib.ej_pair_einsum(ctypes.byref(d), _lib.EJ_BF16, fake, fake, 1, 1, None, None, 0,
                              fake, None) == _lib.EJ_E_INVAL
    assert lib.ej_segment_sum(fake, 9, 4, fake, fake, 0, fake, None) == _lib.EJ_E_INVAL
    for code in (_lib.EJ_BF16, _lib.EJ_F32, _lib.EJ_F64, _lib.EJ_F16, _lib.EJ_I32, _lib.EJ_I64):
        assert lib.ej_segment_sum(fake, code, 4, fake, fake, 0, fake, None) == _lib.EJ_OK
    # int32 tiles give int32 results and only int32 tiles do
    d.out_dtype = _lib.EJ_F32
    assert lib.ej_pair_einsum(ctypes.byref(d), _lib.EJ_I32, fake, fake, 1, 1, None, None, 0,
                              fake, None) == _lib.EJ_E_INVAL
    d.out_dtype = _lib.EJ_I32
    assert lib.ej_pair_einsum(ctypes.byref(d), _lib.EJ_I32, fake, fake, 1, 1, None, None, 0,
                              fake, None) == _lib.EJ_OK
    assert lib.ej_pair_einsum(ctypes.byref(d), _lib.EJ_F32, fake, fake, 1, 1, None, None, 0,
                              fake, None) == _lib.EJ_E_INVAL
    g = ctypes.c_int32(0)
    assert lib.ej_segment_einsum_group(ctypes.byref(d), _lib.EJ_I32, ctypes.byref(g)) == 0
    assert g.value == 1


def test_pair_plan_host_validation():
    """The queued pair plan rejects what it does not cover before any launch."""
    lib = _lib.load()
    fake = ctypes.c_void_p(16)
    d = i32_array([1])
    r = i64_array([4])
    counts = (ctypes.c_int64 * 8)()
    args = lambda nk, cap: (fake, 4, 2, fake, 4, 2, nk, d, i32_array([0]), r, 2, i32_array([0, 1]),
                            i32_array([0, 1]), i64_array([4, 4]), cap, fake, 1 << 20, fake, 1 << 20,
                            fake, fake, fake, fake, fake, 16, 0, None, None,
                            ctypes.cast(counts, ctypes.c_void_p), 0, None)
    assert lib.ej_pair_plan_async(*args(0, 10)) == _lib.EJ_E_INVAL  # no join keys
    assert lib.ej_pair_plan_async(*args(1, 0)) == _lib.EJ_E_INVAL  # no capacity
    assert b"pair_capacity" in lib.ej_last_error()


def test_pair_plan_noalloc_host_validation():
    """The allocation-free plan checks its arguments and its scratch limit
    (64 MiB) on the host, before it looks up the scratch or launches
    anything: a request beyond the limit gets EJ_E_CAPACITY here, where no
    GPU is visible."""
    lib = _lib.load()
    fake = ctypes.c_void_p(16)
    d = i32_array([1])
    counts = (ctypes.c_int64 * 8)()
    args = lambda nl, cap: (fake, nl, 2, fake, 4, 2, 1, d, i32_array([0]), i64_array([4]), 2,
                            i32_array([0, 1]), i32_array([0, 1]), i64_array([4, 4]), cap, fake,
                            fake, fake, fake, fake, 16, 0, None, None,
                            ctypes.cast(counts, ctypes.c_void_p), 0, None)
    assert lib.ej_pair_plan_async_noalloc(*args(4, 2_000_000)) == _lib.EJ_E_CAPACITY
    assert b"static scratch" in lib.ej_last_error()
    assert lib.ej_pair_plan_async_noalloc(*args(4, 0)) == _lib.EJ_E_INVAL
    assert lib.ej_pair_plan_async_noalloc(*args(0, 10)) == _lib.EJ_E_INVAL


def test_dense_plan_host_validation():
    """The dense-rhs plan decides from the join's structure, on the host,
    whether it applies (EJ_E_UNSUPPORTED otherwise) and checks capacities
    before anything is launched."""
    lib = _lib.load()
    fake = ctypes.c_void_p(16)
    counts = (ctypes.c_int64 * 8)()

    def call(keys, agg, lncols=2, rncols=2, n_lhs=4, n_rhs=16, lgrid=(4, 4), rgrid=(4, 4),
             cap=10 ** 6):
        return lib.ej_dense_plan_async(
            fake, n_lhs, lncols, fake, n_rhs, rncols, len(keys),
            i32_array([a for a, _ in keys]), i32_array([b for _, b in keys]), i64_array(lgrid),
            i64_array(rgrid), len(agg), i32_array([a for a, _ in agg]),
            i32_array([b for _, b in agg]), fake, fake, cap, fake, fake, cap, 0, None, None, fake,
            ctypes.cast(counts, ctypes.c_void_p), 0, None)

    mm = ([(1, 0)], [(0, 0), (1, 1)])
    assert call([(1, 1)], mm[1]) == _lib.EJ_E_UNSUPPORTED      # join on rhs dim 1
    assert call(mm[0], [(1, 1), (0, 0)]) == _lib.EJ_E_UNSUPPORTED  # output not lhs-first
    assert call(mm[0], [(0, 0)]) == _lib.EJ_E_UNSUPPORTED      # rhs free dim dropped
    assert call(mm[0], mm[1], n_rhs=15) == _lib.EJ_E_UNSUPPORTED  # rhs not the full grid
    assert call(mm[0], mm[1], n_lhs=16385) == _lib.EJ_E_UNSUPPORTED  # beyond 16384 lhs tiles
    assert call([(0, 0)], [(0, 0), (1, 1)]) == _lib.EJ_E_UNSUPPORTED  # lhs dim 1 not joined
    assert call(mm[0], mm[1], cap=15) == _lib.EJ_E_CAPACITY     # 4 x 4 pairs
    # a rhs grid of 2^32 tiles, and 2^31 pairs: beyond the plan's 32-bit indices
    assert call(mm[0], mm[1], n_rhs=1 << 32, rgrid=(1 << 16, 1 << 16)) == _lib.EJ_E_UNSUPPORTED
    assert call(mm[0], mm[1], n_lhs=16384, lgrid=(4096, 4), n_rhs=4 << 17,
                rgrid=(4, 1 << 17)) == _lib.EJ_E_UNSUPPORTED
    # two join keys whose lhs dims run against the rhs order
    assert call([(2, 0), (1, 1)], [(0, 0), (1, 2)], lncols=3, rncols=3, lgrid=(2, 2, 2),
                rgrid=(2, 2, 2), n_rhs=8) == _lib.EJ_E_UNSUPPORTED


def test_dense_plan_applies_mirrors_the_library():
    from einjax_amd import _device as D

    assert D.dense_plan_applies(819, 2, 2, [(1, 0)], [(0, 0), (1, 1)])
    assert D.dense_plan_applies(15488, 3, 3, [(0, 0), (2, 1)], [(0, 0), (0, 1), (1, 2)])
    assert D.dense_plan_applies(1311, 3, 2, [(2, 0)], [(0, 0), (0, 1), (1, 1)])
    assert not D.dense_plan_applies(819, 2, 2, [(1, 1)], [(0, 0), (1, 1)])
    assert not D.dense_plan_applies(16385, 2, 2, [(1, 0)], [(0, 0), (1, 1)])
    assert not D.dense_plan_applies(10, 2, 2, [(0, 0)], [(0, 0), (1, 1)])
    assert not D.dense_plan_applies(10, 3, 3, [(2, 0), (1, 1)], [(0, 0), (1, 2)])


def test_segment_einsum_group():
    """The group size a run order is made for: two 128 x 128 bf16 output
    tiles per workgroup, four 64 x 64 bf16 or fp32 ones, 1 without the
    seg_group hint or for shapes and layouts the grouped kernels do not take."""
    lib = _lib.load()

    def group(spec, lt, rt, dtype, hint=4):
        st, d = describe(spec, lt, rt)
        assert st == _lib.EJ_OK
        d.seg_group = hint
        g = ctypes.c_int32(-1)
        assert lib.ej_segment_einsum_group(ctypes.byref(d), dtype, ctypes.byref(g)) == _lib.EJ_OK
        return g.value

    assert group("ij,jk->ik", (128, 128), (128, 128), _lib.EJ_BF16) == 2
    assert group("ij,jk->ik", (64, 64), (64, 64), _lib.EJ_BF16) == 4
    assert group("ij,jk->ik", (64, 64), (64, 64), _lib.EJ_F32) == 4
    assert group("ij,jk->ik", (128, 128), (128, 128), _lib.EJ_BF16, hint=0) == 1
    # bf16 operands in either layout run grouped on the LDS ring, except a
    # [k][m] lhs with an [n][k] rhs; fp32 takes [m][k] x [k][n] only
    assert group("ij,kj->ik", (128, 128), (128, 128), _lib.EJ_BF16) == 2  # rhs k-contiguous
    assert group("ji,jk->ik", (64, 64), (64, 64), _lib.EJ_BF16) == 4     # lhs m-contiguous
    assert group("ji,kj->ik", (128, 128), (128, 128), _lib.EJ_BF16) == 1
    assert group("ij,kj->ik", (64, 64), (64, 64), _lib.EJ_F32) == 1
    st, d = describe("ij,jk->ik", (32, 32), (32, 32))
    g = ctypes.c_int32(-1)
    assert lib.ej_segment_einsum_group(ctypes.byref(d), 7, ctypes.byref(g)) == _lib.EJ_E_INVAL
    assert lib.ej_segment_einsum_group(ctypes.byref(d), _lib.EJ_F32, None) == _lib.EJ_E_INVAL


def test_plan_ticket_cycle_stays_below_the_plans_limit():
    """The queued plans take tickets 1 .. 2^30 - 1 (ej_dense_plan_async rejects
    2^30 and above); the host's ticket counter cycles inside that range."""
    from einjax_amd import _device

    t, seen = 0, set()
    for _ in range(3):
        t = _device._next_ticket(t)
        seen.add(t)
    assert seen == {1, 2, 3}
    assert _device._next_ticket((1 << 30) - 2) == (1 << 30) - 1
    assert _device._next_ticket((1 << 30) - 1) == 1


def test_row_ticket_fold():
    """The row plan's packed word holds 20 ticket bits: tickets fold to
    1 .. 2^20 - 1, never 0 (a cleared slot), consecutive ones stay distinct,
    also across the 2^30 cycle of the host counter."""
    from einjax_amd import _device

    m = (1 << 20) - 1
    assert [_device._ticket20(t) for t in (1, 2, m, m + 1, m + 2)] == [1, 2, m, 1, 2]
    t = (1 << 30) - 1
    nxt = _device._next_ticket(t)
    assert nxt == 1 and _device._ticket20(t) != _device._ticket20(nxt)
    for t in range(1, 3 * m, 997):
        f = _device._ticket20(t)
        assert 1 <= f <= m and f != _device._ticket20(_device._next_ticket(t))


def test_count_slot_cleared_before_each_plan(monkeypatch):
    """A dense plan's packed word (ticket << 33 | flag << 32 | U) for ticket
    2^20 + 510 reads as the row plan's next ticket (folded to 512) when
    shifted by 44; the host clears slot 6 before each plan, so a previous
    call's word is never taken for the next call's."""
    from einjax_amd import _device

    t_dense = (1 << 20) + 510
    t_row = _device._ticket20(_device._next_ticket(t_dense))
    stale = t_dense << 33 | 5
    assert stale >> 44 == t_row  # the collision the clearing prevents
    buf = (ctypes.c_int64 * 8)()
    buf[6] = stale
    state = _device._Counts()
    state.addr, state.view, state.ticket = ctypes.addressof(buf), buf, t_dense
    monkeypatch.setattr(_device, "_counts", state)
    addr, view, ticket = _device._count_buffer()
    assert (addr, ticket) == (ctypes.addressof(buf), t_dense + 1)
    assert view[6] == 0 and (view[6] & ((1 << 64) - 1)) >> 44 != t_row


def test_injected_host_alloc_failure(monkeypatch):
    """EJ_INJECT_FAULT=host_alloc: ej_host_alloc fails as if hipHostMalloc had
    run out of memory (EJ_E_HIP and a message), and the Python wrapper that
    takes the queued plan's count buffer raises with that message."""
    import threading

    from einjax_amd import _device

    lib = _lib.load()
    monkeypatch.setenv("EJ_INJECT_FAULT", "launch,host_alloc")
    p = ctypes.c_void_p()
    assert lib.ej_host_alloc(64, ctypes.byref(p)) == _lib.EJ_E_HIP
    msg = lib.ej_last_error()
    assert b"hipHostMalloc failed" in msg and b"injected by EJ_INJECT_FAULT" in msg
    assert p.value is None
    err = []

    def fresh_thread():  # the count buffer is per thread
        try:
            _device._count_buffer()
        except RuntimeError as e:
            err.append(str(e))

    t = threading.Thread(target=fresh_thread)
    t.start()
    t.join()
    assert err and "HIP error in ej_host_alloc" in err[0] and "injected" in err[0]
    # other site names do not match
    monkeypatch.setenv("EJ_INJECT_FAULT", "host_allocx,launch")
    lib.ej_host_alloc(64, ctypes.byref(p))
    assert b"injected" not in lib.ej_last_error()
    if p.value:
        lib.ej_host_free(p)


def test_row_plan_structure_and_arguments():
    """row_plan_applies follows the dense plan's structure with a sparse rhs
    and the row plan's limits; ej_row_plan_async and its workspace size
    refuse bad arguments and structures before any launch."""
    from einjax_amd import _device as D

    lib = _lib.load()
    assert D.row_plan_applies(5243, [512, 512], [512, 512], [(1, 0)], [(0, 0), (1, 1)])
    assert D.row_plan_applies(40, [3, 12, 10], [3, 10, 14], [(0, 0), (2, 1)],
                              [(0, 0), (0, 1), (1, 2)])
    assert not D.row_plan_applies(16385, [512, 512], [512, 512], [(1, 0)], [(0, 0), (1, 1)])
    assert not D.row_plan_applies(100, [512, 512], [512, 8193], [(1, 0)], [(0, 0), (1, 1)])
    assert not D.row_plan_applies(100, [512, 512], [65537, 4], [(1, 0)], [(0, 0), (1, 1)])
    assert not D.row_plan_applies(100, [512, 512], [512, 512], [(0, 0)], [(0, 1), (1, 1)])
    assert not D.row_plan_applies(9000, [9000, 4], [4, 4], [(1, 0)], [(0, 0), (1, 1)])
    nb = ctypes.c_size_t()
    assert lib.ej_row_plan_workspace_size(5243, 5243, 512, ctypes.byref(nb)) == _lib.EJ_OK
    assert nb.value >= 513 * 4 + 82 * 8 + 5243 * 4 + 5243 * 20
    assert lib.ej_row_plan_workspace_size(16385, 5, 512, ctypes.byref(nb)) == _lib.EJ_E_INVAL
    assert lib.ej_row_plan_workspace_size(10, 0, 512, ctypes.byref(nb)) == _lib.EJ_E_INVAL
    assert lib.ej_row_plan_workspace_size(10, 5, 65537, ctypes.byref(nb)) == _lib.EJ_E_INVAL

    def call(keys, agg, lgrid, rgrid, ticket=1, ws_bytes=1 << 20, n_lhs=4, lncols=2):
        z = ctypes.c_void_p(16)  # never dereferenced: refused before any launch
        return lib.ej_row_plan_async(
            z, n_lhs, lncols, z, 4, len(rgrid), len(keys), _lib.i32_array([k[0] for k in keys]),
            _lib.i32_array([k[1] for k in keys]), _lib.i64_array(lgrid), _lib.i64_array(rgrid),
            len(agg), _lib.i32_array([a for a, _ in agg]), _lib.i32_array([b for _, b in agg]),
            z, z, 16, z, z, 16, z, ws_bytes, z, z, ticket, None)

    assert call([(0, 0)], [(0, 1), (1, 1)], [4, 4], [4, 4]) == _lib.EJ_E_UNSUPPORTED
    assert b"row plan" in lib.ej_last_error()
    assert call([(1, 0)], [(0, 0), (1, 1)], [4, 4], [4, 9000]) == _lib.EJ_E_UNSUPPORTED
    assert call([(1, 0)], [(0, 0), (1, 1)], [4, 4], [4, 4], ticket=1 << 20) == _lib.EJ_E_INVAL
    assert call([(1, 0)], [(0, 0), (1, 1)], [4, 4], [4, 4], ws_bytes=8) == _lib.EJ_E_CAPACITY
