"""GPU parity: every phase of the HIP path against the oracle.

Index work (joins, output coordinates, segment plans, tiling coordinates)
must be bit-exact; values must agree within rel-L2 <= 1e-5 (fp32) or
<= 1e-2 (bf16, against fp32-or-better math on the bf16-rounded inputs).
"""

import zlib

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R

import einjax_amd as ej
from einjax_amd import SparseTensor, SparseTensorRelation
from einjax_amd.execution import sparse_dispatch as sd

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 1e-2}


def note(*a):
    print("[case]", *a, flush=True)


def dev_rel(r: R.Rel, dtype="fp32", device="cuda"):
    """Oracle relation -> device SparseTensorRelation (fp32 or bf16 values)."""
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    vals = torch.from_numpy(np.ascontiguousarray(r.values, dtype=np.float32)).to(device)
    return SparseTensorRelation(torch.from_numpy(r.coords).to(device), vals.to(tdt), r.shape,
                                r.tile_shape)


def host_rel(r: R.Rel):
    return SparseTensorRelation(r.coords, r.values, r.shape, r.tile_shape)


def hv(t: torch.Tensor) -> np.ndarray:
    """Device values (float32 or bfloat16) as a host float32 array."""
    return t.float().cpu().numpy()


# ---------------------------------------------------------------------------
# joins

def test_join_golden_vectors(gpu):
    g = np.load("tests/golden/join_order.npz")
    for name in g["names"]:
        note("join golden", name)
        lc, rc = g[f"{name}__lhs"], g[f"{name}__rhs"]
        keys = [tuple(k) for k in g[f"{name}__keys"].tolist()]
        hl, hr = ej.coordinate_join_hash(lc, rc, keys)
        npt.assert_array_equal(hl, g[f"{name}__hash_lhs"], err_msg=name)
        npt.assert_array_equal(hr, g[f"{name}__hash_rhs"], err_msg=name)
        sl, sr = ej.coordinate_join_sorted(lc, rc, keys)
        npt.assert_array_equal(sl, g[f"{name}__sorted_lhs"], err_msg=name)
        npt.assert_array_equal(sr, g[f"{name}__sorted_rhs"], err_msg=name)
        assert hl.dtype == np.int64 and sl.dtype == np.int64


@pytest.mark.parametrize("name", list(G.WORKLOADS))
def test_join_and_plan_full_size(gpu, name):
    """Join pairs, output coordinates and the segment plan at the workloads'
    full sizes, bit-exact against the oracle."""
    note("join+plan full size", name)
    w = G.WORKLOADS[name](values=False)
    L, Rr = w["lhs"], w["rhs"]
    li_o, ri_o = R.coordinate_join(L.coords, Rr.coords, w["join_keys"])
    lhs = SparseTensorRelation(torch.from_numpy(L.coords).cuda(), None, L.shape, L.tile_shape)
    rhs = SparseTensorRelation(torch.from_numpy(Rr.coords).cuda(), None, Rr.shape, Rr.tile_shape)
    lc, rc = lhs.coords, rhs.coords
    li, ri = sd._join_dev(lhs, rhs, w["join_keys"], lc, rc)
    npt.assert_array_equal(li.cpu().numpy(), li_o)
    npt.assert_array_equal(ri.cpu().numpy(), ri_o)
    oc_o = R.compute_output_coords(L.coords, Rr.coords, li_o, ri_o, w["agg_keys"])
    from einjax_amd import _device

    oc = _device.output_coords(lc, rc, li, ri, w["agg_keys"])
    npt.assert_array_equal(oc.cpu().numpy(), oc_o)
    radices = [max(sd._grid(lhs if s == 0 else rhs, d), 1) for s, d in w["agg_keys"]]
    coords, off, perm, seg = _device.segment_plan(lc, rc, li, ri, w["agg_keys"], radices)
    uc_o, perm_o, off_o, seg_o = R.segment_plan(oc_o)
    npt.assert_array_equal(coords.cpu().numpy(), uc_o)
    npt.assert_array_equal(off.cpu().numpy(), off_o)
    npt.assert_array_equal(perm.cpu().numpy(), perm_o)
    npt.assert_array_equal(seg.cpu().numpy(), seg_o)


# Sizes straddling the sort's tile choices (1, 2, 4, 8 keys per thread; up
# to 32 blocks with offsets read inline, more with a scanned histogram), the
# one-workgroup flag scan (up to 65536 pairs), the two-launch scan limit
# (524288) and odd/even radix pass counts.
PLAN_SIZES = [1, 2, 255, 257, 8192, 8193, 16385, 32768, 32769, 65536, 65537, 262145, 600000]


@pytest.mark.parametrize("P", PLAN_SIZES)
@pytest.mark.parametrize("radix", [(64, 64), (4096, 64)])
def test_segment_plan_sizes(gpu, P, radix):
    """Segment plan of P random pairs (12-bit keys: two radix passes; 18-bit
    keys: three) bit-exact against the oracle's stable sort."""
    note("segment plan", P, radix)
    rng = np.random.default_rng(P)
    nl, nr = 3000, 2000
    lc = rng.integers(0, radix[0], (nl, 2), dtype=np.int32)
    rc = rng.integers(0, radix[1], (nr, 2), dtype=np.int32)
    li = rng.integers(0, nl, P).astype(np.int64)
    ri = rng.integers(0, nr, P).astype(np.int64)
    agg = [(0, 0), (1, 1)]
    oc_o = R.compute_output_coords(lc, rc, li, ri, agg)
    uc_o, perm_o, off_o, seg_o = R.segment_plan(oc_o)
    from einjax_amd import _device

    t = lambda a: torch.from_numpy(a).cuda()
    coords, off, perm, seg = _device.segment_plan(t(lc), t(rc), t(li), t(ri), agg, list(radix))
    npt.assert_array_equal(coords.cpu().numpy(), uc_o)
    npt.assert_array_equal(off.cpu().numpy(), off_o)
    npt.assert_array_equal(perm.cpu().numpy(), perm_o)
    npt.assert_array_equal(seg.cpu().numpy(), seg_o)


@pytest.mark.parametrize("n_lhs,n_rhs", [(1, 1), (8192, 8192), (8193, 100), (100, 8193),
                                         (300, 65536), (300, 65537), (20000, 30000)])
def test_join_sizes(gpu, n_lhs, n_rhs):
    """Both join orders around the single-workgroup probe limits (8192 build
    keys in LDS, 8192 probe keys) and at a large probe side, bit-exact
    against the oracle."""
    note("join sizes", n_lhs, n_rhs)
    rng = np.random.default_rng(n_lhs * 7 + n_rhs)
    lc = rng.integers(0, 2000, (n_lhs, 2), dtype=np.int32)
    rc = rng.integers(0, 2000, (n_rhs, 2), dtype=np.int32)
    keys = [(1, 0)]
    hl, hr = ej.coordinate_join_hash(lc, rc, keys)
    li_o, ri_o = R.coordinate_join(lc, rc, keys)
    npt.assert_array_equal(hl, li_o)
    npt.assert_array_equal(hr, ri_o)
    sl, sr = ej.coordinate_join_sorted(lc, rc, keys)
    sl_o, sr_o = R.coordinate_join_sorted(lc, rc, keys)
    npt.assert_array_equal(sl, sl_o)
    npt.assert_array_equal(sr, sr_o)


@pytest.mark.parametrize("n_lhs,n_rhs,ncols", [(4096, 8192, 1), (4097, 8192, 1), (4096, 8193, 1),
                                               (1000, 3000, 3), (50, 70, 3), (1, 8192, 1)])
def test_join_probe_small_limits(gpu, n_lhs, n_rhs, ncols):
    """Probe-order joins around the one-workgroup count (at most 4096 build
    rows sorted in LDS, 8192 probe rows) with one or three key columns (one to
    three 8-bit radix passes in LDS), bit-exact against the oracle."""
    note("join probe small limits", n_lhs, n_rhs, ncols)
    rng = np.random.default_rng(n_lhs * 3 + n_rhs + ncols)
    if ncols == 1:
        lc = rng.integers(0, 3000, (n_lhs, 4), dtype=np.int32)
        rc = rng.integers(0, 3000, (n_rhs, 4), dtype=np.int32)
        keys = [(1, 0)]
    else:  # radix 3000 per column (35-bit keys, five passes), 64 distinct keys
        vals = np.array([0, 7, 999, 2999], np.int32)
        lc = rng.choice(vals, (n_lhs, 4))
        rc = rng.choice(vals, (n_rhs, 4))
        keys = [(1, 0), (2, 2), (3, 1)]
    hl, hr = ej.coordinate_join_hash(lc, rc, keys)
    li_o, ri_o = R.coordinate_join(lc, rc, keys)
    assert len(li_o) > 0
    npt.assert_array_equal(hl, li_o)
    npt.assert_array_equal(hr, ri_o)


@pytest.mark.parametrize("n_lhs,n_rhs", [(100, 200), (5000, 200), (100, 9000)])
@pytest.mark.parametrize("side", ["lhs", "rhs"])
def test_join_and_plan_range_flag(gpu, n_lhs, n_rhs, side):
    """A key or output coordinate outside its declared radix is reported
    (ValueError) by the one-workgroup and by the general count paths."""
    note("join/plan range flag", n_lhs, n_rhs, side)
    from einjax_amd import _device

    rng = np.random.default_rng(n_lhs + n_rhs)
    lc = rng.integers(0, 10, (n_lhs, 2), dtype=np.int32)
    rc = rng.integers(0, 10, (n_rhs, 2), dtype=np.int32)
    t = lambda a: torch.from_numpy(a).cuda()
    # join: a key coordinate of 10 on one side against a radix of 10
    lb, rb = lc.copy(), rc.copy()
    if side == "lhs":
        lb[n_lhs // 2, 1] = 10
    else:
        rb[n_rhs // 2, 0] = 10
    with pytest.raises(ValueError, match="outside"):
        _device.join(t(lb), t(rb), [(1, 0)], [10])
    li, ri = _device.join(t(lc), t(rc), [(1, 0)], [10])
    assert li.numel() > 0
    # plan: an output coordinate (a non-key column) of 10 against a radix of 10
    if side == "lhs":
        lc[int(li[li.numel() // 2]), 0] = 10
    else:
        rc[int(ri[ri.numel() // 2]), 1] = 10
    agg = [(0, 0), (1, 1)]
    with pytest.raises(ValueError, match="outside"):
        _device.segment_plan(t(lc), t(rc), li, ri, agg, [10, 10])
    coords, off, perm, seg = _device.segment_plan(t(lc), t(rc), li, ri, agg, [11, 11])
    oc_o = R.compute_output_coords(lc, rc, li.cpu().numpy(), ri.cpu().numpy(), agg)
    uc_o, perm_o, off_o, _ = R.segment_plan(oc_o)
    npt.assert_array_equal(coords.cpu().numpy(), uc_o)
    npt.assert_array_equal(off.cpu().numpy(), off_o)
    npt.assert_array_equal(perm.cpu().numpy(), perm_o)


def test_join_edge_cases(gpu):
    note("join edge cases")
    e = np.zeros((0, 2), np.int32)
    one = np.array([[0, 0]], np.int32)
    for fn in (ej.coordinate_join_hash, ej.coordinate_join_sorted):
        li, ri = fn(e, e, [(1, 0)])
        assert len(li) == 0 and li.dtype == np.int64
        li, ri = fn(one, e, [])
        assert len(li) == 0
        li, ri = fn(np.array([[0], [1]]), np.array([[0], [1], [2]]), [])
        npt.assert_array_equal(li, [0, 0, 0, 1, 1, 1])
        npt.assert_array_equal(ri, [0, 1, 2, 0, 1, 2])
        li, ri = fn(np.array([[0, 0]]), np.array([[1, 0]]), [(0, 0)])
        assert len(li) == 0
    # all rows share one key: the output is the full product, in order
    lc = np.zeros((300, 1), np.int32)
    rc = np.zeros((200, 1), np.int32)
    li, ri = ej.coordinate_join_hash(lc, rc, [0])
    hl, hr = R.coordinate_join_hash(lc, rc, [0])
    npt.assert_array_equal(li, hl)
    npt.assert_array_equal(ri, hr)
    # coordinates beyond the declared grid still join (radices sized from data)
    lhs = SparseTensorRelation(np.array([[0, 9], [1, 3]], np.int32), np.ones((2, 1, 1)), (2, 4),
                               (1, 1))
    rhs = SparseTensorRelation(np.array([[9, 0], [3, 1]], np.int32), np.ones((2, 1, 1)), (4, 2),
                               (1, 1))
    li, ri = ej.coordinate_join(lhs, rhs, [(1, 0)])
    npt.assert_array_equal(li, [0, 1])
    npt.assert_array_equal(ri, [0, 1])


# ---------------------------------------------------------------------------
# tile einsum

EINSUM_CASES = [
    # spec, lhs tile, rhs tile (MFMA layouts first, then generic strings)
    ("ij,jk->ik", (64, 64), (64, 64)),
    ("ij,jk->ik", (128, 128), (128, 128)),
    ("ij,jk->ik", (32, 32), (32, 32)),
    ("ij,jk->ik", (128, 64), (64, 32)),
    ("ij,kj->ik", (64, 32), (64, 32)),
    ("ji,jk->ik", (64, 64), (64, 128)),
    ("ji,kj->ik", (32, 64), (32, 32)),
    ("ji,jk->ik", (64, 64), (64, 64)),      # [k][m] lhs on the LDS ring
    ("ji,jk->ik", (128, 128), (128, 128)),
    ("ij,kj->ik", (128, 128), (128, 128)),  # [n][k] rhs on the LDS ring
    ("bij,bjk->bik", (1, 64, 64), (1, 64, 64)),
    ("bij,bjk->bik", (4, 32, 32), (4, 32, 64)),
    ("ijk,kl->ijl", (8, 16, 32), (32, 32)),
    ("ik,kj->ji", (32, 32), (32, 64)),
    ("i,j->ij", (3,), (4,)),
    ("i,i->", (5,), (5,)),
    ("ij,ij->ij", (3, 4), (3, 4)),
    ("ii,ij->j", (4, 4), (4, 3)),
    ("ij,kl->ij", (1, 1), (1, 1)),
    ("ijk,jl->il", (2, 3, 4), (3, 5)),
    ("ij,jk->ik", (5, 7), (7, 3)),
    ("ij,jk->ik", (48, 16), (16, 40)),
]


def _rand_tiles(rng, n, tile, dtype):
    v = rng.standard_normal((n, *tile)).astype(np.float32)
    return R.bf16_round(v) if dtype == "bf16" else v


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("spec,lt,rt", EINSUM_CASES)
def test_pair_einsum(gpu, spec, lt, rt, dtype):
    note("pair einsum", spec, lt, rt, dtype)
    rng = np.random.default_rng(zlib.crc32(repr((spec, lt, rt)).encode()))
    nl, nr, P = 7, 5, 23
    lv, rv = _rand_tiles(rng, nl, lt, dtype), _rand_tiles(rng, nr, rt, dtype)
    li = rng.integers(0, nl, P)
    ri = rng.integers(0, nr, P)
    want = R.kernel_einsum(lv, rv, li, ri, spec, precision="fp64")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    got = ej.kernel_einsum(torch.from_numpy(lv).cuda().to(tdt), torch.from_numpy(rv).cuda().to(tdt),
                           torch.from_numpy(li).cuda(), torch.from_numpy(ri).cuda(), spec)
    assert got.dtype == tdt  # the operands' dtype, as jnp.einsum returns
    assert tuple(got.shape) == want.shape
    err = R.rel_l2(hv(got), want)
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("spec,lt,rt", EINSUM_CASES[:14])
def test_segment_einsum_matches_pairs_plus_segsum(gpu, spec, lt, rt, dtype):
    """Fused mode == per-pair results summed in plan order (within fp32
    rounding), on random segment structure with skewed segment lengths."""
    note("segment einsum", spec, lt, rt, dtype)
    from einjax_amd import _device

    rng = np.random.default_rng(5)
    nl, nr, P = 9, 6, 60
    lv, rv = _rand_tiles(rng, nl, lt, dtype), _rand_tiles(rng, nr, rt, dtype)
    li = rng.integers(0, nl, P)
    ri = rng.integers(0, nr, P)
    oc = np.minimum(rng.zipf(1.6, size=(P, 1)) - 1, 11).astype(np.int32)
    uc, perm, off, _ = R.segment_plan(oc)
    pairs = R.kernel_einsum(lv, rv, li, ri, spec, precision="fp64")
    want = np.stack([pairs[perm[off[u]:off[u + 1]]].sum(0) for u in range(len(uc))])
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    desc = _device.describe(spec, lt, rt)
    got = _device.segment_einsum(desc, torch.from_numpy(lv).cuda().to(tdt),
                                 torch.from_numpy(rv).cuda().to(tdt),
                                 torch.from_numpy(li).cuda(), torch.from_numpy(ri).cuda(),
                                 torch.from_numpy(perm).cuda(), torch.from_numpy(off).cuda())
    err = R.rel_l2(hv(got), want)
    assert err <= TOL[dtype], err


def _same_bits(x: torch.Tensor, y: torch.Tensor) -> bool:
    return x.dtype == y.dtype and x.shape == y.shape and torch.equal(
        x.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("spec,lt,rt", EINSUM_CASES)
def test_bf16_output_is_rounded_fp32_output(gpu, spec, lt, rt):
    """bf16 operands: the default bf16 output of every kernel (per pair,
    fused segment sums, segment sum of bf16 pair values) is the fp32 output
    of the same kernel rounded to nearest even, bit for bit: the sums are
    formed in fp32 either way and rounded once."""
    note("bf16 output", spec, lt, rt)
    from einjax_amd import _device

    rng = np.random.default_rng(zlib.crc32(repr((spec, lt, rt, "bf16out")).encode()))
    nl, nr, P = 9, 6, 60
    c = lambda a: torch.from_numpy(a).cuda()
    a = c(_rand_tiles(rng, nl, lt, "bf16")).to(torch.bfloat16)
    b = c(_rand_tiles(rng, nr, rt, "bf16")).to(torch.bfloat16)
    li, ri = c(rng.integers(0, nl, P)), c(rng.integers(0, nr, P))
    oc = np.minimum(rng.zipf(1.6, size=(P, 1)) - 1, 11).astype(np.int32)
    _, perm, off, _ = R.segment_plan(oc)
    perm, off = c(perm), c(off)
    desc = _device.describe(spec, lt, rt)
    p16 = _device.pair_einsum(desc, a, b, li, ri)
    p32 = _device.pair_einsum(desc, a, b, li, ri, out_dtype=torch.float32)
    assert p16.dtype == torch.bfloat16 and p32.dtype == torch.float32
    assert _same_bits(p16, p32.to(torch.bfloat16))
    s16 = _device.segment_einsum(desc, a, b, li, ri, perm, off)
    s32 = _device.segment_einsum(desc, a, b, li, ri, perm, off, out_dtype=torch.float32)
    assert _same_bits(s16, s32.to(torch.bfloat16))
    q16 = _device.segment_sum(p16, perm, off)
    q32 = _device.segment_sum(p16.float(), perm, off)
    assert _same_bits(q16, q32.to(torch.bfloat16))


@pytest.mark.parametrize("lt,rt,n_seg", [((64, 32), (32, 64), 3000), ((128, 32), (32, 128), 2100)])
def test_bf16_output_multi_segment_workgroups(gpu, lt, rt, n_seg):
    """bf16 'ij,jk->ik' with K = 32 and thousands of segments: the ring kernel
    runs several consecutive segments per workgroup and stores each output
    block inside its stage loop; bf16 outputs there are the fp32 ones
    rounded, and empty segments are zero."""
    note("bf16 output, multi-segment workgroups", lt, rt, n_seg)
    from einjax_amd import _device

    rng = np.random.default_rng(n_seg)
    counts = rng.integers(0, 4, n_seg)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    P = int(off[-1])
    c = lambda x: torch.from_numpy(x).cuda()
    a = c(_rand_tiles(rng, 40, lt, "bf16")).to(torch.bfloat16)
    b = c(_rand_tiles(rng, 30, rt, "bf16")).to(torch.bfloat16)
    li, ri = c(rng.integers(0, 40, P)), c(rng.integers(0, 30, P))
    perm = c(rng.permutation(P).astype(np.int32))
    desc = _device.describe("ij,jk->ik", lt, rt)
    s16 = _device.segment_einsum(desc, a, b, li, ri, perm, c(off))
    s32 = _device.segment_einsum(desc, a, b, li, ri, perm, c(off), out_dtype=torch.float32)
    assert _same_bits(s16, s32.to(torch.bfloat16))
    assert torch.all(s16[c(counts == 0)] == 0)
    want = np.zeros((n_seg, lt[0], rt[1]))
    A, B = hv(a).astype(np.float64), hv(b).astype(np.float64)
    lin, rin, pn = li.cpu().numpy(), ri.cpu().numpy(), perm.cpu().numpy()
    for u in range(0, n_seg, 7):  # a sample of segments in float64
        for q in range(off[u], off[u + 1]):
            want[u] += A[lin[pn[q]]] @ B[rin[pn[q]]]
    assert R.rel_l2(hv(s32)[::7], want[::7]) <= TOL["fp32"]


def test_gemm_index_out_of_range_contributes_nothing(gpu):
    note("einsum out-of-range index")
    from einjax_amd import _device

    rng = np.random.default_rng(0)
    lv = rng.standard_normal((3, 32, 32)).astype(np.float32)
    rv = rng.standard_normal((2, 32, 32)).astype(np.float32)
    desc = _device.describe("ij,jk->ik", (32, 32), (32, 32))
    li = torch.tensor([0, 5, -1], dtype=torch.int64, device="cuda")
    ri = torch.tensor([1, 0, 0], dtype=torch.int64, device="cuda")
    out = _device.pair_einsum(desc, torch.from_numpy(lv).cuda(), torch.from_numpy(rv).cuda(), li,
                              ri).cpu().numpy()
    npt.assert_allclose(out[0], lv[0] @ rv[1], rtol=1e-5, atol=1e-4)
    assert np.all(out[1] == 0) and np.all(out[2] == 0)


# ---------------------------------------------------------------------------
# grouped segment einsum: several output segments per workgroup when the
# segments contract the same lhs tiles (an lhs row against a dense rhs)

def _matmul_rels(rng, tile, rows, inner, cols, lhs_density, rhs_density=1.0):
    """bf16 'ij,jk->ik' relations: lhs [rows x inner] tiles at lhs_density,
    rhs [inner x cols] tiles at rhs_density (1.0: dense)."""
    def pick(grid, dens):
        n = grid[0] * grid[1]
        k = max(1, int(round(dens * n)))
        flat = np.sort(rng.choice(n, size=k, replace=False))
        return np.stack(np.unravel_index(flat, grid), axis=1).astype(np.int32)

    ac, bc = pick((rows, inner), lhs_density), pick((inner, cols), rhs_density)
    av = R.bf16_round(rng.standard_normal((len(ac), tile, tile)).astype(np.float32))
    bv = R.bf16_round(rng.standard_normal((len(bc), tile, tile)).astype(np.float32))
    return (R.Rel(ac, av, (rows * tile, inner * tile), (tile, tile)),
            R.Rel(bc, bv, (inner * tile, cols * tile), (tile, tile)))


def _segment_einsum_groups(lhs, rhs, groups, li_override=None, spec="ij,jk->ik"):
    """Runs the device join, plan and fused einsum with each seg_group hint;
    returns the plan's output coordinates and {hint: values}.  spec
    "ji,jk->ik" hands in every lhs tile transposed, "ij,kj->ik" every rhs
    tile (the same product, other operand layouts)."""
    from einjax_amd import _device

    L, Rr = dev_rel(lhs, "bf16"), dev_rel(rhs, "bf16")
    li, ri = sd._join_dev(L, Rr, [(1, 0)], L.coords, Rr.coords)
    coords, offs, perm, _ = _device.segment_plan(L.coords, Rr.coords, li, ri, [(0, 0), (1, 1)],
                                                  [sd._grid(L, 0), sd._grid(Rr, 1)])
    if li_override is not None:
        li = li_override(li)
    lvals, rvals = L.values, Rr.values
    if spec == "ji,jk->ik":
        lvals = lvals.transpose(1, 2).contiguous()
    elif spec == "ij,kj->ik":
        rvals = rvals.transpose(1, 2).contiguous()
    desc = _device.describe(spec, lhs.tile_shape, rhs.tile_shape)
    out = {}
    for gsz in groups:
        desc.seg_group = gsz
        out[gsz] = hv(_device.segment_einsum(desc, lvals, rvals, li, ri, perm, offs))
    return coords.cpu().numpy(), out


@pytest.mark.parametrize("tile,rows,inner,cols,dens", [
    (128, 6, 5, 8, 0.5),    # uniform groups of 4 on 128 x 128 tiles (8 waves)
    (64, 5, 7, 12, 0.4),    # 64 x 64 tiles (4 waves)
    (64, 2, 70, 4, 1.0),    # 70 pairs per segment: pair table in two chunks
])
def test_grouped_segment_einsum(gpu, tile, rows, inner, cols, dens):
    note("grouped segment einsum", tile, rows, inner, cols, dens)
    rng = np.random.default_rng(tile + rows + inner)
    lhs, rhs = _matmul_rels(rng, tile, rows, inner, cols, dens)
    assert sd._segment_run(host_rel(rhs), [(1, 0)], [(0, 0), (1, 1)]) == cols
    coords, out = _segment_einsum_groups(lhs, rhs, (0, cols))
    want = R.execute_sparse(lhs, rhs, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], precision="fp64")
    npt.assert_array_equal(coords, want.coords)
    # same accumulation order per output tile: bitwise equal to one segment per workgroup
    npt.assert_array_equal(out[cols], out[0])
    assert R.rel_l2(out[cols], want.values) <= TOL["bf16"]


@pytest.mark.parametrize("spec", ["ji,jk->ik", "ij,kj->ik"])
@pytest.mark.parametrize("tile,rows,inner,cols,dens", [
    (128, 6, 5, 8, 0.5),
    (64, 5, 7, 12, 0.4),
    (64, 2, 70, 4, 1.0),
])
def test_grouped_segment_einsum_layouts(gpu, spec, tile, rows, inner, cols, dens):
    """The LDS-ring einsum with a transposed operand (a [k][m] lhs or an
    [n][k] rhs tile, the layouts of the backward's gradient einsums), one
    segment per workgroup and grouped: the standard-layout product."""
    note("grouped segment einsum, layout", spec, tile, rows, inner, cols, dens)
    rng = np.random.default_rng(tile + rows + inner + 1)
    lhs, rhs = _matmul_rels(rng, tile, rows, inner, cols, dens)
    coords, out = _segment_einsum_groups(lhs, rhs, (0, cols), spec=spec)
    want = R.execute_sparse(lhs, rhs, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], precision="fp64")
    npt.assert_array_equal(coords, want.coords)
    npt.assert_array_equal(out[cols], out[0])
    assert R.rel_l2(out[0], want.values) <= TOL["bf16"]
    # the standard layout gives the same sums (same fp32 order), bit for bit
    _, std = _segment_einsum_groups(lhs, rhs, (0,))
    npt.assert_array_equal(out[0], std[0])


@pytest.mark.parametrize("cols,rhs_dens", [(6, 1.0), (8, 0.6), (5, 1.0)])
def test_grouped_segment_einsum_wrong_hint(gpu, cols, rhs_dens):
    """A hint the data does not bear out (groups straddling rows, sparse rhs,
    a segment count that is not a multiple of 4) costs speed, not results."""
    note("grouped segment einsum, wrong hint", cols, rhs_dens)
    rng = np.random.default_rng(cols)
    lhs, rhs = _matmul_rels(rng, 128, 5, 6, cols, 0.5, rhs_dens)
    coords, out = _segment_einsum_groups(lhs, rhs, (0, 4, 8))
    want = R.execute_sparse(lhs, rhs, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], precision="fp64")
    npt.assert_array_equal(coords, want.coords)
    npt.assert_array_equal(out[4], out[0])
    npt.assert_array_equal(out[8], out[0])
    assert R.rel_l2(out[0], want.values) <= TOL["bf16"]


def test_grouped_segment_einsum_invalid_index(gpu):
    """An out-of-range lhs index inside a group contributes nothing there,
    as it does with one segment per workgroup."""
    note("grouped segment einsum, invalid index")
    rng = np.random.default_rng(11)
    lhs, rhs = _matmul_rels(rng, 128, 4, 5, 8, 0.6)

    def corrupt(li):
        li = li.clone()
        li[3] = -1
        li[10] = 10 ** 6
        return li

    _, out = _segment_einsum_groups(lhs, rhs, (0, 8), li_override=corrupt)
    npt.assert_array_equal(out[8], out[0])


# ---------------------------------------------------------------------------
# several output blocks per workgroup (every m-block of a group, or several
# consecutive segments): used when the launch would otherwise have at least
# 1024 workgroups of short work

def _segments_fp64(lhs, rhs, li, ri, perm, off, spec, useg):
    """float64 sums of the per-pair einsums of the segments useg, in plan
    order (numpy on the host), for a spot check of large cases."""
    out = []
    for u in useg:
        ps = perm[off[u]:off[u + 1]]
        acc = None
        for p in ps:
            v = np.einsum(spec, lhs.values[li[p]].astype(np.float64),
                          rhs.values[ri[p]].astype(np.float64))
            acc = v if acc is None else acc + v
        out.append(acc)
    return np.stack(out)


def test_multi_segment_workgroups_fp32(gpu):
    """fp32 sparse x sparse with ~4,600 output tiles: four consecutive
    segments per workgroup in the fused einsum.  Checked against the unfused
    path (one pair per workgroup) and, on a sample, float64 sums."""
    note("multi-segment workgroups fp32")
    rng = np.random.default_rng(21)
    g, t = 96, 64

    def rel(n):
        flat = np.sort(rng.choice(g * g, size=n, replace=False))
        c = np.stack(np.unravel_index(flat, (g, g)), axis=1).astype(np.int32)
        return R.Rel(c, rng.uniform(-1, 1, (n, t, t)).astype(np.float32), (g * t, g * t), (t, t))

    lhs, rhs = rel(900), rel(900)
    L, Rr = dev_rel(lhs), dev_rel(rhs)
    fused = ej.execute_sparse(L, Rr, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)])
    split = ej.execute_sparse(L, Rr, [(1, 0)], "ij,jk->ik", [(0, 0), (1, 1)], fused=False)
    U = fused.num_tuples
    assert U >= 4096, U  # enough segments for the multi-segment launch
    npt.assert_array_equal(fused.coords.cpu().numpy(), split.coords.cpu().numpy())
    fv, sv = fused.values.cpu().numpy(), split.values.cpu().numpy()
    assert R.rel_l2(fv, sv) <= 1e-6
    li, ri = R.coordinate_join(lhs.coords, rhs.coords, [(1, 0)])
    oc = R.compute_output_coords(lhs.coords, rhs.coords, li, ri, [(0, 0), (1, 1)])
    _, perm, off, _ = R.segment_plan(oc)
    sample = np.sort(rng.choice(U, 48, replace=False))
    want = _segments_fp64(lhs, rhs, li, ri, perm, off, "ij,jk->ik", sample)
    assert R.rel_l2(fv[sample], want) <= TOL["fp32"]


def test_multi_mblock_workgroups_fp32(gpu):
    """'ijk,kl->ijl' with 32^3 fp32 tiles (M = 1024 rows, 8 m-blocks of 128)
    against a dense rhs, ~1,200 groups of 4 segments: every m-block of a group
    in one workgroup.  Checked on a sample of output tiles in float64."""
    note("multi-m-block workgroups fp32")
    w = G.workload_order3(n=512, l=1024, density=0.1)
    lhs, rhs = w["lhs"], w["rhs"]
    got = ej.execute_sparse(dev_rel(lhs), dev_rel(rhs), w["join_keys"], w["kernel_string"],
                            w["agg_keys"])
    U = got.num_tuples
    assert U // 4 >= 1024, U
    li, ri = R.coordinate_join(lhs.coords, rhs.coords, w["join_keys"])
    oc = R.compute_output_coords(lhs.coords, rhs.coords, li, ri, w["agg_keys"])
    uc, perm, off, _ = R.segment_plan(oc)
    npt.assert_array_equal(got.coords.cpu().numpy(), uc)
    rng = np.random.default_rng(3)
    sample = np.sort(rng.choice(U, 40, replace=False))
    want = _segments_fp64(lhs, rhs, li, ri, perm, off, w["kernel_string"], sample)
    assert R.rel_l2(got.values.cpu().numpy()[sample], want) <= TOL["fp32"]


def test_multi_segment_workgroups_empty_segments(gpu):
    """A caller's plan may hold segments without pairs: their output tiles
    are zero, also when a workgroup covers several segments."""
    note("multi-segment workgroups, empty segments")
    from einjax_amd import _device

    rng = np.random.default_rng(8)
    n_seg, t = 6000, 32
    counts = rng.integers(0, 3, n_seg)  # 0, 1 or 2 pairs per segment
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    P = int(off[-1])
    lv = rng.standard_normal((50, t, t)).astype(np.float32)
    rv = rng.standard_normal((40, t, t)).astype(np.float32)
    li = rng.integers(0, 50, P)
    ri = rng.integers(0, 40, P)
    perm = rng.permutation(P).astype(np.int32)
    desc = _device.describe("ij,jk->ik", (t, t), (t, t))
    c = lambda a: torch.from_numpy(a).cuda()
    got = _device.segment_einsum(desc, c(lv), c(rv), c(li), c(ri), c(perm), c(off)).cpu().numpy()
    pairs = np.einsum("pij,pjk->pik", lv[li].astype(np.float64), rv[ri].astype(np.float64))
    want = np.zeros((n_seg, t, t))
    for u in range(n_seg):
        for q in range(off[u], off[u + 1]):
            want[u] += pairs[perm[q]]
    assert np.all(got[counts == 0] == 0)
    assert R.rel_l2(got, want) <= TOL["fp32"]


# ---------------------------------------------------------------------------
# segment sum

def test_segment_sum_known_answers_and_order(gpu):
    note("segment_sum known answers")
    c, a = ej.segment_sum(np.array([[[1.0, 0], [0, 1]], [[2.0, 0], [0, 2]]]),
                          np.array([[0, 0], [0, 0]], np.int32))
    assert c.shape == (1, 2)
    npt.assert_allclose(a[0], 3 * np.eye(2))
    c, a = ej.segment_sum(np.array([[[1.0]], [[2.0]], [[3.0]]]),
                          np.array([[2, 0], [0, 0], [1, 0]], np.int32))
    npt.assert_array_equal(c, [[0, 0], [1, 0], [2, 0]])
    npt.assert_array_equal(a[:, 0, 0], [2, 3, 1])
    c, a = ej.segment_sum(np.zeros((0, 2, 2)), np.zeros((0, 2), np.int32))
    assert c.shape == (0, 2) and a.shape == (0, 2, 2)
    # pair-order fp32 accumulation is bit-identical to the oracle's
    rng = np.random.default_rng(1)
    oc = rng.integers(0, 6, size=(500, 2)).astype(np.int32)
    v = rng.standard_normal((500, 4, 8)).astype(np.float32) * 1e3
    c, a = ej.segment_sum(v, oc)
    c_o, a_o = R.segment_sum(v, oc)
    npt.assert_array_equal(c, c_o)
    npt.assert_array_equal(a, a_o)


# ---------------------------------------------------------------------------
# end to end: the reference's own cases through the drop-in API

def _rel(dense, tile):
    return SparseTensor("t", dense).to_relation(tile)


@pytest.mark.parametrize("fused", [True, False])
def test_reference_end_to_end_cases(gpu, fused):
    note("reference end-to-end cases, fused =", fused)
    A, B = np.array([[1.0, 2.0], [3.0, 4.0]]), np.eye(2)
    out = ej.execute_sparse(_rel(A, (1, 1)), _rel(B, (1, 1)), [(1, 0)], "ij,jk->ik",
                            [(0, 0), (1, 1)], (2, 2), (1, 1), fused=fused)
    npt.assert_allclose(out.to_dense(), A @ B, atol=1e-6)
    A, B = np.diag([1.0, 2, 3, 4]), np.diag([5.0, 6, 7, 8])
    out = ej.execute_sparse(_rel(A, (1, 1)), _rel(B, (1, 1)), [(1, 0)], "ij,jk->ik",
                            [(0, 0), (1, 1)], (4, 4), (1, 1), fused=fused)
    npt.assert_allclose(out.to_dense(), A @ B, atol=1e-6)
    A = np.array([[1.0, 2, 0, 0], [3, 4, 0, 0], [0, 0, 5, 6], [0, 0, 7, 8]])
    out = ej.execute_sparse(_rel(A, (2, 2)), _rel(np.eye(4), (2, 2)), [(1, 0)], "ij,jk->ik",
                            [(0, 0), (1, 1)], (4, 4), (2, 2), fused=fused)
    npt.assert_allclose(out.to_dense(), A, atol=1e-6)
    a, b = np.array([1.0, 0, 3]), np.array([0.0, 2, 4])
    out = ej.execute_sparse(_rel(a.reshape(3, 1), (1, 1)), _rel(b.reshape(1, 3), (1, 1)), [],
                            "ij,kl->ij", [(0, 0), (1, 1)], (3, 3), (1, 1), fused=fused)
    npt.assert_allclose(out.to_dense(), np.outer(a, b), atol=1e-6)
    A, B = np.diag([1.0, 2, 3]), np.diag([4.0, 5, 6])
    out = ej.execute_sparse(_rel(A, (1, 1)), _rel(B, (1, 1)), [(0, 0), (1, 1)], "ij,ij->ij",
                            [(0, 0), (0, 1)], (3, 3), (1, 1), fused=fused)
    npt.assert_allclose(out.to_dense(), A * B, atol=1e-6)
    A = np.zeros((4, 4)); A[0, 0] = 1
    B = np.zeros((4, 4)); B[2, 2] = 1
    out = ej.execute_sparse(_rel(A, (2, 2)), _rel(B, (2, 2)), [(1, 0)], "ij,jk->ik",
                            [(0, 0), (1, 1)], (4, 4), (2, 2), fused=fused)
    assert out.num_tuples == 0
    npt.assert_allclose(out.to_dense(), np.zeros((4, 4)))
    A, B = np.diag([1.0, 2]), np.diag([3.0, 4])
    out = ej.execute_sparse(_rel(A, (1, 1)), _rel(B, (1, 1)), [(1, 0)], "ij,jk->ik",
                            [(0, 0), (1, 1)], fused=fused)
    npt.assert_allclose(out.to_dense(), A @ B, atol=1e-6)


def test_block_sparse_matmul_api(gpu):
    note("block_sparse_matmul api")
    A = np.array([[1.0, 0, 2, 0], [0, 3, 0, 4], [5, 0, 6, 0]])
    B = np.array([[1.0, 0], [0, 2], [3, 0], [0, 4]])
    out = ej.block_sparse_matmul_generic(_rel(A, (1, 1)), _rel(B, (1, 1)))
    npt.assert_allclose(out.to_dense(), A @ B, atol=1e-6)
    la, rb = _rel(np.array([[1.0, 2], [3, 4]]), (1, 1)), _rel(np.eye(2), (1, 1))
    out = ej.block_sparse_matmul(la.coords, la.values, rb.coords, rb.values, (1, 1, 1), (2, 2),
                                 (2, 2))
    npt.assert_allclose(out.to_dense(), [[1, 2], [3, 4]], atol=1e-6)
    assert out.shape == (2, 2) and out.tile_shape == (1, 1)
    A = np.zeros((4, 4)); A[0, 0] = 1
    B = np.zeros((4, 4)); B[2, 2] = 1
    out = ej.block_sparse_matmul_generic(_rel(A, (2, 2)), _rel(B, (2, 2)))
    assert out.num_tuples == 0 and out.values.dtype == np.float64
    reg = ej.KernelRegistry()
    fn = reg.lookup("ij,jk->ik", backend="gpu", sparsity="sparse")
    assert fn is ej.block_sparse_matmul_generic
    assert reg.lookup("ij,kj->ik", backend="gpu", sparsity="sparse") is ej.execute_sparse


@pytest.mark.parametrize("name", ["blocksparse_1k", "order3_small", "banded_small",
                                  "zipf_small"])
@pytest.mark.parametrize("fused", [True, False])
def test_workload_end_to_end(gpu, name, fused):
    """Whole execute_sparse against the oracle's (fp64-accumulated) result:
    coordinates bit-exact, values within the dtype's tolerance."""
    note("workload end-to-end", name, "fused =", fused)
    if name == "blocksparse_1k":
        w = G.workload_blocksparse_1k()
    elif name == "order3_small":
        w = G.workload_order3(n=512, l=128, density=0.02)
    elif name == "banded_small":
        w = G.workload_batched_banded(b=2, n=1024)
    else:
        w = G.workload_sparse_sparse_zipf(n=4096)
    want = R.execute_sparse(w["lhs"], w["rhs"], w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    lhs, rhs = dev_rel(w["lhs"], w["dtype"]), dev_rel(w["rhs"], w["dtype"])
    got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            fused=fused)
    assert got.is_device
    npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
    assert got.values.dtype == (torch.bfloat16 if w["dtype"] == "bf16" else torch.float32)
    err = R.rel_l2(hv(got.values), want.values)
    assert err <= TOL[w["dtype"]], err
    # host inputs give host outputs with the same content
    if name == "blocksparse_1k" and fused:
        h = ej.execute_sparse(host_rel(w["lhs"]), host_rel(w["rhs"]), w["join_keys"],
                              w["kernel_string"], w["agg_keys"])
        assert isinstance(h.values, np.ndarray) and h.values.dtype == np.float32
        npt.assert_array_equal(h.coords, want.coords)
        npt.assert_array_equal(h.values, got.values.cpu().numpy())


@pytest.mark.parametrize("name", ["blocksparse_1k", "order3_small", "zipf_small", "zipf_small_bf16"])
def test_queued_step_matches_exact_path(gpu, name, monkeypatch):
    """A repeated execute_sparse on the same relations queues its whole step
    on the pair count remembered from the previous call.  Its output must be
    bit-identical to the exact path's, with the remembered bound equal to,
    below (falls back to the exact path) and far above the true count."""
    note("queued step", name)
    if name == "blocksparse_1k":
        w = G.workload_blocksparse_1k()
    elif name == "order3_small":
        w = G.workload_order3(n=512, l=128, density=0.02)
    elif name == "zipf_small_bf16":  # one segment per workgroup on the bf16 DMA kernel
        w = dict(G.workload_sparse_sparse_zipf(n=4096), dtype="bf16")
    else:
        w = G.workload_sparse_sparse_zipf(n=4096)
    statuses = []
    real = _device_mod().run_queued_step

    def spy(*a, **k):
        st, res = real(*a, **k)
        statuses.append(st)
        return st, res

    monkeypatch.setattr(_device_mod(), "run_queued_step", spy)
    monkeypatch.setattr(sd, "_dense_step", lambda *a, **k: None)  # the general queued plan
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)
    sd._pair_hints.clear()
    sd._steps.clear()
    lhs, rhs = dev_rel(w["lhs"], w["dtype"]), dev_rel(w["rhs"], w["dtype"])
    run = lambda: ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    exact = run()
    assert statuses == [] and len(sd._pair_hints) == 1
    key = next(iter(sd._pair_hints))
    P = sd._hint_get(key, lhs, rhs)
    ref_c, ref_v = exact.coords.cpu().numpy(), hv(exact.values)
    want = R.execute_sparse(w["lhs"], w["rhs"], w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    npt.assert_array_equal(ref_c, want.coords)
    assert R.rel_l2(ref_v, want.values) <= TOL[w["dtype"]]
    for bound, status in [(P, "ok"), (max(P - 1, 1), "bound"), (3 * P + 7, "ok")]:
        sd._hint_set(key, lhs, rhs, bound)
        sd._steps.clear()  # the hint, not a prepared step, bounds this call
        got = run()
        assert statuses[-1] == status, (bound, statuses)
        npt.assert_array_equal(got.coords.cpu().numpy(), ref_c)
        npt.assert_array_equal(hv(got.values), ref_v)
        assert got.values.shape == exact.values.shape
        assert sd._hint_get(key, lhs, rhs) == P
    # Timing events around the queued einsum launch leave the result as it is.
    evs = []
    got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            _einsum_events=evs)
    assert statuses[-1] == "ok" and len(evs) == 1
    npt.assert_array_equal(hv(got.values), ref_v)
    assert evs[0][0].elapsed_time(evs[0][1]) > 0


def test_queued_step_range_fallback(gpu, monkeypatch):
    """Relations whose shape metadata understates their coordinates: the
    queued step detects the out-of-range keys, the exact path (radices from
    the data) answers, and the queued path is not tried again."""
    note("queued step range fallback")
    w = G.workload_blocksparse_1k()
    statuses = []
    real = _device_mod().run_queued_step

    def spy(*a, **k):
        st, res = real(*a, **k)
        statuses.append(st)
        return st, res

    monkeypatch.setattr(_device_mod(), "run_queued_step", spy)
    sd._pair_hints.clear()
    sd._steps.clear()
    L, Rr = w["lhs"], w["rhs"]
    small = lambda r: R.Rel(r.coords, r.values, r.tile_shape, r.tile_shape)
    lhs, rhs = dev_rel(small(L), w["dtype"]), dev_rel(small(Rr), w["dtype"])
    want = R.execute_sparse(L, Rr, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            precision="fp64")
    for _ in range(3):
        got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
        npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
        assert R.rel_l2(hv(got.values), want.values) <= TOL[w["dtype"]]
    assert statuses == ["range"]


def test_queued_step_large_join(gpu, monkeypatch):
    """The queued step with a build side above the one-workgroup join (the
    full-size Zipf workload, 20,971 lhs tiles, 54,516 pairs): bit-identical to
    the exact path; with shape metadata that understates the coordinates the
    range flag sends it to the exact path."""
    note("queued step, large join")
    statuses = []
    real = _device_mod().run_queued_step

    def spy(*a, **k):
        st, res = real(*a, **k)
        statuses.append(st)
        return st, res

    monkeypatch.setattr(_device_mod(), "run_queued_step", spy)
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)  # the general queued plan
    w = G.workload_sparse_sparse_zipf(values=False)
    gen = torch.Generator(device="cuda").manual_seed(4)

    def rel(r, shape):
        v = torch.rand((len(r.coords), *r.tile_shape), generator=gen, device="cuda") * 2 - 1
        return SparseTensorRelation(torch.from_numpy(r.coords).cuda(), v, shape, r.tile_shape)

    lhs, rhs = rel(w["lhs"], w["lhs"].shape), rel(w["rhs"], w["rhs"].shape)
    assert lhs.num_tuples > 4096
    run = lambda a, b: ej.execute_sparse(a, b, w["join_keys"], w["kernel_string"], w["agg_keys"])
    sd._pair_hints.clear()
    sd._steps.clear()
    exact = run(lhs, rhs)
    queued = run(lhs, rhs)
    assert statuses == ["ok"]
    assert torch.equal(exact.coords, queued.coords)
    assert torch.equal(exact.values.view(torch.int32), queued.values.view(torch.int32))
    oc_lhs = SparseTensorRelation(lhs.coords, lhs.values, lhs.tile_shape, lhs.tile_shape)
    oc_rhs = SparseTensorRelation(rhs.coords, rhs.values, rhs.tile_shape, rhs.tile_shape)
    sd._pair_hints.clear()
    sd._steps.clear()
    for _ in range(2):
        got = run(oc_lhs, oc_rhs)
        assert torch.equal(got.coords, exact.coords)
        assert torch.equal(got.values.view(torch.int32), exact.values.view(torch.int32))
    assert statuses == ["ok", "range"]


@pytest.mark.parametrize("n_lhs,n_rhs,grid,slack", [
    (300, 500, 40, 0), (50, 60, 2, 3), (700, 1800, 64, 9), (1000, 2100, 64, 0),  # one pass
    (1000, 2100, 64, 100), (1000, 3000, 90, 0), (1000, 8000, 64, 11), (1000, 3000, 100, 7),
    (3000, 8000, 64, 5), (4000, 8192, 48, 1000), (6000, 9000, 80, 0)])
def test_pair_plan_matches_exact_phases(gpu, n_lhs, n_rhs, grid, slack):
    """ej_pair_plan_async (join count and fill, output keys, sort, flag scan
    and segment fill in one call) against the separate exact phases: pairs,
    output coordinates, offsets and permutation bit-exact.  Covered: the
    one-pass plan (output keys of 2 to 12 bits, up to 32768 pairs: 32,685
    pairs, and the same with a capacity past the limit, which takes the
    general plan), one-workgroup and general joins,
    radix sorts whose first histogram comes from the pair fill and sorts
    above the inline-offset tiling (more than 65536 pairs), with a pair
    capacity equal to P or above it."""
    note("pair plan", n_lhs, n_rhs, grid, slack)
    from einjax_amd import _device

    rng = np.random.default_rng(n_lhs + n_rhs + grid)
    lc = rng.integers(0, grid, (n_lhs, 2), dtype=np.int32)
    rc = rng.integers(0, grid, (n_rhs, 2), dtype=np.int32)
    t = lambda a: torch.from_numpy(a).cuda()
    keys, agg = [(1, 0)], [(0, 0), (1, 1)]
    li, ri = _device.join(t(lc), t(rc), keys, [grid])
    coords, off, perm, _ = _device.segment_plan(t(lc), t(rc), li, ri, agg, [grid, grid])
    P, U = li.numel(), coords.shape[0]
    desc = _device.describe("ij,jk->ik", (2, 2), (2, 2))
    vals = lambda n: torch.ones((n, 2, 2), device="cuda")
    st, res = _device.queued_segment_einsum(t(lc), t(rc), keys, [grid], agg, [grid, grid], desc,
                                            vals(n_lhs), vals(n_rhs), P + slack)
    assert st == "ok", st
    Pq, cq, oq, pq, _, liq, riq = res
    assert Pq == P
    for got, want in ((liq, li), (riq, ri), (cq, coords), (oq, off), (pq, perm)):
        assert torch.equal(got, want)
    assert U == cq.shape[0]


@pytest.mark.parametrize("m,n,density", [(2048, 512, 0.2), (4096, 1024, 0.05), (2048, 1536, 0.06),
                                         (4096, 512, 0.02)])
def test_queued_run_order_bf16_groups(gpu, m, n, density, monkeypatch):
    """Block-sparse x dense with 128^2 bf16 tiles: the queued step runs the
    grouped einsum (two output tiles per workgroup) in the plan's run order
    (groups of 2, heaviest first per XCD); its output must be bit-identical
    to the exact path's (own plan, no order), with 4 to 12 output tiles per
    row and 30 to 112 groups (66 and 30: not a multiple of the 8 XCDs).
    Grouping is forced here: below GROUP_MIN_SEGMENTS output segments the
    steps run one segment per workgroup, which writes no run order and gives
    the same bits."""
    note("queued run order bf16", m, n, density)
    dm = _device_mod()
    w = G.workload_blocksparse_16k(seed=3, m=m, n=n, density=density)
    lhs, rhs = dev_rel(w["lhs"], "bf16"), dev_rel(w["rhs"], "bf16")
    args = (lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    written = []
    lib = dm._lib.load()
    real = lib.ej_pair_plan_async

    def spy(*a):
        rc = real(*a)
        written.append((a[25], a[27]._obj.value if hasattr(a[27], "_obj") else None))
        return rc

    monkeypatch.setattr(sd, "_dense_step", lambda *a, **k: None)  # the general queued plan
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)
    monkeypatch.setattr(dm, "GROUP_MIN_SEGMENTS", 0)
    sd._pair_hints.clear()
    sd._steps.clear()
    exact = ej.execute_sparse(*args)
    monkeypatch.setattr(lib, "ej_pair_plan_async", spy)
    for _ in range(2):
        got = ej.execute_sparse(*args)
        assert torch.equal(got.coords, exact.coords)
        assert torch.equal(got.values.view(torch.int16), exact.values.view(torch.int16))
    assert written and all(g == 2 and wr == 1 for g, wr in written), written
    # the default threshold: these few segments run ungrouped
    monkeypatch.undo()
    assert dm.GROUP_MIN_SEGMENTS > (m // 128) * (n // 128)
    monkeypatch.setattr(sd, "_dense_step", lambda *a, **k: None)
    monkeypatch.setattr(sd, "_row_step", lambda *a, **k: None)
    monkeypatch.setattr(lib, "ej_pair_plan_async", spy)
    sd._steps.clear()
    written.clear()
    got = ej.execute_sparse(*args)
    assert torch.equal(got.coords, exact.coords)
    assert torch.equal(got.values.view(torch.int16), exact.values.view(torch.int16))
    assert written and all(g == 0 for g, _ in written), written


def test_run_order_header_must_match_live_groups(gpu):
    """ej_segment_einsum_async follows a run order only when its header
    (run_order[0]) equals the number of live groups; an order made for
    another group count is ignored as a whole, so every output tile is still
    written once.  A valid permutation gives the same output as no order."""
    note("run order header")
    import ctypes

    from einjax_amd import _device, _lib

    w = G.workload_blocksparse_16k(seed=5, m=2048, n=1024, density=0.2)
    lhs, rhs = dev_rel(w["lhs"], "bf16"), dev_rel(w["rhs"], "bf16")
    li, ri = sd._join_dev(lhs, rhs, w["join_keys"], lhs.coords, rhs.coords)
    coords, off, perm, _ = _device.segment_plan(lhs.coords, rhs.coords, li, ri, w["agg_keys"],
                                                [16, 8])
    U = coords.shape[0]
    desc = _device.describe("ij,jk->ik", (128, 128), (128, 128))
    desc.seg_group = 8
    desc.out_dtype = _lib.EJ_BF16
    gq = ctypes.c_int32(1)
    lib = _lib.load()
    _lib.check(lib.ej_segment_einsum_group(ctypes.byref(desc), _lib.EJ_BF16, ctypes.byref(gq)),
               "ej_segment_einsum_group")
    group = gq.value
    assert group == 2 and U == 128
    ngroups = (U + group - 1) // group
    n_dev = torch.tensor([U], dtype=torch.int64, device="cuda")

    def run(order):
        out = torch.full((U, 128, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        o = None if order is None else torch.tensor(order, dtype=torch.int32, device="cuda")
        _lib.check(lib.ej_segment_einsum_async(
            ctypes.byref(desc), _lib.EJ_BF16, _device.ptr(lhs.values), _device.ptr(rhs.values),
            lhs.values.shape[0], rhs.values.shape[0], _device.ptr(li), _device.ptr(ri),
            _device.ptr(perm), _device.ptr(off), U, _device.ptr(n_dev), _device.ptr(o), group,
            _device.ptr(out), _device.stream_ptr()), "ej_segment_einsum_async")
        torch.cuda.synchronize()
        return out

    ref = run(None)
    assert not torch.isnan(ref.float()).any()
    same = lambda x: torch.equal(x.view(torch.int16), ref.view(torch.int16))
    assert same(run([ngroups] + list(range(ngroups))[::-1]))
    rng = np.random.default_rng(1)
    assert same(run([ngroups] + rng.permutation(ngroups).tolist()))
    # made for one group more / fewer: ignored, every tile written once
    assert same(run([ngroups + 1, 1] + list(range(ngroups))))
    assert same(run([ngroups - 1] + [1, 0] + list(range(2, ngroups - 1)) + [0]))


def _device_mod():
    from einjax_amd import _device

    return _device


def test_headline_workload_full_size(gpu):
    """16384^2 block-sparse (5%, 128^2 bf16 tiles) x dense 16384x4096 at full
    size: coordinates bit-exact; the default bf16 output is the fp32 output
    rounded; the fp32 output passes a checksum of checksums (C @ x against
    A @ (B @ x) in float64), equals the unfused path's, and a row-band
    subset matches the oracle's full result."""
    note("headline workload full size")
    w = G.workload_blocksparse_16k()
    L, Rr = w["lhs"], w["rhs"]
    lhs, rhs = dev_rel(L, "bf16"), dev_rel(Rr, "bf16")
    args = (lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    fused = ej.execute_sparse(*args, out_dtype=torch.float32)
    unfused = ej.execute_sparse(*args, fused=False, out_dtype=torch.float32)
    fused16 = ej.execute_sparse(*args)
    torch.cuda.synchronize()
    assert fused.num_tuples == 4096 and fused16.values.dtype == torch.bfloat16
    npt.assert_array_equal(fused.coords.cpu().numpy(), unfused.coords.cpu().numpy())
    assert torch.equal(fused16.coords, fused.coords)
    assert torch.equal(fused16.values.view(torch.int16),
                       fused.values.to(torch.bfloat16).view(torch.int16))
    fv, uv = hv(fused.values), hv(unfused.values)
    assert R.rel_l2(fv, uv) <= 1e-5
    del unfused
    # checksum: C x == A (B x), float64 on the host
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096)
    Bx = np.zeros(16384)
    for (bi, bk), t in zip(Rr.coords, Rr.values):
        Bx[bi * 128:(bi + 1) * 128] += t.astype(np.float64) @ x[bk * 128:(bk + 1) * 128]
    ABx = np.zeros(16384)
    for (ai, aj), t in zip(L.coords, L.values):
        ABx[ai * 128:(ai + 1) * 128] += t.astype(np.float64) @ Bx[aj * 128:(aj + 1) * 128]
    Cx = np.zeros(16384)
    for (ci, ck), t in zip(fused.coords.cpu().numpy(), fv):
        Cx[ci * 128:(ci + 1) * 128] += t.astype(np.float64) @ x[ck * 128:(ck + 1) * 128]
    assert R.rel_l2(Cx, ABx) <= 1e-5
    # a band of 8 row-tiles against the oracle
    band = L.coords[:, 0] < 8
    sub = R.Rel(L.coords[band], L.values[band], L.shape, L.tile_shape)
    want = R.execute_sparse(sub, Rr, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            precision="fp64")
    rows = fused.coords.cpu().numpy()[:, 0] < 8
    npt.assert_array_equal(fused.coords.cpu().numpy()[rows], want.coords)
    assert R.rel_l2(fv[rows], want.values) <= 1e-5  # bf16 products are exact in fp32
    assert R.rel_l2(hv(fused16.values)[rows], want.values) <= TOL["bf16"]


def test_fused_is_deterministic(gpu):
    note("determinism")
    w = G.workload_sparse_sparse_zipf(n=4096)
    lhs, rhs = dev_rel(w["lhs"]), dev_rel(w["rhs"])
    a = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    b = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    assert torch.equal(a.coords, b.coords)
    assert torch.equal(a.values.view(torch.int32), b.values.view(torch.int32))


# ---------------------------------------------------------------------------
# tiling

@pytest.mark.parametrize("dtype", ["f64host", "f64dev", "f32", "bf16"])
def test_to_relation_parity(gpu, dtype):
    """Tiles keep the input's dtype: float64 host data gives float64 tiles,
    as the reference's (tensor/sparse.py:191, :210), so 1e-300 survives."""
    note("to_relation", dtype)
    rng = np.random.default_rng(4)
    d = rng.standard_normal((64, 96)) * np.kron(rng.random((8, 6)) < 0.3, np.ones((8, 16)))
    d[3, 5] = np.nan  # NaN is nonzero
    d[60, 0] = -0.0  # -0.0 is zero
    d[9, 17] = 1e-300  # nonzero in float64 only
    tile = (8, 16)
    if dtype in ("f64host", "f64dev"):
        src = d if dtype == "f64host" else torch.from_numpy(d).cuda()
        want = R.dense_to_relation(d, tile)
    else:
        f = d.astype(np.float32)
        if dtype == "bf16":
            f = R.bf16_round(f)
        want = R.dense_to_relation(f.astype(np.float64), tile)
        t = torch.from_numpy(f).cuda()
        src = t.to(torch.bfloat16) if dtype == "bf16" else t
    got = SparseTensor("x", src).to_relation(tile)
    gc = got.coords.cpu().numpy() if dtype != "f64host" else got.coords
    if dtype == "f64host":
        gv = got.values
        assert isinstance(gv, np.ndarray) and gv.dtype == np.float64
    elif dtype == "f64dev":
        assert got.values.dtype == torch.float64 and got.is_device
        gv = got.values.cpu().numpy()
    else:
        gv = got.values.float().cpu().numpy()
    npt.assert_array_equal(gc, want.coords)
    exact = want.values if dtype.startswith("f64") else want.values.astype(np.float32)
    npt.assert_array_equal(gv, exact)  # NaN == NaN, +0.0 for zeros
    assert not np.any(np.signbit(gv[gv == 0]))
    if dtype.startswith("f64"):
        assert (gv == 1e-300).sum() == 1
        # the device relation's to_dense gives back the float64 values
        dev = got if dtype == "f64dev" else got.to_device(torch.float64)
        npt.assert_array_equal(dev.to_dense().cpu().numpy(), R.relation_to_dense(want))


def test_to_relation_edge_cases(gpu):
    note("to_relation edges")
    with pytest.raises(ValueError):
        SparseTensor("x", np.eye(3)).to_relation((2, 2))
    r = SparseTensor("z", np.zeros((4, 4))).to_relation((2, 2))
    assert r.coords.shape == (0, 2) and r.values.shape == (0, 2, 2)
    d = np.zeros((4, 4, 4)); d[0, 0, 0] = 1.0; d[3, 3, 3] = 2.0
    r = SparseTensor("t3", d).to_relation((2, 2, 2))
    npt.assert_array_equal(r.coords, [[0, 0, 0], [1, 1, 1]])
    npt.assert_array_equal(r.to_dense(), d)
    r = SparseTensor("v", np.array([0.0, 1, 0, 3, 0, 0])).to_relation((2,))
    npt.assert_array_equal(r.coords, [[0], [1]])


def test_device_to_dense_roundtrip(gpu):
    note("device to_dense")
    w = G.workload_blocksparse_1k()
    rel = dev_rel(w["lhs"])
    dense = rel.to_dense()
    assert dense.is_cuda
    npt.assert_array_equal(dense.cpu().numpy(), R.relation_to_dense(w["lhs"]).astype(np.float32))
    back = SparseTensor("a", dense).to_relation((32, 32))
    assert torch.equal(back.coords, rel.coords) and torch.equal(back.values, rel.values)


@pytest.mark.parametrize("name", ["blocksparse_1k", "zipf_small"])
def test_repeated_calls_track_the_data(gpu, name):
    """A repeated execute_sparse on the same relations takes its prepared
    step (argument lists built once) and still joins, plans and multiplies
    the data as it is at each call: bitwise equal to the first call, twice
    the result after the lhs values are doubled in place, and the oracle's
    result after the lhs coordinates are replaced by another tensor."""
    note("repeated calls", name)
    w = (G.workload_blocksparse_1k() if name == "blocksparse_1k"
         else G.workload_sparse_sparse_zipf(n=4096))
    sd._steps.clear()
    sd._pair_hints.clear()
    lhs, rhs = dev_rel(w["lhs"], w["dtype"]), dev_rel(w["rhs"], w["dtype"])
    run = lambda: ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    first = [run() for _ in range(3)]
    assert len(sd._steps) == 1
    for r in first[1:]:
        assert torch.equal(r.coords, first[0].coords)
        assert torch.equal(r.values.view(torch.int32), first[0].values.view(torch.int32))
    lhs.values.mul_(2)
    doubled = run()
    assert torch.equal(doubled.coords, first[0].coords)
    assert torch.equal(doubled.values, first[0].values * 2)
    lhs.values.div_(2)
    keep = np.arange(0, len(w["lhs"].coords), 2)
    L2 = R.Rel(w["lhs"].coords[keep], w["lhs"].values[keep], w["lhs"].shape, w["lhs"].tile_shape)
    lhs.coords = torch.from_numpy(np.ascontiguousarray(L2.coords)).cuda()
    lhs.values = lhs.values[torch.from_numpy(keep).cuda()].contiguous()
    want = R.execute_sparse(L2, w["rhs"], w["join_keys"], w["kernel_string"], w["agg_keys"],
                            precision="fp64")
    for _ in range(2):
        got = run()
        npt.assert_array_equal(got.coords.cpu().numpy(), want.coords)
        assert R.rel_l2(hv(got.values), want.values) <= TOL[w["dtype"]]
