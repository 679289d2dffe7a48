"""GPU parity of the backward pass (reference: autodiff/custom_vjp.py:204-278)
against the oracle's pair_einsum_vjp, which finite differences pin.

Gradients are compared in float64 against the oracle: rel-L2 <= 1e-5 for
fp32 operands, <= 1e-2 for bf16 operands (gradients returned in bf16).  The
pair grouping (ej_index_plan) is bit-exact.
"""

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R

import einjax_amd as ej
from einjax_amd import _device as D
from einjax_amd import SparseTensor
from einjax_amd.autodiff.custom_vjp import _reverse_einsum_string

pytestmark = pytest.mark.gpu


def note(*a):
    print("[case]", *a, flush=True)


def rel_l2(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.linalg.norm(ref)
    return np.linalg.norm(x - ref) / (d if d > 0 else 1.0)


def rel_from_dense(dense, tile):
    return SparseTensor("t", np.asarray(dense, dtype=np.float64)).to_relation(tile)


# ---------------------------------------------------------------------------
# pair grouping

@pytest.mark.parametrize("n,targets", [(1, 1), (1000, 7), (70000, 5000), (5, 0),
                                       (65536, 4094), (30000, 1), (0, 9), (65537, 10),
                                       (200, 4095), (1025, 3), (40000, 16127), (40000, 16128),
                                       (3000, 200000), (32768, 4863), (32769, 100),
                                       (20000, 4864), (2, 4863), (32768, 0), (26208, 4096)])
def test_index_plan_parity(gpu, n, targets):
    note("index_plan", n, targets)
    rng = np.random.default_rng(n)
    idx = rng.integers(-2, targets + 3, size=n).astype(np.int64)
    perm, off = D.index_plan(torch.from_numpy(idx).cuda(), targets)
    key = np.where((idx >= 0) & (idx < targets), idx, targets)
    npt.assert_array_equal(perm.cpu().numpy(), np.argsort(key, kind="stable"))
    npt.assert_array_equal(off.cpu().numpy(), np.searchsorted(np.sort(key), np.arange(targets + 1)))


# ---------------------------------------------------------------------------
# the reference's own cases (tests/test_autodiff.py:157-476), through torch
# autograd, against the oracle's backward

def grads_of(A, B, tile, join_keys, spec, loss, need=(True, True)):
    lhs, rhs = rel_from_dense(A, tile[0]), rel_from_dense(B, tile[1])
    li, ri = ej.coordinate_join(lhs, rhs, join_keys)
    lv = torch.from_numpy(lhs.values.astype(np.float32)).cuda().requires_grad_(need[0])
    rv = torch.from_numpy(rhs.values.astype(np.float32)).cuda().requires_grad_(need[1])
    out = ej.sparse_einsum_raw(lv, rv, lhs.coords, rhs.coords, li, ri, spec)
    val = loss(out)
    val.backward()
    return lhs, rhs, li, ri, out, val, lv.grad, rv.grad


def test_reference_grad_cases(gpu):
    note("reference grad cases")
    A = np.array([[1.0, 2.0], [3.0, 4.0]])
    B = np.array([[5.0, 6.0], [7.0, 8.0]])
    # test_grad_lhs_matmul / test_grad_rhs_matmul: loss = sum(out)
    lhs, rhs, li, ri, out, _, gl, gr = grads_of(A, B, ((2, 2), (2, 2)), [(1, 0)], "ij,jk->ik",
                                                lambda o: o.sum())
    wl, wr = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik",
                               np.ones(tuple(out.shape)))
    npt.assert_allclose(gl.cpu().numpy(), wl, rtol=1e-6)
    npt.assert_allclose(gr.cpu().numpy(), wr, rtol=1e-6)
    npt.assert_allclose(gl.cpu().numpy()[0], np.ones((2, 2)) @ B.T)
    # test_grad_both_sides: value_and_grad of sum(out ** 2), (1, 1) tiles
    A2, B2 = np.array([[1.0, 0.0], [0.0, 2.0]]), np.array([[3.0, 0.0], [0.0, 4.0]])
    lhs, rhs, li, ri, out, val, gl, gr = grads_of(A2, B2, ((1, 1), (1, 1)), [(1, 0)],
                                                  "ij,jk->ik", lambda o: (o ** 2).sum())
    npt.assert_allclose(val.item(), np.sum((A2 @ B2) ** 2), atol=1e-5)
    o64 = R.kernel_einsum(lhs.values, rhs.values, li, ri, "ij,jk->ik", precision="fp64")
    wl, wr = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik", 2 * o64)
    npt.assert_allclose(gl.cpu().numpy(), wl, rtol=1e-6)
    npt.assert_allclose(gr.cpu().numpy(), wr, rtol=1e-6)
    # test_grad_sparse_diagonal
    lhs, rhs, li, ri, out, _, gl, _ = grads_of(np.diag([1.0, 2, 3, 4]), np.diag([5.0, 6, 7, 8]),
                                               ((2, 2), (2, 2)), [(1, 0)], "ij,jk->ik",
                                               lambda o: o.sum(), need=(True, False))
    wl, _ = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik",
                              np.ones(tuple(out.shape)))
    npt.assert_allclose(gl.cpu().numpy(), wl, rtol=1e-6)
    # test_grad_weighted_loss
    W = torch.tensor([[1.0, 2.0], [3.0, 4.0]], device="cuda")
    lhs, rhs, li, ri, out, _, gl, _ = grads_of(A, B, ((2, 2), (2, 2)), [(1, 0)], "ij,jk->ik",
                                               lambda o: (o[0] * W).sum(), need=(True, False))
    wl, _ = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik",
                              W.cpu().numpy()[None].astype(np.float64))
    npt.assert_allclose(gl.cpu().numpy(), wl, rtol=1e-6)
    # test_tile_in_multiple_matches
    A3 = np.zeros((4, 4)); A3[0, 0], A3[0, 2] = 1.0, 2.0
    B3 = np.zeros((4, 4)); B3[0, 0], B3[2, 0] = 3.0, 4.0
    lhs, rhs, li, ri, out, _, gl, _ = grads_of(A3, B3, ((2, 2), (2, 2)), [(1, 0)], "ij,jk->ik",
                                               lambda o: o.sum(), need=(True, False))
    wl, _ = R.pair_einsum_vjp(lhs.values, rhs.values, li, ri, "ij,jk->ik",
                              np.ones(tuple(out.shape)))
    npt.assert_allclose(gl.cpu().numpy(), wl, rtol=1e-6)
    # test_grad_shape_matches_input
    lhs, rhs, li, ri, out, _, gl, gr = grads_of(np.eye(4), np.eye(4), ((2, 2), (2, 2)), [(1, 0)],
                                                "ij,jk->ik", lambda o: o.sum())
    assert gl.shape == tuple(lhs.values.shape) and gr.shape == tuple(rhs.values.shape)
    # test_outer_product_grad: no join keys, "ij,kl->ijkl"
    a, b = np.array([[1.0], [2.0]]), np.array([[3.0], [4.0]])
    lhs, rhs, li, ri, out, _, gl, _ = grads_of(a, b, ((1, 1), (1, 1)), [], "ij,kl->ijkl",
                                               lambda o: o.sum(), need=(True, False))
    npt.assert_allclose(gl.cpu().numpy().reshape(-1), [7.0, 7.0])


def test_reverse_strings_and_errors(gpu):
    assert _reverse_einsum_string("ij,jk->ik") == ("ik,jk->ij", "ij,ik->jk")
    assert _reverse_einsum_string("i,i->") == (",i->i", "i,->i")
    with pytest.raises(ValueError):
        _reverse_einsum_string("ij,jk")
    # "ij,jk->k": the lhs label i appears in neither the cotangent nor the rhs
    lv = torch.ones((1, 2, 2), device="cuda")
    with pytest.raises(ValueError):
        ej.sparse_einsum_raw_vjp(lv, lv, [0], [0], "ij,jk->k", torch.ones((1, 2), device="cuda"))


# ---------------------------------------------------------------------------
# random cases against the oracle

SPECS = [("ij,jk->ik", (32, 64), (64, 32)), ("ij,kj->ik", (16, 32), (48, 32)),
         ("bij,bjk->bik", (1, 64, 32), (1, 32, 64)), ("ij,kl->ijkl", (4, 3), (2, 5)),
         ("i,i->", (16,), (16,)), ("ij,ij->ij", (8, 16), (8, 16)),
         ("ijk,kl->ijl", (8, 8, 32), (32, 16)), ("ij,jk->ik", (128, 128), (128, 128))]


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "bf16-bf16"])
@pytest.mark.parametrize("spec,lt,rt", SPECS)
def test_vjp_parity(gpu, dtype, spec, lt, rt):
    """dtype: operand values' dtype; "bf16-bf16" also hands in a bf16
    cotangent (bf16 gradient einsums), the others an fp32 one."""
    note("vjp", dtype, spec, lt, rt)
    g_bf16 = dtype == "bf16-bf16"
    dtype = "bf16" if g_bf16 else dtype
    rng = np.random.default_rng(len(spec) + lt[0])
    nl, nr, P = 13, 9, 60
    L = rng.standard_normal((nl, *lt)).astype(np.float32)
    Rv = rng.standard_normal((nr, *rt)).astype(np.float32)
    if dtype == "bf16":
        L, Rv = R.bf16_round(L), R.bf16_round(Rv)
    li = rng.integers(0, nl - 2, P)   # the last two lhs tiles are in no pair
    ri = rng.integers(0, nr, P)
    out_shape = R.kernel_einsum(L, Rv, li, ri, spec, precision="fp64").shape
    g = rng.standard_normal(out_shape).astype(np.float32)
    if g_bf16:
        g = R.bf16_round(g)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    lv = torch.from_numpy(L).cuda().to(tdt)
    rv = torch.from_numpy(Rv).cuda().to(tdt)
    gt = torch.from_numpy(g).cuda()
    gl, gr = ej.sparse_einsum_raw_vjp(lv, rv, torch.from_numpy(li).cuda(),
                                      torch.from_numpy(ri).cuda(), spec,
                                      gt.to(torch.bfloat16) if g_bf16 else gt)
    assert gl.dtype == tdt and gr.dtype == tdt
    wl, wr = R.pair_einsum_vjp(L, Rv, li, ri, spec, g)
    tol = 1e-5 if dtype == "fp32" else 1e-2
    assert rel_l2(gl.float().cpu().numpy(), wl) <= tol
    assert rel_l2(gr.float().cpu().numpy(), wr) <= tol
    assert torch.all(gl[nl - 2:] == 0)


def test_vjp_through_autograd_bf16_and_determinism(gpu):
    note("autograd bf16")
    rng = np.random.default_rng(5)
    L = R.bf16_round(rng.standard_normal((6, 64, 64)).astype(np.float32))
    Rv = R.bf16_round(rng.standard_normal((5, 64, 64)).astype(np.float32))
    li, ri = rng.integers(0, 6, 40), rng.integers(0, 5, 40)
    lv = torch.from_numpy(L).cuda().to(torch.bfloat16).requires_grad_()
    rv = torch.from_numpy(Rv).cuda().to(torch.bfloat16).requires_grad_()
    out = ej.sparse_einsum_raw(lv, rv, None, None, li, ri, "ij,jk->ik")
    assert out.dtype == torch.bfloat16  # the values' dtype, as jnp.einsum returns
    W = torch.from_numpy(R.bf16_round(rng.standard_normal(tuple(out.shape)).astype(
        np.float32))).cuda()
    (out * W.to(torch.bfloat16)).sum().backward()  # cotangent W, in bf16
    assert lv.grad.dtype == torch.bfloat16 and rv.grad.dtype == torch.bfloat16
    wl, wr = R.pair_einsum_vjp(L, Rv, li, ri, "ij,jk->ik", W.cpu().numpy())
    assert rel_l2(lv.grad.float().cpu().numpy(), wl) <= 1e-2
    assert rel_l2(rv.grad.float().cpu().numpy(), wr) <= 1e-2
    a = ej.sparse_einsum_raw_vjp(lv.detach(), rv.detach(), li, ri, "ij,jk->ik", W)
    b = ej.sparse_einsum_raw_vjp(lv.detach(), rv.detach(), li, ri, "ij,jk->ik", W)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_vjp_empty_and_host(gpu):
    note("vjp empty / host")
    L = np.ones((3, 2, 2), np.float32)
    gl, gr = ej.sparse_einsum_raw_vjp(L, L, np.zeros(0, np.int64), np.zeros(0, np.int64),
                                      "ij,jk->ik", np.zeros((0, 2, 2), np.float32))
    assert isinstance(gl, np.ndarray) and gl.shape == (3, 2, 2) and not gl.any() and not gr.any()
    out = ej.sparse_einsum_raw(L, L, None, None, np.array([0, 2]), np.array([1, 1]), "ij,jk->ik")
    assert isinstance(out, np.ndarray) and out.shape == (2, 2, 2)
    npt.assert_allclose(out, np.full((2, 2, 2), 2.0))


def test_sparse_einsum_high_level(gpu):
    """tests/test_autodiff.py:484-530."""
    note("sparse_einsum high level")
    r = ej.sparse_einsum(rel_from_dense(np.eye(2), (1, 1)), rel_from_dense(np.eye(2), (1, 1)),
                         join_keys=[(1, 0)], kernel_string="ij,jk->ik", agg_keys=[(0, 0), (1, 1)])
    assert isinstance(r, ej.SparseTensorRelation)
    r = ej.sparse_einsum(rel_from_dense(np.eye(4), (2, 2)), rel_from_dense(np.ones((4, 6)), (2, 3)),
                         join_keys=[(1, 0)], kernel_string="ij,jk->ik", agg_keys=[(0, 0), (1, 1)])
    assert r.shape == (4, 6)
    npt.assert_allclose(r.to_dense(), np.ones((4, 6)))
    r = ej.sparse_einsum(rel_from_dense(np.eye(4), (2, 2)), rel_from_dense(np.eye(4), (2, 2)),
                         join_keys=[(1, 0)], kernel_string="ij,jk->ik", agg_keys=[(0, 0), (1, 1)],
                         output_shape=(4, 4), output_tile_shape=(2, 2))
    assert r.shape == (4, 4) and r.tile_shape == (2, 2)


# ---------------------------------------------------------------------------
# the headline workload at full size

def test_vjp_blocksparse_16k_adjoint_and_rows(gpu):
    """Backward of the 16384^2 bf16 block-sparse x dense product (26,208
    pairs): the adjoint identity <g, f(dL, R)> = <grad_L, dL> (and the same
    for R) with f the forward tile einsum, plus a few lhs and rhs tiles
    against the oracle."""
    w = G.workload_blocksparse_16k(values=False)
    L, Rr = w["lhs"], w["rhs"]
    note("vjp blocksparse 16k")
    gen = torch.Generator(device="cuda").manual_seed(0)
    lv = torch.randn((len(L.coords), 128, 128), generator=gen, device="cuda").to(torch.bfloat16)
    rv = (torch.randn((len(Rr.coords), 128, 128), generator=gen, device="cuda") / 128).to(
        torch.bfloat16)
    lc, rc = torch.from_numpy(L.coords).cuda(), torch.from_numpy(Rr.coords).cuda()
    li, ri = ej.coordinate_join(ej.SparseTensorRelation(lc, lv, L.shape, L.tile_shape),
                                ej.SparseTensorRelation(rc, rv, Rr.shape, Rr.tile_shape),
                                w["join_keys"])
    assert li.numel() == 26208
    g = torch.randn((li.numel(), 128, 128), generator=gen, device="cuda")
    gl, gr = ej.sparse_einsum_raw_vjp(lv, rv, li, ri, "ij,jk->ik", g)
    # float32 gradients for the identity (bf16 outputs would add rounding)
    gl32, gr32 = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g)
    assert torch.equal(gl32.to(torch.bfloat16), gl) and torch.equal(gr32.to(torch.bfloat16), gr)
    dL = torch.randn(lv.shape, generator=gen, device="cuda").to(torch.bfloat16)
    dR = torch.randn(rv.shape, generator=gen, device="cuda").to(torch.bfloat16)
    desc = D.describe("ij,jk->ik", (128, 128), (128, 128))
    f32 = torch.float32
    lhs_side = (g.double() * D.pair_einsum(desc, dL, rv, li, ri, out_dtype=f32).double()).sum().item()
    rhs_side = (gl32.double() * dL.double()).sum().item()
    assert abs(lhs_side - rhs_side) <= 1e-4 * max(abs(lhs_side), 1.0)
    lhs_side = (g.double() * D.pair_einsum(desc, lv, dR, li, ri, out_dtype=f32).double()).sum().item()
    rhs_side = (gr32.double() * dR.double()).sum().item()
    assert abs(lhs_side - rhs_side) <= 1e-4 * max(abs(lhs_side), 1.0)
    # a few tiles against the oracle, from their own pairs
    li_h, ri_h = li.cpu().numpy(), ri.cpu().numpy()
    for l in (0, 400, len(L.coords) - 1):
        sel = np.nonzero(li_h == l)[0]
        want = np.zeros((128, 128))
        for p in sel:
            want += g[p].double().cpu().numpy() @ rv[ri_h[p]].double().cpu().numpy().T
        assert rel_l2(gl32[l].cpu().numpy(), want) <= 1e-5
    for r in (0, 2047, len(Rr.coords) - 1):
        sel = np.nonzero(ri_h == r)[0]
        want = np.zeros((128, 128))
        for p in sel:
            want += lv[li_h[p]].double().cpu().numpy().T @ g[p].double().cpu().numpy()
        assert rel_l2(gr32[r].cpu().numpy(), want) <= 1e-5
    # the bf16 cotangent path (bf16 gradient einsums, fp32 sums, one rounding)
    # against the fp32 path on the same rounded cotangent
    g16 = g.to(torch.bfloat16)
    gl16, gr16 = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g16)
    assert gl16.dtype == torch.bfloat16 and gr16.dtype == torch.bfloat16
    gl32b, gr32b = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g16.float())
    assert rel_l2(gl16.float().cpu().numpy(), gl32b.cpu().numpy()) <= 4e-3
    assert rel_l2(gr16.float().cpu().numpy(), gr32b.cpu().numpy()) <= 4e-3


@pytest.mark.parametrize("n_lhs,n_pairs,seed", [(700, 3000, 1), (1100, 5000, 2), (600, 900, 3)])
def test_vjp_lhs_gradient_ragged(gpu, n_lhs, n_pairs, seed):
    """The lhs gradient of 128x128 bf16 tiles (the LDS-ring one-tile-per-
    workgroup kernel with its run order) on ragged segments: many tiles with
    no pair, a few with hundreds, invalid indices on either side.  Against a
    float32 torch reference and the fp32-cotangent path; repeated calls
    bitwise equal."""
    note("vjp ragged lhs gradient", n_lhs, n_pairs, seed)
    rng = np.random.default_rng(seed)
    n_rhs = 300
    # skewed lhs targets: a few heavy tiles, many light, some with none
    heavy = rng.integers(0, n_lhs, size=8)
    li_h = np.where(rng.random(n_pairs) < 0.3, rng.choice(heavy, size=n_pairs),
                    rng.integers(0, n_lhs, size=n_pairs)).astype(np.int64)
    li_h[rng.random(n_pairs) < 0.01] = -1
    li_h[rng.random(n_pairs) < 0.01] = n_lhs + 5
    ri_h = rng.integers(0, n_rhs, size=n_pairs).astype(np.int64)
    ri_h[rng.random(n_pairs) < 0.01] = -3
    gen = torch.Generator(device="cuda").manual_seed(seed)
    lv = torch.randn((n_lhs, 128, 128), generator=gen, device="cuda").to(torch.bfloat16)
    rv = (torch.randn((n_rhs, 128, 128), generator=gen, device="cuda") / 16).to(torch.bfloat16)
    g = torch.randn((n_pairs, 128, 128), generator=gen, device="cuda").to(torch.bfloat16)
    li, ri = torch.from_numpy(li_h).cuda(), torch.from_numpy(ri_h).cuda()
    gl16, _ = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g, need_rhs=False)
    again, _ = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g, need_rhs=False)
    assert torch.equal(gl16, again)
    gl32, _ = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g.float(), need_rhs=False)
    assert rel_l2(gl16.float().cpu().numpy(), gl32.cpu().numpy()) <= 4e-3
    ok = (li_h >= 0) & (li_h < n_lhs) & (ri_h >= 0) & (ri_h < n_rhs)
    sel = torch.from_numpy(np.nonzero(ok)[0]).cuda()
    prod = torch.bmm(g[sel].float(), rv[ri[sel]].float().transpose(1, 2).contiguous())
    want = torch.zeros((n_lhs, 128, 128), device="cuda").index_add_(0, li[sel], prod)
    assert rel_l2(gl16.float().cpu().numpy(), want.cpu().numpy()) <= 1e-2
    untouched = np.setdiff1d(np.arange(n_lhs), li_h[ok])
    assert untouched.size > 0 and not gl16[torch.from_numpy(untouched).cuda()].any()
    # an fp32 cotangent with full 24-bit significands: the lhs gradient splits
    # it into three bf16 terms in the kernel; against float64
    g32 = torch.randn((n_pairs, 128, 128), generator=gen, device="cuda")
    gl, _ = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g32, need_rhs=False)
    assert gl.dtype == torch.float32
    prod64 = torch.bmm(g32[sel].double(), rv[ri[sel]].double().transpose(1, 2).contiguous())
    want64 = torch.zeros((n_lhs, 128, 128), dtype=torch.float64, device="cuda").index_add_(
        0, li[sel], prod64)
    assert rel_l2(gl.cpu().numpy(), want64.cpu().numpy()) <= 1e-5
    assert not gl[torch.from_numpy(untouched).cuda()].any()
    # and the rhs gradient under it (the cotangent split as the rhs of
    # 'ij,ik->jk', whose lhs tiles are read transposed)
    _, gr = D.pair_einsum_vjp("ij,jk->ik", lv, rv, li, ri, g32, need_lhs=False)
    assert gr.dtype == torch.float32
    prodr = torch.bmm(lv[li[sel]].double().transpose(1, 2).contiguous(), g32[sel].double())
    wantr = torch.zeros((n_rhs, 128, 128), dtype=torch.float64, device="cuda").index_add_(
        0, ri[sel], prodr)
    assert rel_l2(gr.cpu().numpy(), wantr.cpu().numpy()) <= 1e-5
    untouched_r = np.setdiff1d(np.arange(n_rhs), ri_h[ok])
    if untouched_r.size:
        assert not gr[torch.from_numpy(untouched_r).cuda()].any()
