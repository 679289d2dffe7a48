"""Value parity at the full benchmark sizes of the three non-headline workloads
(sparse x sparse Zipf 32768^2 fp32, batched banded b=32 4096 bf16, order-3
2048^3 x 2048x512 fp32), through the default fused execute_sparse
(reference: execution/sparse_dispatch.py:226-297).

Each test checks, at the full size:
  - output coordinates bit-exact (against the oracle's join + segment plan,
    or the closed form where the output is every tile of its grid);
  - a float64 checksum of checksums: C x against A (B x) for a random x
    contracted with the output's last dimension;
  - a band of output tiles against the oracle's float64 execute_sparse
    (the whole result for the Zipf workload, whose heaviest output tiles sum
    20 pairs).
The headline workload's full-size test is in test_gpu_parity.py.
"""

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import generators as G
from oracle import reference_path as R

import einjax_amd as ej
from einjax_amd import SparseTensorRelation

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 1e-2}


def note(*a):
    print("[case]", *a, flush=True)


def _dev(r: R.Rel, values: torch.Tensor) -> SparseTensorRelation:
    return SparseTensorRelation(torch.from_numpy(r.coords).cuda(), values, r.shape, r.tile_shape)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _sub(r: R.Rel, mask, values: np.ndarray) -> R.Rel:
    return R.Rel(r.coords[mask], values, r.shape, r.tile_shape)


def test_zipf_sparse_x_sparse_full_size(gpu):
    """32768^2 x 32768^2 fp32, 64^2 tiles, 2% tile density with Zipf(1.2)
    row occupancy: 5,243 tiles a side, 54,516 pairs, 31,573 output tiles of
    1 to 20 pairs.  The whole result is compared with the oracle."""
    note("zipf full size")
    w = G.workload_sparse_sparse_zipf()
    L, Rr = w["lhs"], w["rhs"]
    lhs = _dev(L, torch.from_numpy(L.values).cuda())
    rhs = _dev(Rr, torch.from_numpy(Rr.values).cuda())
    got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    assert got.values.dtype == torch.float32
    gc, gv = got.coords.cpu().numpy(), _host(got.values)
    li, ri = R.coordinate_join(L.coords, Rr.coords, w["join_keys"])
    oc = R.compute_output_coords(L.coords, Rr.coords, li, ri, w["agg_keys"])
    uc, _, off, _ = R.segment_plan(oc)
    assert len(li) == 54516 and int(np.diff(off).max()) == 20
    npt.assert_array_equal(gc, uc)
    want = R.execute_sparse(L, Rr, w["join_keys"], w["kernel_string"], w["agg_keys"],
                            precision="fp64")
    npt.assert_array_equal(want.coords, uc)
    err = R.rel_l2(gv, want.values)
    assert err <= TOL["fp32"], err
    # the heaviest output tiles (20 pairs each) on their own
    heavy = np.nonzero(np.diff(off) == 20)[0]
    assert R.rel_l2(gv[heavy], want.values[heavy]) <= TOL["fp32"]
    # checksum of checksums: C x == A (B x) in float64
    t = 64
    x = np.random.default_rng(11).standard_normal(L.shape[0])
    xb = x.reshape(-1, t)
    Bx = np.zeros((Rr.shape[0] // t, t))
    np.add.at(Bx, Rr.coords[:, 0], np.einsum("nab,nb->na", Rr.values.astype(np.float64),
                                             xb[Rr.coords[:, 1]]))
    ABx = np.zeros((L.shape[0] // t, t))
    np.add.at(ABx, L.coords[:, 0], np.einsum("nab,nb->na", L.values.astype(np.float64),
                                             Bx[L.coords[:, 1]]))
    Cx = np.zeros_like(ABx)
    np.add.at(Cx, gc[:, 0], np.einsum("nab,nb->na", gv.astype(np.float64), xb[gc[:, 1]]))
    assert R.rel_l2(Cx, ABx) <= TOL["fp32"]


def test_batched_banded_full_size(gpu):
    """b = 32 batches of 4096^2 bf16 with 64^2 tiles, causal band of 8 tile
    diagonals on A (15,488 tiles), B dense (131,072 tiles): 991,232 pairs
    into 131,072 output tiles of 1 to 8 pairs.  Default bf16 output and
    out_dtype=float32; the bf16 output is the fp32 output rounded."""
    note("banded full size")
    w = G.workload_batched_banded(values=False)
    L, Rr = w["lhs"], w["rhs"]
    gen = torch.Generator(device="cuda").manual_seed(21)
    av = torch.randn((len(L.coords), 1, 64, 64), generator=gen, device="cuda").to(torch.bfloat16)
    bv = torch.randn((len(Rr.coords), 1, 64, 64), generator=gen, device="cuda").to(torch.bfloat16)
    lhs, rhs = _dev(L, av), _dev(Rr, bv)
    args = (lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    g32 = ej.execute_sparse(*args, out_dtype=torch.float32)
    g16 = ej.execute_sparse(*args)
    torch.cuda.synchronize()
    assert g32.values.dtype == torch.float32 and g16.values.dtype == torch.bfloat16
    # every output tile of the (32, 64, 64) grid is present, in lexicographic order
    grid = np.stack(np.unravel_index(np.arange(32 * 64 * 64), (32, 64, 64)), 1).astype(np.int32)
    npt.assert_array_equal(g32.coords.cpu().numpy(), grid)
    assert torch.equal(g16.coords, g32.coords)
    assert torch.equal(g16.values.view(torch.int16),
                       g32.values.to(torch.bfloat16).view(torch.int16))
    # bands against the oracle: batch 0 rows 0-15 (segments of 1 to 8 pairs)
    # and batch 31 rows 56-63
    a_host = _host(av)
    for b, rows in ((0, range(0, 16)), (31, range(56, 64))):
        lm = (L.coords[:, 0] == b) & np.isin(L.coords[:, 1], list(rows))
        rm = Rr.coords[:, 0] == b
        sub_l = _sub(L, lm, a_host[lm])
        sub_r = _sub(Rr, rm, _host(bv[torch.from_numpy(np.nonzero(rm)[0]).cuda()]))
        want = R.execute_sparse(sub_l, sub_r, w["join_keys"], w["kernel_string"],
                                w["agg_keys"], precision="fp64")
        sel = (grid[:, 0] == b) & np.isin(grid[:, 1], list(rows))
        npt.assert_array_equal(grid[sel], want.coords)
        idx = torch.from_numpy(np.nonzero(sel)[0]).cuda()
        assert R.rel_l2(_host(g32.values[idx]), want.values) <= TOL["fp32"]
        assert R.rel_l2(_host(g16.values[idx]), want.values) <= TOL["bf16"]
    # checksum of checksums per batch: C_b x == A_b (B_b x) in float64
    x = np.random.default_rng(12).standard_normal(4096)
    c32 = g32.values.reshape(32, 64, 64, 64, 64)  # [b, i, k, r, c]
    b4 = bv.reshape(32, 64, 64, 64, 64)
    for b in range(32):
        Bb = b4[b].float().cpu().numpy().astype(np.float64)  # [j, k, r, c]
        Bx = np.einsum("jkrc,kc->jr", Bb, x.reshape(64, 64))
        ABx = np.zeros((64, 64))
        am = L.coords[:, 0] == b
        np.add.at(ABx, L.coords[am, 1], np.einsum("nrc,nc->nr",
                                                  a_host[am, 0].astype(np.float64),
                                                  Bx[L.coords[am, 2]]))
        Cb = c32[b].cpu().numpy().astype(np.float64)
        Cx = np.einsum("ikrc,kc->ir", Cb, x.reshape(64, 64))
        assert R.rel_l2(Cx, ABx) <= TOL["fp32"], b


def test_order3_full_size(gpu):
    """X 2048^3 fp32 with 32^3 tiles at 0.5% (1,311 tiles) against W 2048x512
    dense (1,024 tiles of 32^2): 20,976 pairs into 18,016 output tiles of
    32^3 (2.36 GB), kept tiled-sparse."""
    note("order-3 full size")
    w = G.workload_order3()
    L, Rr = w["lhs"], w["rhs"]
    lhs = _dev(L, torch.from_numpy(L.values).cuda())
    rhs = _dev(Rr, torch.from_numpy(Rr.values).cuda())
    got = ej.execute_sparse(lhs, rhs, w["join_keys"], w["kernel_string"], w["agg_keys"])
    assert got.values.dtype == torch.float32 and got.tile_shape == (32, 32, 32)
    gc = got.coords.cpu().numpy()
    li, ri = R.coordinate_join(L.coords, Rr.coords, w["join_keys"])
    oc = R.compute_output_coords(L.coords, Rr.coords, li, ri, w["agg_keys"])
    uc, _, off, _ = R.segment_plan(oc)
    assert len(li) == 20976 and len(uc) == got.num_tuples
    npt.assert_array_equal(gc, uc)
    # band i < 4 against the oracle
    lm = L.coords[:, 0] < 4
    want = R.execute_sparse(_sub(L, lm, L.values[lm]), Rr, w["join_keys"], w["kernel_string"],
                            w["agg_keys"], precision="fp64")
    sel = np.nonzero(gc[:, 0] < 4)[0]
    npt.assert_array_equal(gc[sel], want.coords)
    err = R.rel_l2(_host(got.values[torch.from_numpy(sel).cuda()]), want.values)
    assert err <= TOL["fp32"], err
    # checksum of checksums: sum_l C[i,j,l] x[l] == sum_k X[i,j,k] (W x)[k]
    t = 32
    x = np.random.default_rng(13).standard_normal(Rr.shape[1])
    xb = x.reshape(-1, t)
    Wx = np.zeros((Rr.shape[0] // t, t))
    np.add.at(Wx, Rr.coords[:, 0], np.einsum("nab,nb->na", Rr.values.astype(np.float64),
                                             xb[Rr.coords[:, 1]]))
    ij_l = L.coords[:, 0].astype(np.int64) * 64 + L.coords[:, 1]
    ij_c = gc[:, 0].astype(np.int64) * 64 + gc[:, 1]
    keys = np.unique(np.concatenate([ij_l, ij_c]))
    XWx = np.zeros((len(keys), t, t))
    np.add.at(XWx, np.searchsorted(keys, ij_l),
              np.einsum("nabk,nk->nab", L.values.astype(np.float64), Wx[L.coords[:, 2]]))
    Cx = np.zeros_like(XWx)
    pos = np.searchsorted(keys, ij_c)
    for s in range(0, len(gc), 2048):  # 2.36 GB of output: contract in chunks
        chunk = got.values[s:s + 2048].cpu().numpy().astype(np.float64)
        np.add.at(Cx, pos[s:s + 2048], np.einsum("nabl,nl->nab", chunk, xb[gc[s:s + 2048, 2]]))
    assert R.rel_l2(Cx, XWx) <= TOL["fp32"]
