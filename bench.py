"""Benchmark of the tensor-relational sparse einsum on one MI355X.

Workload (the headline configuration): 'ij,jk->ik' with A a 16384 x 16384
bf16 block-sparse matrix (128 x 128 tiles, 5% of tiles nonzero, uniform,
N(0,1)) and B a dense 16384 x 4096 bf16 matrix (N(0, 1/sqrt(16384))) held as
a 128 x 128 tile relation; fp32 accumulation, bf16 output tiles (the
operands' dtype).  Synthetic, seeded (numpy default_rng(0)), resident in HBM
before timing.

A step is one execute_sparse call on the resident relations: tile join,
segment plan and the fused gather + MFMA tile GEMM + segment sum.  After the
first call the step takes its queued form (join and plan on the device,
bounded by the previous call's pair count, then the einsum, with one host wait
for the plan's counts).  value = effective TFLOP/s = nonzero-tile FLOPs
(2*M*N*K per matched pair) / step time.

Also reported: every stage timed alone with HIP events on the stream the
kernels run on (the reference's unfused phase split: join, gather, per-pair
GEMM, segment sum; plus tiling), achieved GB/s against HBM for
join+gather+segment-sum, the roofline of the dominant kernel, and the CPU
oracle timed on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 20] [--no-cpu-baseline] [--all-configs]
                       [--ingest] [--backward] [--copy-calibration]
"""

from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2516.6, "fp32": 157.3}
METRIC = "effective TFLOP/s (nnz tiles) + HBM GB/s per einsum, 1 MI355X vs host CPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


@contextlib.contextmanager
def gc_paused():
    """Python's cyclic collector paused, after one collection, for a timed
    region.  A full collection in a process holding torch takes ~50-65 ms on
    the host (170k tracked objects); the host wrapper's allocations trigger
    one every few hundred to few thousand calls, and it then lands in
    whichever timed call triggered it (a ~3 ms average over 20 calls)."""
    if not gc.isenabled():  # already paused by an enclosing region
        yield
        return
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def fused_in_step_ms(execute_sparse, lhs, rhs, jk, ks, ak, reps: int):
    """Average duration of the fused einsum as the step launches it (the
    queued form: after the device-side join and plan, with the plan's run
    order), from HIP events recorded on the launch stream around each
    launch; None when the step does not take the queued form."""
    import torch

    evs = []
    for _ in range(reps):
        execute_sparse(lhs, rhs, jk, ks, ak, _einsum_events=evs)
    torch.cuda.synchronize()
    if len(evs) < reps:
        return None
    return sum(s.elapsed_time(e) for s, e in evs) / len(evs)


def event_time_ms(fn, reps: int) -> float:
    """Average duration of fn() over reps, with HIP events on the current stream."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def warm_up(fn, ms: float = 30.0, min_calls: int = 2) -> None:
    """Calls fn until ~ms of GPU work has run (at least min_calls times):
    the GPU's clocks rise over tens of ms of sustained load."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while n < min_calls or (time.perf_counter() - t0) * 1e3 < ms:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def wall_time_ms(fn, reps: int, warm: int = 1) -> float:
    import torch

    with gc_paused():
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps


def load_traffic(kernel: str):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 --pmc
    summary (profiles/traffic.json), or None when absent."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text()).get(kernel)
        return None if d is None else float(d["hbm_bytes_per_dispatch"])
    except Exception:
        return None


def _cpu_info() -> dict:
    """The host the CPU baseline ran on: model, logical CPUs, the CPUs this
    process may use, and the BLAS / OpenMP thread settings."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    blas = []
    try:
        from threadpoolctl import threadpool_info

        blas = [{"api": i.get("internal_api"), "num_threads": i.get("num_threads")}
                for i in threadpool_info()]
    except Exception:
        pass
    env = {k: os.environ[k] for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS",
                                      "MKL_NUM_THREADS", "XLA_FLAGS") if k in os.environ}
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(),
            "sched_getaffinity": len(os.sched_getaffinity(0)), "blas_threadpools": blas,
            "thread_env": env}


def cpu_baseline(w, band_tiles: int, min_seconds: float = 10.0):
    """The oracle (NumPy restatement of the reference path, fp32 math) over
    bands of `band_tiles` A row tiles, cycling through the whole workload
    until at least min_seconds of CPU work have been timed.  Each band runs
    the reference's phases one after another, each timed on its own
    (reference: sparse_dispatch.py:29-171 and tensor/sparse.py:160-219):
    bucketing of the band's dense rows into tiles, the dict hash join, the
    gather of the matched tiles, the batched fp32 tile einsum, the output
    coordinates and the sequential segment sum.  value counts the phases of
    execute_sparse (join to segment sum); bucketing is reported beside it."""
    from oracle import reference_path as R
    from oracle import workload as W

    info = _cpu_info()
    cores = max([b["num_threads"] or 1 for b in info["blas_threadpools"]] or [1])
    L, Rr = w["lhs"], w["rhs"]
    tm, tk = L.tile_shape
    n_bands = -(-(L.shape[0] // tm) // band_tiles)
    bands = []
    for b in range(n_bands):
        sel = (L.coords[:, 0] >= b * band_tiles) & (L.coords[:, 0] < (b + 1) * band_tiles)
        bands.append(R.Rel(L.coords[sel], L.values[sel], L.shape, L.tile_shape))
    phases = dict.fromkeys(["bucketing", "join", "gather", "einsum", "output_coords",
                            "segment_sum"], 0.0)
    flops = 0.0
    n_runs = 0
    t = 0.0
    rv32 = Rr.values.astype(np.float32)
    # Bucketing (np.nonzero + np.unique over the band's nonzeros) is slow in
    # NumPy: it is timed on the first band only and scaled to the workload.
    sub = bands[0]
    dense = np.zeros((band_tiles * tm, L.shape[1]))
    for (i, j), v in zip(sub.coords, sub.values):
        dense[i * tm:(i + 1) * tm, j * tk:(j + 1) * tk] = v
    t0 = time.perf_counter()
    R.dense_to_relation(dense, L.tile_shape)
    t_bucket_band = time.perf_counter() - t0
    del dense
    while t < min_seconds:
        sub = bands[n_runs % n_bands]
        t1 = time.perf_counter()
        li, ri = R.coordinate_join(sub.coords, Rr.coords, w["join_keys"])
        t2 = time.perf_counter()
        ga = sub.values.astype(np.float32)[li]
        gb = rv32[ri]
        t3 = time.perf_counter()
        tiles = R.batched_einsum(R.add_batch_dim(w["kernel_string"]), ga, gb)
        t4 = time.perf_counter()
        oc = R.compute_output_coords(sub.coords, Rr.coords, li, ri, w["agg_keys"])
        t5 = time.perf_counter()
        R.segment_sum(tiles, oc)
        t6 = time.perf_counter()
        for k, dt in zip(list(phases)[1:], (t2 - t1, t3 - t2, t4 - t3, t5 - t4, t6 - t5)):
            phases[k] += dt
        t += t6 - t1
        flops += W.flops_gemm(w["kernel_string"], L.tile_shape, Rr.tile_shape, len(li))
        n_runs += 1
        del ga, gb, tiles
    phases["bucketing"] = t_bucket_band * n_runs
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": int(cores),
        "kind": "port",
        "sample": (f"{n_runs} runs of the oracle's phases, each on a band of {band_tiles} "
                   f"A row tiles x full B, cycling over the {n_bands} bands "
                   f"({n_runs / n_bands:.2f} x the whole workload, {flops / 1e9:.0f} GFLOP); "
                   f"join to segment sum {t:.1f} s; bucketing, beside it, timed on one band "
                   f"({t_bucket_band:.1f} s) and counted once per run"),
        "phases_s": phases,
        "phase_frac": {k: v / t for k, v in phases.items() if k != "bucketing"},
        "einsum_tflops": flops / phases["einsum"] / 1e12,
        "host": info,
        "excluded": "per-tile-shape statistics (_compute_sparsity_metrics), construction "
                    "metadata, as the reference computes them before execute_sparse",
    }


CONFIG_NAMES = ["blocksparse_1k", "blocksparse_16k_bf16", "sparse_sparse_zipf",
                "batched_banded_bf16", "order3"]


def measure_config(name: str, reps: int = 20, warm: int = 10) -> dict:
    """One workload at full size: the execute_sparse step (wall clock) and
    the fused segment einsum alone (HIP events), with the effective TFLOP/s,
    the MFMA fraction and the compulsory-byte rate of the fused kernel.
    Coordinates come from the seeded generator; tile values are drawn on the
    GPU (N(0,1), or U(-1,1) for the Zipf workload) since only timing is
    reported here (parity at these shapes is the test suite's job)."""
    import torch

    from einjax_amd import SparseTensorRelation, _device, execute_sparse
    from einjax_amd.execution import sparse_dispatch as sd
    from oracle import generators as G
    from oracle import workload as W

    w = G.WORKLOADS[name](values=False)
    L, Rr = w["lhs"], w["rhs"]
    bf16 = w["dtype"] == "bf16"
    dt = torch.bfloat16 if bf16 else torch.float32
    gen = torch.Generator(device="cuda").manual_seed(0)
    uniform = name == "sparse_sparse_zipf"

    def dev(r):
        shape = (r.coords.shape[0], *r.tile_shape)
        v = torch.rand(shape, generator=gen, device="cuda") * 2 - 1 if uniform else \
            torch.randn(shape, generator=gen, device="cuda")
        return SparseTensorRelation(torch.from_numpy(r.coords).cuda(), v.to(dt), r.shape,
                                    r.tile_shape)

    lhs, rhs = dev(L), dev(Rr)
    jk, ak, ks = w["join_keys"], w["agg_keys"], w["kernel_string"]

    def step():
        return execute_sparse(lhs, rhs, jk, ks, ak)

    with gc_paused():
        warm_up(step, min_calls=warm)
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        ms_step = (time.perf_counter() - t0) * 1e3 / reps
    lc, rc = lhs.coords, rhs.coords
    li, ri = sd._join_dev(lhs, rhs, jk, lc, rc)
    P = li.numel()
    radices = [sd._grid(lhs if s == 0 else rhs, d) for s, d in ak]
    coords, offs, perm, _ = _device.segment_plan(lc, rc, li, ri, ak, radices)
    U = coords.shape[0]
    desc = _device.describe(ks, L.tile_shape, Rr.tile_shape)
    run = sd._segment_run(rhs, jk, ak)
    desc.seg_group = run
    fused = lambda: _device.segment_einsum(desc, lhs.values, rhs.values, li, ri, perm, offs)
    t_fused = fused_in_step_ms(execute_sparse, lhs, rhs, jk, ks, ak, reps)
    if t_fused is None:
        t_fused = event_time_ms(fused, reps)
    t_fused_single = None
    if run:
        desc.seg_group = 0
        t_fused_single = event_time_ms(fused, reps)
    F = W.flops_gemm(ks, L.tile_shape, Rr.tile_shape, P)
    e = 2 if bf16 else 4
    out_tile = sd._infer_output_tile_shape(ks, L.tile_shape, Rr.tile_shape)
    B_fused = W.bytes_fused(int(torch.unique(li).numel()), int(torch.unique(ri).numel()),
                            L.tile_shape, Rr.tile_shape, e, U, out_tile, len(ak), e)
    peak = MFMA_PEAK_TFLOPS["bf16" if bf16 else "fp32"]
    res = {
        "workload": w["name"], "dtype": w["dtype"], "pairs": P, "output_tiles": U,
        "lhs_tiles": int(L.coords.shape[0]), "rhs_tiles": int(Rr.coords.shape[0]),
        "gflop": F / 1e9, "ms_per_step": ms_step, "tflops_step": F / ms_step / 1e9,
        "segment_run": run, "fused_ms": t_fused, "fused_tflops": F / t_fused / 1e9,
        "fused_mfma_frac": F / t_fused / 1e9 / peak, "fused_compulsory_bytes": B_fused,
        "fused_compulsory_gbs": B_fused / t_fused / 1e6,
        "fused_compulsory_hbm_frac": B_fused / t_fused / 1e6 / HBM_PEAK_GBS,
    }
    if t_fused_single is not None:
        res["fused_ms_one_segment_per_workgroup"] = t_fused_single
    del lhs, rhs, li, ri, coords, offs, perm
    torch.cuda.empty_cache()
    return res


def measure_ingest(cpu: bool = True) -> dict:
    """Relation construction at full size: the per-tile-shape statistics of
    every tile shape, nonzero counting, dense -> COO and COO -> tiles, for the
    16384^2 bf16 block-sparse operand (225 tile shapes) and the statistics of
    the 2048^3 fp32 order-3 operand (1728 tile shapes).  Each operand is
    dense in HBM before timing; times are wall clock around each call,
    including its host synchronisation.  The algorithmic bytes of the
    statistics are one read of the dense operand; of dense -> COO that read
    plus the COO written; of COO -> tiles the COO read plus the tiles
    written."""
    import torch

    from einjax_amd import SparseTensorRelation, _device
    from oracle import generators as G
    from oracle import reference_path as R

    out = {}
    for name, gen, dt in (("blocksparse_16k_bf16_A", G.workload_blocksparse_16k, torch.bfloat16),
                          ("order3_X", G.workload_order3, torch.float32)):
        w = gen(values=False)
        L = w["lhs"]
        tile = L.tile_shape
        nd = len(L.shape)
        vals = (torch.rand((len(L.coords), *tile), device="cuda") + 0.5).to(dt)
        rel = SparseTensorRelation(torch.from_numpy(L.coords).cuda(), vals, L.shape, tile)
        dense = rel.to_dense()
        del rel
        shapes = R.all_tile_shapes(L.shape)
        e = dense.element_size()
        n_el = dense.numel()
        t_stats = wall_time_ms(lambda: _device.scheme_stats(shapes, L.shape, dense=dense), 3)
        B_stats = n_el * e
        r = {"shape": list(L.shape), "dtype": str(dt).split(".")[-1], "tile_shapes": len(shapes),
             "stats_ms": t_stats, "stats_gbs": B_stats / (t_stats * 1e-3) / 1e9,
             "stats_hbm_frac": B_stats / (t_stats * 1e-3) / 1e9 / HBM_PEAK_GBS}
        t_cnt = wall_time_ms(lambda: _device.count_nonzero(dense), 3)
        r["count_nonzero_ms"] = t_cnt
        r["count_nonzero_gbs"] = B_stats / (t_cnt * 1e-3) / 1e9
        if name.startswith("blocksparse"):
            nnz = len(L.coords) * int(np.prod(tile))
            t_ext = wall_time_ms(lambda: _device.extract_coo(dense), 3)
            B_ext = n_el * e + nnz * (4 * nd + 8)
            idx, v64 = _device.extract_coo(dense)
            t_bc = wall_time_ms(lambda: _device.bucket_coo(idx, v64, L.shape, tile), 3)
            B_bc = nnz * (4 * nd + 8) + len(L.coords) * int(np.prod(tile)) * 4
            t_bd = wall_time_ms(lambda: _device.bucket_dense(dense, tile), 3)
            r.update({"nnz": nnz, "extract_coo_ms": t_ext,
                      "extract_coo_gbs": B_ext / (t_ext * 1e-3) / 1e9,
                      "bucket_coo_ms": t_bc, "bucket_coo_gbs": B_bc / (t_bc * 1e-3) / 1e9,
                      "bucket_dense_ms": t_bd})
            if cpu:
                # The oracle's statistics on the host COO: two tile shapes timed,
                # scaled to all 225 (each tile shape costs one np.unique over
                # every nonzero row).
                hidx = idx.cpu().numpy()
                hv = v64.cpu().numpy()
                sample = [(128, 128), (64, 256)]
                t0 = time.perf_counter()
                R.sparsity_metrics(hidx, hv, sample)
                t_cpu = time.perf_counter() - t0
                r["cpu_baseline"] = {
                    "value": t_cpu / len(sample) * len(shapes) * 1e3, "unit": "ms",
                    "cores": 1, "kind": "port",
                    "sample": f"oracle sparsity_metrics for {sample} on the {nnz} nonzeros "
                              f"({t_cpu:.1f} s), scaled to {len(shapes)} tile shapes"}
            del idx, v64
        out[name] = r
        del dense
        torch.cuda.empty_cache()
    return out


def measure_backward(lhs, rhs, li, ri, kernel_string, F: float, reps: int = 20) -> dict:
    """Backward of the headline's per-pair einsum (sparse_einsum_raw's
    gradient): both operand gradients for a cotangent of every pair in the
    forward output's dtype (bf16: bf16 gradient einsums, fp32 sums), each
    gradient alone, and both for an fp32 cotangent (operands widened to
    fp32).  FLOPs: 2·M·N·K per pair per gradient."""
    import torch

    from einjax_amd import _device

    g32 = torch.randn((li.numel(), lhs.tile_shape[0], rhs.tile_shape[1]), device="cuda")
    g = g32.to(lhs.values.dtype)
    vjp = lambda gg, **k: _device.pair_einsum_vjp(kernel_string, lhs.values, rhs.values, li, ri,
                                                  gg, **k)
    run = {
        "both": lambda: vjp(g),
        "lhs": lambda: vjp(g, need_rhs=False),
        "rhs": lambda: vjp(g, need_lhs=False),
        "both_fp32_cotangent": lambda: vjp(g32),
    }
    out = {}
    for k, fn in run.items():
        warm_up(fn)
        t = wall_time_ms(fn, reps, warm=0)
        flops = 2 * F if k.startswith("both") else F
        out[f"{k}_ms"] = t
        out[f"{k}_tflops"] = flops / (t * 1e-3) / 1e12
    del g, g32
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--all-configs", action="store_true",
                    help="also time every workload configuration at full size (adds 'configs')")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 1 GiB device buffer 4 times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes) and exit")
    ap.add_argument("--backward", action="store_true",
                    help="also time the backward of the headline einsum (adds 'backward')")
    ap.add_argument("--ingest", action="store_true",
                    help="also time relation construction at full size (adds 'ingest')")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path runs "
              "one process per GPU and this build has no multi-GPU mode)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        a = torch.randn(2 ** 28, device="cuda")
        b = torch.empty_like(a)
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel() * a.element_size(), "copies": 4}))
        return

    sys.path.insert(0, str(ROOT))
    from einjax_amd import SparseTensorRelation, _device, execute_sparse
    from einjax_amd.execution import sparse_dispatch as sd
    from oracle import generators as G
    from oracle import workload as W

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    t0 = time.perf_counter()
    w = G.workload_blocksparse_16k()
    L, Rr = w["lhs"], w["rhs"]
    log(f"generated {w['name']} in {time.perf_counter() - t0:.1f} s")

    def dev(r):
        return SparseTensorRelation(torch.from_numpy(r.coords).cuda(),
                                    torch.from_numpy(r.values).cuda().to(torch.bfloat16), r.shape,
                                    r.tile_shape)

    lhs, rhs = dev(L), dev(Rr)
    torch.cuda.synchronize()
    jk, ak, ks = w["join_keys"], w["agg_keys"], w["kernel_string"]

    def step():
        return execute_sparse(lhs, rhs, jk, ks, ak)

    # The CPU baseline and the stage timings run before the timed steps, so
    # that the GPU is at its working clocks when the warm-up steps start.
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on a sample ...")
        cpu = cpu_baseline(w, band_tiles=16)

    # ---- stages ----------------------------------------------------------
    # The collector runs now and is then off until the timed steps end: a
    # collection inside a timed region adds its ~60 ms to that region, and
    # one between the warm-up and the timed steps idles the GPU long enough
    # (tens of ms) for its clocks to drop, so that the timed steps start cold.
    gc.collect()
    gc.disable()
    lc, rc = lhs.coords, rhs.coords
    li, ri = sd._join_dev(lhs, rhs, jk, lc, rc)
    P = li.numel()
    radices = [sd._grid(lhs if s == 0 else rhs, d) for s, d in ak]
    coords, offs, perm, _ = _device.segment_plan(lc, rc, li, ri, ak, radices)
    U = coords.shape[0]
    desc = _device.describe(ks, L.tile_shape, Rr.tile_shape)
    desc.seg_group = sd._segment_run(rhs, jk, ak)  # as execute_sparse sets it
    reps = 10
    t_join = wall_time_ms(lambda: sd._join_dev(lhs, rhs, jk, lc, rc), reps)
    t_plan = wall_time_ms(lambda: _device.segment_plan(lc, rc, li, ri, ak, radices), reps)
    # The fused einsum as the exact path launches it (its own segment plan,
    # no run order); the step's launch is timed below.
    t_fused_exact = event_time_ms(
        lambda: _device.segment_einsum(desc, lhs.values, rhs.values, li, ri, perm, offs), reps)
    ga = _device.gather_tiles(lhs.values, li)
    gb = _device.gather_tiles(rhs.values, ri)
    t_gather = event_time_ms(lambda: (_device.gather_tiles(lhs.values, li),
                                      _device.gather_tiles(rhs.values, ri)), reps)
    t_pair = event_time_ms(lambda: _device.pair_einsum(desc, ga, gb, n_pairs=P), reps)
    pv = _device.pair_einsum(desc, ga, gb, n_pairs=P)
    t_segsum16 = event_time_ms(lambda: _device.segment_sum(pv, perm, offs), reps)
    del pv
    pv = _device.pair_einsum(desc, ga, gb, n_pairs=P, out_dtype=torch.float32)
    t_segsum = event_time_ms(lambda: _device.segment_sum(pv, perm, offs), reps)
    del ga, gb, pv
    dense_a = lhs.to_dense()
    t_bucket = wall_time_ms(lambda: _device.bucket_dense(dense_a, L.tile_shape), 5)
    del dense_a
    # The step with fp32 output tiles (out_dtype=float32): twice the bytes written.
    step32 = lambda: execute_sparse(lhs, rhs, jk, ks, ak, out_dtype=torch.float32)
    t_step32 = wall_time_ms(step32, 20)
    t_fused32 = fused_in_step_ms(
        lambda *a, **k: execute_sparse(*a, out_dtype=torch.float32, **k), lhs, rhs, jk, ks, ak,
        20)
    torch.cuda.synchronize()
    # The fused einsum as the step launches it (after the device-side join
    # and plan, in the plan's run order): HIP events on the launch stream,
    # 200 queued steps, right before the warm-up steps: its ~40 ms of
    # sustained load also brings the GPU toward its working clocks, which a
    # handful of warm-up steps alone (~1 ms) do not.  It is measured again
    # after the timed steps, at the clocks they ran at; that figure is the
    # roofline's (both are on the line).
    t_fused_ramp = fused_in_step_ms(execute_sparse, lhs, rhs, jk, ks, ak, 200) or t_fused_exact

    # ---- the timed steps -------------------------------------------------
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    t_fused = fused_in_step_ms(execute_sparse, lhs, rhs, jk, ks, ak, 200) or t_fused_exact
    gc.enable()

    e = 2
    F = W.flops_gemm(ks, L.tile_shape, Rr.tile_shape, P)
    out_tile = (L.tile_shape[0], Rr.tile_shape[1])
    B_join = W.bytes_join(L.coords.shape[0], Rr.coords.shape[0], P)
    B_gather = W.bytes_gather(P, L.tile_shape, Rr.tile_shape, e)
    B_segsum = W.bytes_segsum(P, U, out_tile, 2, 4)  # fp32 pair values and sums
    B_segsum16 = W.bytes_segsum(P, U, out_tile, 2, e)  # bf16 pair values and sums
    B_bucket = W.bytes_bucket(int(np.prod(L.shape)), L.coords.shape[0], L.tile_shape, e, 2)
    n_lhs_used = len(np.unique(li.cpu().numpy()))
    n_rhs_used = len(np.unique(ri.cpu().numpy()))
    B_fused = W.bytes_fused(n_lhs_used, n_rhs_used, L.tile_shape, Rr.tile_shape, e, U,
                            out_tile, 2, e)
    jgs_gbs = (B_join + B_gather + B_segsum) / ((t_join + t_gather + t_segsum) * 1e-3) / 1e9
    jgs16_gbs = (B_join + B_gather + B_segsum16) / ((t_join + t_gather + t_segsum16) * 1e-3) / 1e9
    fused_tflops = F / (t_fused * 1e-3) / 1e12
    kernel_name = "seg_gemm_kernel<SegOpBf16<128,128>,3,2,2,4,false>"
    traffic = load_traffic(kernel_name)

    res = {
        "metric": METRIC,
        "value": F / (ms_step * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded numpy default_rng(0); relations resident in HBM)",
        "config": {
            "workload": "block-sparse x dense 'ij,jk->ik': A 16384x16384 bf16, 128x128 tiles, "
                        "5% tile density uniform; B dense 16384x4096 bf16 N(0,1/128); fp32 "
                        "accumulate, bf16 output tiles",
            "pairs": P, "output_tiles": U, "lhs_tiles": int(L.coords.shape[0]),
            "rhs_tiles": int(Rr.coords.shape[0]), "gflop": F / 1e9,
        },
        "roofline": {
            "bound": "mfma", "kernel": kernel_name,
            "achieved": fused_tflops, "peak": MFMA_PEAK_TFLOPS["bf16"], "unit": "TFLOP/s",
            "frac": fused_tflops / MFMA_PEAK_TFLOPS["bf16"],
            "traffic": traffic,
            "algorithmic_bytes": B_fused,
        },
        "fp32_output": {
            "ms_per_step": t_step32, "tflops": F / (t_step32 * 1e-3) / 1e12,
            "fused_ms": t_fused32,
            "fused_mfma_frac": None if t_fused32 is None else
            F / (t_fused32 * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"],
        },
        "stages_ms": {
            "join": t_join, "segment_plan": t_plan, "fused_gemm_segsum": t_fused,
            "fused_gemm_segsum_before_warmup": t_fused_ramp,
            "fused_gemm_segsum_exact_path": t_fused_exact,
            "gather": t_gather, "pair_gemm": t_pair, "segment_sum": t_segsum,
            "segment_sum_bf16_values": t_segsum16, "bucket_dense_A": t_bucket,
        },
        "stages_gbs": {
            "join": B_join / (t_join * 1e-3) / 1e9,
            "gather": B_gather / (t_gather * 1e-3) / 1e9,
            "segment_sum": B_segsum / (t_segsum * 1e-3) / 1e9,
            "segment_sum_bf16_values": B_segsum16 / (t_segsum16 * 1e-3) / 1e9,
            "bucket_dense_A": B_bucket / (t_bucket * 1e-3) / 1e9,
            "join_gather_segsum": jgs_gbs,
            "join_gather_segsum_hbm_frac": jgs_gbs / HBM_PEAK_GBS,
            "join_gather_segsum_bf16_values_hbm_frac": jgs16_gbs / HBM_PEAK_GBS,
        },
        "unfused_tflops": F / ((t_join + t_plan + t_gather + t_pair + t_segsum) * 1e-3) / 1e12,
        "pair_gemm_tflops": F / (t_pair * 1e-3) / 1e12,
        "cpu_baseline": cpu,
    }
    if args.backward:
        log("backward ...")
        res["backward"] = measure_backward(lhs, rhs, li, ri, ks, F)
    if args.all_configs:
        del lhs, rhs, li, ri, coords, offs, perm, out
        torch.cuda.empty_cache()
        res["configs"] = {}
        for name in CONFIG_NAMES:
            log(f"config {name} ...")
            res["configs"][name] = measure_config(name)
    if args.ingest:
        torch.cuda.empty_cache()
        log("relation construction ...")
        res["ingest"] = measure_ingest(cpu=not args.no_cpu_baseline)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
