"""Benchmark of the north-star workload on one MI355X.

Workload (the metric's config): 3D type-1,
M = 2e7 fp64 coordinates uniform in [-pi, pi)^3, complex64 strengths with
re/im i.i.d. N(0,1) (numpy default_rng(0)), N = 256^3 modes, eps = 1e-5,
isign = +1, upsampfac 2 (w = 6, fine grid 512^3).

A step is one end-to-end pass with inputs already resident in HBM:
set_sources (fp64 fold/rescale, stable sort, z-sweep key starts) + execute
(spread, pruned 512^3 FFT with crop/deconvolution). W untimed warmup steps,
then K steps between torch.cuda.synchronize() calls; HIP events recorded on
the launch stream inside the timed region give per-step min/median/max and
per-stage times (read after the region, so nothing synchronises inside it).
The Python heap is collected and frozen (gc.collect + gc.freeze) before the
warm-up: a full collection of the interpreter's import-time objects costs
30-40 ms of host time, and one that lands inside the region leaves the GPU
idle for that long (one just before the region left the GPU at lower
clocks for its first steps). The warm-up records the same stage events as
the timed steps. Collector pauses inside the region are reported.

One JSON line is printed:
  value      = M / (ms_per_step) in NU pts/s (end to end, device-resident)
  roofline   = the spread kernel (the metric's "spread HBM GB/s"): algorithmic
               bytes M*(8 + 8*3 + 4) + 8*512^3 per launch over its mean
               HIP-event duration in the timed steps, against 8 TB/s; traffic
               from the committed rocprofv3 summary when it was measured on
               the current kernel source (None otherwise)
  cpu_baseline = the same type-1 on the host cores (fp32 OpenMP spread +
               scipy.fft, the oracle's port; finufft is not installed)
"""

import argparse
import gc
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "NU pts/s end-to-end + spread HBM GB/s, 3D type-1 M=2e7 N=256^3 eps=1e-5"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--M", type=float, default=2e7)
    ap.add_argument("--N", type=int, default=256)
    ap.add_argument("--eps", type=float, default=1e-5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--exec-only", action="store_true",
                    help="time execute() only (plan built once), for profiling")
    ap.add_argument("--workload", default="t1",
                    choices=["t1", "t3-generic", "t1-1d", "t1-2d-batch", "t2-2d-radial", "t3",
                             "expi"],
                    help="t1: the north-star line (default). t3-generic: the reference's "
                         "type-3 Table I case (generic geometry, 1e6 sources on a 640^3 "
                         "grid, M = N^2 targets), execute() only. t1-1d, t1-2d-batch, "
                         "t2-2d-radial, t3 and expi: BASELINE.json configs[0] (1D type-1), "
                         "configs[1] (2D type-1, execute_batch of 8 vectors), configs[2] "
                         "(2D type-2 on radial spokes), configs[4] (3D type-3) and its expi "
                         "leg (1e7 phases), the plan built once, for timing and profiling "
                         "those paths")
    ap.add_argument("--t3-N", type=int, default=1024, choices=[512, 1024, 2048],
                    help="t3-generic: targets M = N^2")
    ap.add_argument("--copy-calibration", type=float, default=0.0, metavar="GIB",
                    help="only copy a GIB-sized device buffer 5 times: the plain copy "
                         "kernel whose FETCH_SIZE / WRITE_SIZE scale the traffic counters")
    return ap.parse_args()


def copy_calibration(gib):
    """5 device-to-device copies of gib GiB (torch's copy kernel): each reads
    and writes exactly that many bytes of HBM."""
    import torch

    nbytes = int(gib * (1 << 30))
    a = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": nbytes, "launches": 5}))


def cpu_baseline(x, c, N, eps):
    """The oracle's fp32 OpenMP type-1 port on the full workload, timed once
    after a small warm-up call (about 3-10 s of host work)."""
    import numpy as np

    from oracle import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    small = [v[:200_000] for v in x]
    O.cpu_type1_f32(small, c[:200_000], (64, 64, 64), eps, workers=threads)
    t0 = time.perf_counter()
    _, parts = O.cpu_type1_f32(x, c, N, eps, workers=threads)
    dt = time.perf_counter() - t0
    M = x[0].size
    return {"value": M / dt, "unit": "NU pts/s", "cores": threads, "kind": "port",
            "sample": (f"full workload once (M={M:.0e}, N={N[0]}^3, eps={eps:g}, fp32 OpenMP "
                       f"spread + scipy.fft workers={threads}); {dt:.2f} s"),
            "seconds": {k: round(v, 4) for k, v in parts.items()}}


def spread_traffic(kernel):
    """HBM bytes per spread launch (FETCH_SIZE + WRITE_SIZE, calibrated) from
    the committed rocprofv3 summary, with its provenance. The summary records
    the kernel it measured and the SHA-256 of the kernel's sources at the
    time (mn_zsweep.hip followed by the mn_zsweep.h it includes); when either
    differs from what runs now, the figure is stale and traffic is reported
    as None."""
    import hashlib

    tf = ROOT / "profiles" / "spread_zsweep_3d_t1_M2e7_N256_traffic.json"
    csrc = ROOT / "mlx_nufft_amd" / "csrc"
    try:
        d = json.loads(tf.read_text())
        sha = hashlib.sha256(b"".join((csrc / f).read_bytes()
                                      for f in ("mn_zsweep.hip", "mn_zsweep.h"))).hexdigest()
    except (ValueError, OSError):
        return None, {"file": str(tf.relative_to(ROOT)), "status": "missing"}
    info = {"file": str(tf.relative_to(ROOT)), "kernel": d.get("kernel"),
            "source_sha256": d.get("source_sha256"), "commit": d.get("commit")}
    if d.get("kernel") != kernel or d.get("source_sha256") != sha:
        info["status"] = "stale (kernel or source changed since the measurement)"
        return None, info
    info["status"] = "current"
    return d.get("bytes_per_launch"), info


# The reference's published type-3 execute times for this workload (M5 Max,
# mlx-nufft.pdf p.8 Table I), by N: other hardware, context only.
T3_REF_M5MAX_S = {512: 0.097, 1024: 0.118, 2048: 0.205}


def bench_t3(args):
    """Type-3, the reference's generic acceptance geometry
    (ref: harness/gen.py:54-67, gen_generic; harness/run_acceptance.py:37-41,
    106-125): P = 1e6 sources uniform in [-30, 30]^3, M = N^2 targets
    uniform in [-20, 20]^3, strengths a e^{i th}, eps = 3e-5, isign = +1,
    crit64; the fine grid is 486^3 (spread) and 640^3 (FFT). A step is one
    execute() with the plan built and the strengths resident in HBM."""
    import numpy as np
    import torch

    import mlx_nufft_amd as mn
    from mlx_nufft_amd import _lib

    _lib.require_gpu()
    N, P = args.t3_N, 1_000_000
    rng = np.random.default_rng(0)
    x = tuple(rng.uniform(-30.0, 30.0, P) for _ in range(3))
    s = tuple(rng.uniform(-20.0, 20.0, N * N) for _ in range(3))
    c = (rng.uniform(0.2, 1.0, P) * np.exp(1j * rng.uniform(0, 2 * np.pi, P))).astype(np.complex64)
    cd = torch.from_numpy(c).cuda()
    plan = mn.Type3Plan(x, s, eps=3e-5, isign=+1, prec="crit64")
    gc.collect()  # before the warm-up, not between it and the timed steps
    for _ in range(args.warmup):
        plan.execute(cd, return_np=False)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        plan.execute(cd, return_np=False)
        b.record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step_ms = sorted(a.elapsed_time(b) for a, b in ev)
    _, st = plan.execute_profiled(cd)
    ref_s = T3_REF_M5MAX_S[N]
    out = {
        "metric": "type-3 execute time, generic geometry, 1e6 sources, M = N^2 targets",
        "value": ms * 1e-3,
        "unit": "s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic: numpy default_rng(0), the reference's generic type-3 geometry",
        "config": {"workload": f"3D type-3 generic P=1e6 M={N * N} eps=3e-5 (Table I)",
                   "P": P, "M": N * N, "eps": 3e-5, "w": plan.w, "nf": list(plan.nf),
                   "n_up": list(plan.n_up),
                   "spread": "owner-computes fp64" if plan.spread_owner else "LDS tiles fp64",
                   "fft": "fp64 line passes" if plan.fft_lines else "pad + rocFFT fp64"},
        "step_ms": {"min": step_ms[0], "median": step_ms[len(step_ms) // 2], "max": step_ms[-1]},
        "stages_ms": {k: round(v * 1e3, 4) for k, v in st.items()},
        "reference_m5max_s": ref_s,
        "speedup_vs_reference_m5max": ref_s / (ms * 1e-3),
    }
    print(json.dumps(out))


def bench_other(args):
    """One call of the path, the plan built once and its inputs resident in
    HBM, for BASELINE.json's other configurations (their shapes,
    distributions and default_rng(0) data):
      t1-1d         configs[0]: 1D type-1, M = 1e5, N = 4096, eps 1e-6, execute();
      t1-2d-batch   configs[1]: 2D type-1, M = 1e7 shared by 8 vectors,
                    N = 1024^2, eps 1e-6, execute_batch();
      t2-2d-radial  configs[2]: 2D type-2 on 512 spokes x 2048 samples
                    (angles uniform in [0, pi), radii evenly spaced in
                    [-pi, pi)), N = 1024^2, eps 1e-6, isign -1, execute();
      t3            configs[4]: 3D type-3, 1e6 sources in [-1, 1]^3, 1e6
                    targets in [-200, 200]^3, eps 1e-5, execute();
      expi          configs[4]'s expi leg: 1e7 fp64 phases in [-1e6, 1e6].
    One JSON line: the time per call (host clock over the timed calls) and,
    where the plan times its stages with HIP events, one profiled call's
    stages."""
    import numpy as np
    import torch

    import mlx_nufft_amd as mn
    from mlx_nufft_amd import _lib

    _lib.require_gpu()
    rng = np.random.default_rng(0)

    def cplx(shape):
        return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)

    wl = args.workload
    plan = None
    if wl == "t1-1d":
        M = 100_000
        x = (rng.uniform(-np.pi, np.pi, M),)
        plan = mn.Type1PlanND(x, (4096,), eps=1e-6, isign=+1)
        cd = torch.from_numpy(cplx(M)).cuda()
        cfg = {"workload": "1D type-1 M=1e5 N=4096 eps=1e-6 (BASELINE.json configs[0])"}
        run = lambda: plan.execute(cd, return_np=False)  # noqa: E731
    elif wl == "t1-2d-batch":
        M, B = 10_000_000, 8
        x = tuple(rng.uniform(-np.pi, np.pi, M) for _ in range(2))
        cd = torch.from_numpy(cplx((B, M))).cuda()
        plan = mn.Type1PlanND(x, (1024, 1024), eps=1e-6, isign=+1)
        cfg = {"workload": "2D type-1 M=1e7 x 8 vectors N=1024^2 eps=1e-6 "
                           "(BASELINE.json configs[1]), execute_batch", "spread": plan.pts.kind}
        run = lambda: plan.execute_batch(cd, return_np=False)  # noqa: E731
    elif wl == "t2-2d-radial":
        f = cplx((1024, 1024))
        theta = rng.uniform(0.0, np.pi, 512)
        r = np.linspace(-np.pi, np.pi, 2048, endpoint=False)
        x = (np.outer(np.cos(theta), r).ravel(), np.outer(np.sin(theta), r).ravel())
        plan = mn.Type2PlanND(x, (1024, 1024), eps=1e-6, isign=-1)
        fd = torch.from_numpy(f).cuda()
        cfg = {"workload": "2D type-2 radial 512 spokes x 2048 samples N=1024^2 eps=1e-6 "
                           "(BASELINE.json configs[2])"}
        run = lambda: plan.execute(fd, return_np=False)  # noqa: E731
    elif wl == "t3":
        M = 1_000_000
        x = tuple(rng.uniform(-1.0, 1.0, M) for _ in range(3))
        s = tuple(rng.uniform(-200.0, 200.0, M) for _ in range(3))
        plan = mn.Type3Plan(x, s, eps=1e-5, isign=+1)
        cd = torch.from_numpy(cplx(M)).cuda()
        cfg = {"workload": "3D type-3 1e6 x 1e6 eps=1e-5 (BASELINE.json configs[4])"}
        run = lambda: plan.execute(cd, return_np=False)  # noqa: E731
    else:
        phi = torch.from_numpy(rng.uniform(-1e6, 1e6, 10_000_000)).cuda()
        cfg = {"workload": "expi on 1e7 fp64 phases in [-1e6, 1e6] (BASELINE.json configs[4])"}
        run = lambda: mn.expi(phi)  # noqa: E731
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    out = {"metric": "execute time", "value": ms, "unit": "ms", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
           "higher_is_better": False, "config": cfg}
    if wl == "t3":
        _, st = plan.execute_profiled(cd)
        out["stages_ms"] = {k: round(v * 1e3, 4) for k, v in st.items()}
    elif plan is not None:
        plan.profile = True
        run()
        out["stages_ms"] = {k: round(v, 4) for k, v in plan.last_profile.items()}
        plan.profile = False
    print(json.dumps(out))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); "
              "the path would shard the fine grid into x-slabs, one per GPU, but no "
              "multi-GPU path is built", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration > 0:
        copy_calibration(args.copy_calibration)
        return
    if args.workload == "t3-generic":
        bench_t3(args)
        return
    if args.workload != "t1":
        bench_other(args)
        return
    import numpy as np
    import torch

    import mlx_nufft_amd as mn
    from mlx_nufft_amd import _lib

    _lib.require_gpu()
    M, N, eps = int(args.M), (args.N,) * 3, args.eps
    rng = np.random.default_rng(0)
    x = [rng.uniform(-np.pi, np.pi, M) for _ in range(3)]
    c = (rng.standard_normal(M) + 1j * rng.standard_normal(M)).astype(np.complex64)
    dev = torch.device("cuda")
    xd = [torch.from_numpy(v).to(dev) for v in x]
    cd = torch.from_numpy(c).to(dev)

    plan = mn.Type1PlanND(tuple(xd), N, eps=eps, isign=+1)
    n_up = plan.n_up
    grid_cells = int(np.prod(n_up))

    def step():
        if not args.exec_only:
            plan.set_sources(tuple(xd))
        plan.execute(cd, return_np=False)

    # A full collection of the interpreter's import-time objects takes 30-40 ms
    # of host time; landing in the timed region it starves the GPU for that
    # long. Collect and freeze them first (GC stays on; pauses are reported),
    # before the warm-up: a GPU left idle for that long ran the next 8 or so
    # steps at lower clocks (3.3 down to 2.83 ms).
    gc.collect()
    gc.freeze()
    # The warm-up steps run as the timed ones do, stage events included;
    # their times are dropped.
    plan.profile = plan.profile_deferred = True
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    plan.drain_profiles()
    # Timed region: K steps between two synchronisations. HIP events on the
    # launch stream bracket every step and every stage (the spread kernel is
    # one launch per step); they are read only after the region ends.
    step_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
    host_ms, gc_ms, gc_t = [], [], [0.0]

    def gc_cb(phase, info):
        if phase == "start":
            gc_t[0] = time.perf_counter()
        else:
            gc_ms.append((time.perf_counter() - gc_t[0]) * 1e3)

    gc.callbacks.append(gc_cb)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in step_ev:
        a.record()
        h = time.perf_counter()
        step()
        host_ms.append((time.perf_counter() - h) * 1e3)
        b.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    gc.callbacks.remove(gc_cb)
    plan.profile = plan.profile_deferred = False
    ms = (t1 - t0) * 1e3 / args.steps
    step_raw = [a.elapsed_time(b) for a, b in step_ev]
    step_ms = sorted(step_raw)
    stage_sum = {}
    for _, prof in plan.drain_profiles():
        for k, v in prof.items():
            stage_sum[k] = stage_sum.get(k, 0.0) + v
    stages = {k: v / args.steps for k, v in stage_sum.items()}

    spread_ms = stages.get("spread", float("nan"))
    alg_bytes = M * (8 + 8 * 3 + 4) + 8 * grid_cells
    achieved = alg_bytes / (spread_ms * 1e-3) / 1e9
    exec_ms = sum(stages.get(k, 0.0) for k in ("zero", "spread", "fft", "deconv"))

    # type-2 leg of the round trip: interp back at the
    # same points from the type-1 output, timed the same way (not in `value`).
    fk = plan.execute(cd, return_np=False)
    plan_w, plan_bins = plan.w, [plan.bins.m[d] for d in range(3)]
    zsweep = plan.pts.kind == "zsweep"
    spread_kernel = (f"k_spread_zsweep<{plan_w}, false, 1>" if zsweep
                     else f"k_spread_tiled<3,{plan_w},false>")
    traffic, traffic_src = spread_traffic(spread_kernel)
    del plan
    p2 = mn.Type2PlanND(tuple(xd), N, eps=eps, isign=-1)
    for _ in range(max(1, args.warmup)):
        p2.execute(fk, return_np=False)
    p2.profile = True
    t2_stages = {}
    reps = max(3, args.steps // 4)
    for _ in range(reps):
        p2.execute(fk, return_np=False)
        for k, v in p2.last_profile.items():
            t2_stages[k] = t2_stages.get(k, 0.0) + v / reps
    interp_ms = t2_stages.get("interp", float("nan"))
    interp_gbs = alg_bytes / (interp_ms * 1e-3) / 1e9
    del p2
    out = {
        "metric": METRIC,
        "value": M / (ms * 1e-3),
        "unit": "NU pts/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: numpy default_rng(0) uniform coords, N(0,1) complex64 strengths",
        "config": {"workload": "3D type-1 M=2e7 N=256^3 eps=1e-5 (BASELINE.json configs[3])",
                   "M": M, "N": list(N), "eps": eps, "isign": 1, "w": plan_w,
                   "n_up": list(n_up),
                   "spread": ("z-sweep, 8x8 column blocks, 8-cell z-chunks, MFMA windows"
                              if zsweep else f"LDS tiles {plan_bins}"),
                   "step": ("execute only" if args.exec_only else
                            "set_sources + execute, device-resident")},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": spread_kernel, "alg_bytes_per_launch": alg_bytes,
                     "ms_per_launch": spread_ms},
        "step_ms": {"min": step_ms[0], "median": step_ms[len(step_ms) // 2],
                    "max": step_ms[-1], "argmax": step_raw.index(step_ms[-1])},
        "host_ms_per_step": {"median": sorted(host_ms)[len(host_ms) // 2], "max": max(host_ms),
                             "argmax": host_ms.index(max(host_ms))},
        "gc_pauses_ms": [round(v, 2) for v in gc_ms],
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "exec_ms": exec_ms,
        "exec_pts_per_s": M / (exec_ms * 1e-3) if exec_ms else None,
        "type2_roundtrip": {"stages_ms": {k: round(v, 4) for k, v in t2_stages.items()},
                            "interp_GBs": interp_gbs, "interp_frac": interp_gbs / HBM_PEAK_GBS},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x, c, N, eps)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
