#!/usr/bin/env python
"""Throughput of the Voronoi-foam tracer, forward + backward, on one MI355X.

Workload (default): config C3 -- 1M points (superquadric surface + uniform
box), SH degree 3, sdfoam alpha, inv_s = exp(0.3), 1600x1200 pinhole rays,
one depth quantile, upstream gradients N(0,1); all synthetic and seeded.
Inputs are resident in HBM before the timed region.

A step is one training pass of the path through the drop-in API:
``Pipeline.trace_forward`` (with contribution and depth) then
``Pipeline.trace_backward`` -- each runs the fp16 offset prepass and its
kernel, as the reference does.

Output: one JSON line on stdout.  ``roofline`` is the dominant kernel's HBM
rate: the HBM bytes per launch that rocprofv3 counted for it (L2-to-memory
read and write requests weighted by their sizes; profiles/traffic_*.json)
over its average duration, measured live by HIP events recorded on its launch
stream, against MI355X's 8 TB/s.  Beside it, ``model_frac`` prices the
kernel's algorithmic bytes (the gather model below, which counts every gather
as an HBM access although L2 and the MALL serve most of them) the same way.
``cpu_baseline`` is the scalar host oracle (a port of the reference's
algorithm) on a strided sample of the same rays, on every CPU the process may
use, plus a one-thread run.

Gather model (per launch; D = attribute width, deg = CSR row length of the
stepped cell, Q = quantiles):
  forward : per ray 48 + 12Q; per step 28 + 4D + 4 (contribution) + 8 deg
  backward: per ray 60 + 12Q; per step 36 + 8D + 8 deg
  prepass : 12 E + 16 N
With the walk record (default, as TraceRays runs it) the forward also writes
24 B per step and the backward reads them instead of the face rows and the
attribute row.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Mrays/s fwd+bwd at 1M pts/1600x1200 rays; % HBM roofline"
RENDER_METRIC = "Mpixels/s inference render (trace_benchmark, RGBA8)"
FETCH_METRIC = "GB/s of training batches delivered by BatchFetcher (rays + rgb)"
TRI_METRIC = "Triangulation rebuilds/s (Delaunay + tables) on a config's point set"
HOST_LINK_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_affinity() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_quota():
    """CPUs this process's cgroup may use (cgroup v2 cpu.max or v1 CFS
    quota), or None when unlimited."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                return max(1, int(int(q) / int(period)))
            return None
    except (OSError, ValueError):
        pass
    try:
        with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f:
            q = int(f.read())
        with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
            period = int(f.read())
        return max(1, q // period) if q > 0 else None
    except (OSError, ValueError):
        return None


def cpu_threads() -> int:
    """Every CPU the process may run on: its affinity set, bounded by its
    cgroup's CPU quota."""
    n = cpu_affinity()
    q = cpu_quota()
    return max(1, min(n, q) if q else n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5],
                    help="workload C1-C5; C3 is the headline (C5: each step draws its own "
                         "2^20 rays and looks up their start cells)")
    ap.add_argument("--cpu-stride", type=int, default=-1,
                    help="CPU baseline traces every n-th ray (0 skips it; default: the "
                         "smallest n that keeps the sample to at most 1.92M rays: every ray "
                         "of C3, about 30 s on 16 threads)")
    ap.add_argument("--alpha-mode", default="sdfoam", choices=["sdfoam", "standard"],
                    help="sdfoam (NeuS alpha, backward_sdf; the headline) or standard "
                         "(density alpha, the density backward; the scene's last channel is a "
                         "density)")
    ap.add_argument("--attr-dtype", default="float32", choices=["float32", "float16"],
                    help="attribute storage of the pipeline (fp16: create_pipeline(L, "
                         "'float16'); arithmetic stays fp32)")
    ap.add_argument("--fetch", action="store_true",
                    help="time BatchFetcher feeding training batches (2^20 shuffled rows of "
                         "rays [M, 6] and colours [M, 3], M = 64 cameras x 960 x 640)")
    ap.add_argument("--triangulate", action="store_true",
                    help="time Triangulation.rebuild (sort, GPU Delaunay with Qhull on the "
                         "open points, tables) on C3's 1M points, with Qhull on every point "
                         "beside it")
    ap.add_argument("--perturb", type=float, default=0.001,
                    help="--triangulate: the incremental rebuilds move each point by this "
                         "share of its cell radius (farthest Delaunay neighbour) times N(0, 1) "
                         "per coordinate (past ~0.005 most points are dirty and the rebuild "
                         "is a full one)")
    ap.add_argument("--render", action="store_true",
                    help="time the inference render (Pipeline.trace_benchmark, the reference's "
                         "benchmark.py) on the config's camera instead of the training step")
    ap.add_argument("--walk-record", type=int, default=1, choices=[0, 1],
                    help="1: the forward records each ray's steps and the backward replays "
                         "them (TraceRays does this); 0: the backward scans the faces again")
    ap.add_argument("--cell-table", type=int, default=1, choices=[0, 1],
                    help="1: the forward walks over its cell table (the default of "
                         "trace_forward); 0: over the caller's arrays")
    ap.add_argument("--scene-cache", default="",
                    help="npz file to load the generated scene from / save it to")
    ap.add_argument("--calibrate-copy-gib", type=float, default=0.0,
                    help="only run a device-to-device copy of this many GiB (a kernel of known "
                         "traffic, to scale rocprof FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--calibrate-gather-gib", type=float, default=0.0,
                    help="only run a gather of this many GiB of 128-byte rows in a random "
                         "order, each row read once (a gather of known traffic, to scale rocprof "
                         "FETCH_SIZE for the tracer's gathers) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(rays would shard across GPUs with one gradient all-reduce; not built)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import sdfoam_amd
    from sdfoam_amd import _lib, scenes

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    _lib.lib()

    if args.calibrate_copy_gib > 0:
        n = int(args.calibrate_copy_gib * (1 << 30)) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": 4 * n, "launches": 3}), flush=True)
        return 0

    if args.calibrate_gather_gib > 0:
        rows = int(args.calibrate_gather_gib * (1 << 30)) // 128
        src = torch.ones((rows, 32), dtype=torch.float32, device=dev)
        perm = torch.randperm(rows, device=dev, generator=torch.Generator(device=dev).manual_seed(1))
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.index_select(src, 0, perm, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_gather_rows": rows, "row_bytes": 128,
                          "index_bytes": 8 * rows, "launches": 3}), flush=True)
        return 0

    if args.fetch:
        return fetch_bench(args, dev)
    if args.triangulate:
        return triangulate_bench(args, dev)

    t0 = time.time()
    if args.scene_cache and os.path.exists(args.scene_cache):
        log(f"loading scene from {args.scene_cache}")
        w = scenes.load_workload(args.scene_cache)
    else:
        log(f"generating config C{args.config} (Delaunay on the GPU)")
        w = scenes.make_config(args.config, mode=args.alpha_mode,
                               tetrahedra=lambda p: gpu_simplices(p, dev))
        if args.scene_cache:
            scenes.save_workload(w, args.scene_cache)
    log(f"scene ready in {time.time() - t0:.1f}s: N={w.num_points} E={w.adjacency.size} R={w.num_rays}")

    def u32(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev).view(torch.uint32)

    def to_dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    if w.alpha_mode != args.alpha_mode:
        raise RuntimeError(f"scene cache holds a {w.alpha_mode} scene")
    half = args.attr_dtype == "float16"
    adt = torch.float16 if half else torch.float32
    pts = to_dev(w.points)
    attrs = to_dev(w.attributes).to(adt)
    adj, offs = u32(w.adjacency), u32(w.offsets)
    inv = torch.tensor([w.inv_s], dtype=torch.float32, device=dev)
    tree = sdfoam_amd.build_aabb_tree(pts)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, args.attr_dtype)
    D = pipe.attribute_dim()
    Q = int(w.quantiles.shape[-1])
    if args.render:
        return render_bench(args, w, pts, attrs, adj, offs, inv, pipe, D)

    # ray batches: one fixed batch (C1-C4), or C5's ten seeded batches
    batches = []
    if args.config == 5:
        cams = w.extra["cameras"]
        for s in range(10):
            if s == 0:
                r_np, q_np, g_np, dg_np = w.rays, w.quantiles, w.grad_rgba, w.depth_grad
            else:
                r_np, q_np = scenes.c5_step_rays(cams, s, w.num_rays)
                grng = np.random.default_rng(7000 + s)
                g_np = grng.normal(size=(w.num_rays, 4)).astype(np.float32)
                dg_np = grng.normal(size=(w.num_rays, Q)).astype(np.float32)
            batches.append(dict(rays=to_dev(r_np), q=to_dev(q_np), g=to_dev(g_np).to(adt),
                                dg=to_dev(dg_np), rays_np=r_np))
    else:
        batches.append(dict(rays=to_dev(w.rays), q=to_dev(w.quantiles),
                            g=to_dev(w.grad_rgba).to(adt), dg=to_dev(w.depth_grad),
                            rays_np=w.rays))
    lookup_in_step = args.config == 5
    for b in batches:
        b["start"] = sdfoam_amd.get_starting_point(b["rays"], pts, tree)
    torch.cuda.synchronize()
    host_start = scenes.start_points_for(w.points, batches[0]["rays_np"])
    if not np.array_equal(batches[0]["start"].view(torch.int32).cpu().numpy().view(np.uint32).reshape(-1),
                          host_start.reshape(-1)):
        raise RuntimeError("GPU start cells differ from the host nearest neighbour")

    use_record = bool(args.walk_record)

    def step(k):
        b = batches[k % len(batches)]
        start = (sdfoam_amd.get_starting_point(b["rays"], pts, tree) if lookup_in_step
                 else b["start"])
        out = pipe.trace_forward(pts, attrs, adj, offs, b["rays"], start, depth_quantiles=b["q"],
                                 return_contribution=True, alpha_mode=args.alpha_mode,
                                 inv_s=inv, record_walk=use_record,
                                 cell_table=bool(args.cell_table))
        bwd = pipe.trace_backward(pts, attrs, adj, offs, b["rays"], start, out["rgba"], b["g"],
                                  b["q"], out["depth_indices"], b["dg"],
                                  alpha_mode=args.alpha_mode, inv_s=inv,
                                  trace_plan=out.get("trace_plan"))
        return out, bwd

    log(f"warmup {args.warmup}")
    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()

    log(f"timing {args.steps} steps")
    _lib.set_timing(True)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    last = None
    for k in range(args.steps):
        last = step(args.warmup + k)
    torch.cuda.synchronize()
    t_end = time.perf_counter()
    launches = _lib.collect_timings()
    _lib.set_timing(False)
    ms_per_step = (t_end - t_start) * 1e3 / args.steps
    log(f"{ms_per_step:.3f} ms/step")
    # the last step's walk record: its pool (sized by the steps before it)
    # and the chunks its walk asked for
    record = None
    plan = last[0].get("trace_plan") if last is not None else None
    if plan is not None and plan.entries is not None:
        asked = plan.record_counters().cpu().numpy()
        record = {"bytes": int(plan.nbytes), "pool_chunks": int(plan.chunks),
                  "chunks_asked": int(asked.sum()), "chunks_asked_max_xcd": int(asked.max()),
                  "budget_trips": int(plan.budget),
                  "full_bytes": int(_lib.lib().sdf_walk_record_bytes(plan.num_rays,
                                                                     plan.ray_image_width,
                                                                     plan.budget))}

    per_kernel: dict[str, list[float]] = {}
    for name, ms in launches:
        per_kernel.setdefault(name, []).append(ms)
    avg = {k: float(np.mean(v)) for k, v in per_kernel.items()}

    # walk statistics for the byte model (untimed), averaged over the timed steps
    S = F_st = F_all = 0
    for k in range(args.steps):
        b = batches[(args.warmup + k) % len(batches)]
        if "stats" not in b:
            st = pipe.walk_stats(pts, attrs, adj, offs, b["rays"], b["start"],
                                 alpha_mode=args.alpha_mode, inv_s=inv)
            torch.cuda.synchronize()
            b["stats"] = (int(st["steps"].sum().item()), int(st["faces_stepped"].sum().item()),
                          int(st["faces"].sum().item()))
        S += b["stats"][0]
        F_st += b["stats"][1]
        F_all += b["stats"][2]
    S //= args.steps
    F_st //= args.steps
    F_all //= args.steps
    R = w.num_rays
    N = w.num_points
    E = int(w.adjacency.size)
    # attribute elements (rows, contribution, gradient rows) at their storage
    # width.  The gather model prices every access as an HBM access, whether
    # or not the walk record replaces it (the record's own 24 B per step,
    # written by the forward and read by the backward, are counted apart).
    ab = 2 if half else 4
    recorded = use_record
    gather_fwd = R * (48 + 12 * Q) + S * (28 + ab * D + ab) + 8 * F_st
    gather_bwd = R * (60 + 12 * Q) + S * (36 + 2 * ab * D) + 8 * F_st
    record_bytes = 24 * S if recorded else 0
    bytes_pre = 12 * E + 16 * N
    # offset-table builds per step (the backward reuses the forward's table
    # when it gets the forward's trace plan)
    pre_per_step = len(per_kernel.get("prefetch_adjacent_diff", [])) / args.steps
    # the forward's one-pass offset table + cell table: the table's bytes, each
    # cell's position, offsets and attribute row read and its record written
    bytes_prep = bytes_pre + N * (12 + 8 + ab * D) + int(
        _lib.lib().sdf_cell_table_bytes(w.sh_degree, 1 if half else 0, N))
    prep_per_step = len(per_kernel.get("scene_prep", [])) / args.steps
    bytes_step = gather_fwd + gather_bwd + pre_per_step * bytes_pre + prep_per_step * bytes_prep
    kernel_bytes = {"forward": gather_fwd, "backward": gather_bwd,
                    "prefetch_adjacent_diff": bytes_pre, "scene_prep": bytes_prep}
    dominant = max((k for k in avg if k in kernel_bytes), key=lambda k: avg[k] * len(per_kernel[k]))
    kernel_s = avg[dominant] * 1e-3
    model_gbps = kernel_bytes[dominant] / kernel_s / 1e9

    variant = ("" if use_record else "_scan") + ("" if args.alpha_mode == "sdfoam" else "_standard") \
        + ("_f16" if half else "")
    counters = load_counters(f"traffic_{dominant}{variant}_C{args.config}.json")
    traffic = counters.get("hbm_bytes_per_launch") if counters else None
    if traffic:
        # measured HBM bytes of this kernel (rocprofv3 FETCH_SIZE / WRITE_SIZE,
        # calibrated) over its live duration
        achieved, basis = traffic / kernel_s / 1e9, "rocprof HBM bytes per launch / live kernel time"
    else:
        why = STALE_COUNTERS.get(f"traffic_{dominant}{variant}_C{args.config}.json")
        achieved, basis = model_gbps, ("gather model (" + (
            f"rocprof counters stale: {why}" if why else "no rocprof counters for this workload")
            + ")")

    if args.config == 5:
        rays_desc = f"{R} rays per step sampled from 64 cameras 960x640 (10 seeded batches)"
    elif args.config == 4:
        rays_desc = f"8 cameras x {w.rays.shape[2]}x{w.rays.shape[1]} rays"
    else:
        rays_desc = f"{w.rays.shape[1]}x{w.rays.shape[0]} rays"
    result = {
        "metric": METRIC,
        "value": R / (ms_per_step * 1e-3) / 1e6,
        "unit": "Mrays/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"C{args.config}: {N} points, SH degree {w.sh_degree}, "
                        f"{args.alpha_mode} alpha, {args.attr_dtype} attributes, "
                        f"inv_s={w.inv_s:.4f}, {rays_desc}, Q={Q}, "
                        + ("start-cell lookup + " if lookup_in_step else "")
                        + "trace_forward(contribution, depth) + trace_backward"
                        + (" replaying the forward's walk record" if recorded else ""),
            "points": N,
            "adjacency": E,
            "rays": R,
            "sh_degree": w.sh_degree,
            "alpha_mode": args.alpha_mode,
            "attr_dtype": args.attr_dtype,
        },
        "rays_per_s": R / (ms_per_step * 1e-3),
        "cell_steps_per_s": S / (ms_per_step * 1e-3),
        "cell_steps_per_ray": S / R,
        "faces_per_step": F_st / max(S, 1),
        "faces_scanned": F_all,
        "kernel_ms": avg,
        "walk_record": record,
        "algorithmic_bytes": {"forward": gather_fwd, "backward": gather_bwd, "prefetch": bytes_pre,
                              "step": bytes_step, "walk_record_each_way": record_bytes},
        "step_algorithmic_GBps": bytes_step / (ms_per_step * 1e-3) / 1e9,
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "basis": basis,
            "kernel_ms": avg[dominant],
            "l2_hit": counters.get("l2_hit") if counters else None,
            "counters": counters.get("source") if counters else None,
            "algorithmic_bytes": kernel_bytes[dominant],
            "model_achieved": model_gbps,
            "model_frac": model_gbps / HBM_PEAK_GBS,
        },
    }

    if args.cpu_stride != 0:
        b0 = batches[0]
        n_rays = b0["rays_np"].size // 6
        stride = args.cpu_stride if args.cpu_stride > 0 else max(1, -(-n_rays // CPU_SAMPLE_RAYS))
        result["cpu_baseline"] = cpu_baseline(
            w, b0["rays_np"], host_start, b0["q"].cpu().numpy(),
            b0["g"].float().cpu().numpy(), b0["dg"].cpu().numpy(), stride, args.alpha_mode)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


CPU_SAMPLE_RAYS = 1_920_000


def file_sha256(path):
    import hashlib

    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


STALE_COUNTERS = {}  # profile name -> why its counters were not used


def load_counters(name):
    """A committed rocprofv3 counter summary of one kernel (profiles/<name>):
    HBM bytes per launch, L2 hit rate, source table; or None.  The summary
    lists the kernel sources it was measured on with their SHA-256; if any
    of them has changed since (or the list is missing) the summary is stale
    and None is returned (the reason goes to STALE_COUNTERS)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        c = json.load(f)
    srcs = c.get("sources")
    if not srcs:
        STALE_COUNTERS[name] = "no source hashes"
        return None
    for rel, sha in srcs.items():
        p = os.path.join(ROOT, rel)
        if not os.path.exists(p) or file_sha256(p) != sha:
            STALE_COUNTERS[name] = f"{rel} changed since the profile"
            return None
    return c


def load_traffic(name):
    """HBM bytes per launch that a committed rocprofv3 counter summary
    (profiles/<name>) records, or None (missing or stale)."""
    c = load_counters(name)
    return c.get("hbm_bytes_per_launch") if c else None


def gpu_simplices(points, dev):
    """Tetrahedra [T, 4] of float32 points by the library's GPU Delaunay
    (Qhull on every point where it falls back)."""
    import numpy as np
    import torch

    from sdfoam_amd.triangulation import _Undecided, gpu_tetrahedra, qhull_tetrahedra

    pts = torch.from_numpy(np.ascontiguousarray(points, dtype=np.float32)).to(dev)
    try:
        return gpu_tetrahedra(pts)[0].cpu().numpy()
    except _Undecided:
        return qhull_tetrahedra(points)[0]


def triangulate_bench(args, dev) -> int:
    """Triangulation.rebuild(points, incremental=False) on the C3 point set
    (850k noisy superquadric surface points and 150k uniform ones; --config 4:
    C4's 1.8M blob and 1.2M 1/r^2 shell points): the
    reference's rebuild (src/delaunay/delaunay.cu:271-345) with the point
    order, the tetrahedralisation and every table.  Each step is one
    rebuild; the CPU baseline is Qhull (scipy) on every point, once.  The
    certify kernel is latency-bound per-lane clipping in fp64, far from the
    HBM roofline: the roofline entry reports its algorithmic bytes (points
    in, report rows out) over the time of the certify call."""
    import numpy as np
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes
    from sdfoam_amd.triangulation import qhull_tetrahedra

    if args.config == 4:
        pts_np, _ = scenes._scene_blobs_shell(np.random.default_rng(4), 1_800_000, 1_200_000)
    elif args.config == 3:
        pts_np, _ = scenes._scene_c3(np.random.default_rng(0))
    else:
        raise SystemExit("--triangulate takes --config 3 (default) or 4")
    pts = torch.from_numpy(np.ascontiguousarray(pts_np, dtype=np.float32)).to(dev)
    n = pts.shape[0]
    tri = sdfoam_amd.Triangulation(pts[:50_000].contiguous())  # warm the kernels
    for _ in range(args.warmup):
        tri.rebuild(pts, incremental=False)
    torch.cuda.synchronize()
    stats = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tri.rebuild(pts, incremental=False)
        stats.append(tri.last_stats)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    if tri.last_method != "gpu":
        raise RuntimeError("the GPU tetrahedralisation fell back to Qhull")
    last = stats[-1]
    certify = float(np.mean([s["certify_s"] for s in stats]))
    # incremental rebuilds (the reference's rebuild(points, true) between
    # full ones): the sorted points moved by --perturb of their cell radius
    base = pts[tri.permutation().view(torch.int32).long()].contiguous()
    _, radius = sdfoam_amd.farthest_neighbor(base, tri.point_adjacency(),
                                             tri.point_adjacency_offsets())
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    inc = []
    for i in range(args.warmup + args.steps):
        moved = base + args.perturb * radius[:, None] * torch.randn(
            base.shape, generator=gen, device=dev)
        if i == args.warmup:
            torch.cuda.synchronize()
            t_inc = time.perf_counter()
        tri.rebuild(moved, incremental=True)
        if i >= args.warmup:
            inc.append(tri.last_stats)
    torch.cuda.synchronize()
    dt_inc = (time.perf_counter() - t_inc) / args.steps
    if tri.last_method != "gpu":
        raise RuntimeError("the GPU tetrahedralisation fell back to Qhull")
    inc_done = [s for s in inc if s.get("incremental")]
    sorted_pts = base.cpu().numpy()
    tq = time.perf_counter()
    qhull_tetrahedra(sorted_pts)
    t_qhull = time.perf_counter() - tq
    algo_bytes = 12 * n + 16 * last["reports"]
    achieved = algo_bytes / certify / 1e9
    result = {
        "metric": TRI_METRIC,
        "value": 1.0 / dt,
        "unit": "rebuilds/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"Triangulation.rebuild of the C{args.config} point set",
                   "points": n, "tets": last["tets"]},
        "phases_s": {"certify": certify,
                     "open_points_qhull": float(np.mean([s["open_points_qhull_s"] for s in stats])),
                     "merge": float(np.mean([s["merge_s"] for s in stats]))},
        "open_points": last["open"],
        "open_levels": last.get("open_levels", []),
        "qhull_points": last.get("open_points_qhull"),
        "open_phase_s": {"levels": last.get("open_levels_s"), "qhull": last.get("open_qhull_s")},
        "incremental": {
            "ms_per_rebuild": dt_inc * 1e3, "perturb": args.perturb,
            "rebuilds": len(inc), "incremental": len(inc_done),
            "fallback": [s["incremental_fallback"] for s in inc if "incremental_fallback" in s][:1],
            "dirty_points": int(np.mean([s["dirty"] for s in inc_done])) if inc_done else None,
            "kept_old_tets": int(np.mean([s["kept_old"] for s in inc_done])) if inc_done else None,
            "open_points": int(np.mean([s["open"] for s in inc_done])) if inc_done else None,
            "phases_s": {k: float(np.mean([s[k + "_s"] for s in inc_done]))
                         for k in ("check", "certify", "open_points_qhull", "merge", "select")}
            if inc_done else None},
        "roofline": {"kernel": "certify_kernel", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic(f"traffic_certify_C{args.config}.json")},
        "cpu_baseline": {"value": 1.0 / t_qhull, "unit": "rebuilds/s", "cores": 1,
                         "kind": "library",
                         "sample": "Qhull (scipy.spatial.Delaunay) on all 1M points, once; "
                                   "tetrahedra only, no tables"},
    }
    print(json.dumps(result), flush=True)
    return 0


def fetch_bench(args, dev) -> int:
    """Two BatchFetchers over parallel host arrays, as the reference's data
    loader drives them (data_loader/__init__.py:126-141, train.py:130-131):
    rays [M, 6] and colours [M, 3] float32, M = 64 x 960 x 640, batches of
    2^20 shuffled rows.  Timed: `steps` pairs of next() with the copies done
    on the GPU, for the device-resident fetchers (the default here: the
    arrays are uploaded once and each batch is gathered on the GPU) and for
    the streamed ones (host gather and upload, as the reference does).  The
    naive path (numpy gather of the same rows, then a pageable copy to the
    device) is timed beside them.  The roofline entry prices the resident
    gather against HBM: per row 36 bytes read (each row on its own) and 36
    written."""
    import numpy as np
    import torch

    import sdfoam_amd

    M = 64 * 960 * 640
    B = 1 << 20
    rng = np.random.default_rng(0)
    rays = torch.from_numpy(rng.standard_normal((M, 6), dtype=np.float32))
    rgb = torch.from_numpy(rng.random((M, 3), dtype=np.float32))
    log(f"host arrays ready: {M} rows ({(rays.nbytes + rgb.nbytes) / 1e9:.2f} GB)")

    def time_pairs(resident):
        fr = sdfoam_amd.BatchFetcher(rays, B, True, resident=resident)
        fc = sdfoam_amd.BatchFetcher(rgb, B, True, resident=resident)
        for _ in range(args.warmup):
            fr.next()
            fc.next()
        torch.cuda.synchronize()
        # the gathers run on the current stream, where these events sit
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            fr.next()
            fc.next()
        e1.record()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / args.steps
        fr.close()
        fc.close()
        return dt, e0.elapsed_time(e1) * 1e-3 / args.steps

    dt, dt_kernels = time_pairs(True)
    dt_streamed, _ = time_pairs(False)
    batch_bytes = B * (24 + 12)
    # naive host path for the same batch shape
    t0 = time.perf_counter()
    n_naive = 3
    for _ in range(n_naive):
        idx = rng.integers(0, M, size=B)
        ra = torch.from_numpy(rays.numpy()[idx]).to(dev)
        ca = torch.from_numpy(rgb.numpy()[idx]).to(dev)
    torch.cuda.synchronize()
    dt_naive = (time.perf_counter() - t0) / n_naive
    del ra, ca
    achieved = batch_bytes / dt / 1e9
    hbm = 2 * batch_bytes / dt_kernels / 1e9
    result = {
        "metric": FETCH_METRIC,
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "batches_per_s": 1.0 / dt,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"BatchFetcher x2 (rays [M,6], rgb [M,3] float32), M={M}, "
                               f"batch {B} shuffled rows, device-resident", "rows": M,
                   "batch": B},
        "roofline": {"kernel": "batch_gather_kernel", "bound": "hbm", "achieved": hbm,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": hbm / HBM_PEAK_GBS,
                     "traffic": load_traffic("traffic_batch_gather_fetch.json")},
        "kernel_ms_per_step": dt_kernels * 1e3,
        "streamed_ms_per_step": dt_streamed * 1e3,
        "streamed_GBps": batch_bytes / dt_streamed / 1e9,
        "streamed_host_link_frac": batch_bytes / dt_streamed / 1e9 / HOST_LINK_PEAK_GBS,
        "naive_host_ms_per_step": dt_naive * 1e3,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


RENDER_WEIGHT_THRESHOLD = 0.05  # the reference's benchmark.py


def render_bench(args, w, pts, attrs, adj, offs, inv, pipe, D) -> int:
    """Frames of Pipeline.trace_benchmark on the configuration's camera: the
    reference's inference benchmark (benchmark.py:41-147) on a synthetic
    scene.  Timed: the render kernel alone (the offset table and the start
    cell are built once, as benchmark.py builds them once)."""
    import numpy as np
    import torch

    import sdfoam_amd
    from sdfoam_amd import _lib, scenes

    if args.config not in (1, 2, 3):
        print("--render needs a single-camera config (1-3)", file=sys.stderr)
        return 2
    dev = pts.device
    cam = scenes.camera_dict(w.extra["camera"], "pinhole")
    H, W = int(cam["height"]), int(cam["width"])
    cam_t = dict(cam)
    for k in ("position", "forward", "right", "up"):
        cam_t[k] = torch.tensor(np.asarray(cam[k], dtype=np.float32))
    diff = sdfoam_amd.prefetch_adjacent_diff(pts, adj, offs)
    ray0 = np.concatenate([cam["position"], cam["forward"]]).reshape(1, 6).astype(np.float32)
    start_np = scenes.start_points_for(w.points, ray0).astype(np.uint32)
    start = torch.from_numpy(start_np.view(np.int32)).to(dev).view(torch.uint32)
    out = torch.zeros((H, W), dtype=torch.uint32, device=dev)

    def frame():
        pipe.trace_benchmark(pts, attrs, adj, offs, diff, cam_t, start, out,
                             weight_threshold=RENDER_WEIGHT_THRESHOLD,
                             alpha_mode=args.alpha_mode, inv_s=inv)

    for _ in range(args.warmup):
        frame()
    torch.cuda.synchronize()
    _lib.set_timing(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        frame()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    launches = _lib.collect_timings()
    _lib.set_timing(False)
    ms_frame = (t1 - t0) * 1e3 / args.steps
    render_ms = float(np.mean([ms for name, ms in launches if name == "render"]))
    # byte model of the render: per pixel the RGBA8 store; per step the CSR
    # bounds, the face rows, the next index and position, the attribute row
    rays = torch.from_numpy(w.rays).to(dev)
    st = pipe.walk_stats(pts, attrs, adj, offs, rays,
                         torch.from_numpy(scenes.start_points_for(w.points, w.rays)
                                          .astype(np.uint32).view(np.int32)).to(dev)
                         .view(torch.uint32),
                         alpha_mode=args.alpha_mode, inv_s=inv,
                         weight_threshold=RENDER_WEIGHT_THRESHOLD)
    torch.cuda.synchronize()
    S = int(st["steps"].sum().item())
    F_st = int(st["faces_stepped"].sum().item())
    ab = 2 if args.attr_dtype == "float16" else 4
    R = H * W
    bytes_frame = R * 4 + S * (8 + 4 + 12 + ab * D) + 8 * F_st
    achieved = bytes_frame / (render_ms * 1e-3) / 1e9
    traffic = None
    if args.alpha_mode == "sdfoam" and args.attr_dtype == "float32":
        traffic = load_traffic(f"traffic_render_C{args.config}.json")
    result = {
        "metric": RENDER_METRIC,
        "value": R / (ms_frame * 1e-3) / 1e6,
        "unit": "Mpixels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_frame,
        "fps": 1e3 / ms_frame,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"C{args.config} camera {W}x{H}, {w.num_points} points, SH degree "
                        f"{w.sh_degree}, {args.alpha_mode} alpha, {args.attr_dtype} attributes, "
                        f"weight threshold {RENDER_WEIGHT_THRESHOLD}, inv_s={w.inv_s:.4f}",
            "points": w.num_points,
            "pixels": R,
        },
        "kernel_ms": {"render": render_ms},
        "cell_steps_per_pixel": S / R,
        "roofline": {"kernel": "render", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic},
    }
    if args.cpu_stride != 0:
        from oracle import oracle

        # the same frame on the host (C3: about 7 s on 16 threads)
        oracle.build()
        small = cam
        diff_np = diff.view(torch.int16).cpu().numpy().view(np.uint16)[: w.adjacency.size]
        threads = cpu_threads()
        t = time.perf_counter()
        oracle.trace_benchmark(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                               diff_np, small, int(start_np[0]), alpha_mode=args.alpha_mode,
                               inv_s=w.inv_s, weight_threshold=RENDER_WEIGHT_THRESHOLD,
                               threads=threads)
        dt = time.perf_counter() - t
        result["cpu_baseline"] = {
            "value": W * H / dt / 1e6, "unit": "Mpixels/s", "cores": threads, "kind": "port",
            "sample": f"one {W}x{H} frame of the same camera, {dt:.1f}s on {threads} threads "
                      f"of {cpu_model()}"}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline(w, rays, start, quantiles, grad_rgba, depth_grad, stride: int,
                 alpha_mode: str = "sdfoam") -> dict:
    """Scalar host oracle (fp32 attributes), forward + backward, every
    `stride`-th ray."""
    import numpy as np

    from oracle import oracle

    oracle.build()
    threads = cpu_threads()

    def run(step, nthreads):
        r = rays.reshape(-1, 6)[::step]
        sp = start.reshape(-1)[::step]
        qv = quantiles.reshape(-1, quantiles.shape[-1])[::step]
        g = grad_rgba.reshape(-1, 4)[::step]
        dg = depth_grad.reshape(-1, depth_grad.shape[-1])[::step]
        log(f"CPU baseline: {r.shape[0]} rays on {nthreads} threads")
        t0 = time.perf_counter()
        f = oracle.trace_forward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, r,
                                 sp, qv, alpha_mode=alpha_mode, inv_s=w.inv_s, threads=nthreads)
        oracle.trace_backward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, r, sp,
                              f.rgba, g, qv, f.depth_indices, dg, alpha_mode=alpha_mode,
                              inv_s=w.inv_s, threads=nthreads, side_buffers=False)
        dt = time.perf_counter() - t0
        log(f"CPU baseline: {dt:.1f}s")
        return r.shape[0], int(np.sum(f.steps)), dt

    n, steps, dt = run(stride, threads)
    # one thread on 1 ray in 48 or fewer (a few seconds)
    stride1 = max(stride * 16, 48)
    n1, steps1, dt1 = run(stride1, 1)
    return {
        "value": n / dt / 1e6,
        "unit": "Mrays/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"every ray of the same workload ({n} rays" if stride == 1 else
                   f"1 ray in {stride} of the same workload ({n} rays") + f", {steps} cell steps), "
                  f"forward + backward, {dt:.1f}s on {threads} threads (every CPU the process "
                  f"may use) of {cpu_model()}",
        "cell_steps_per_s": steps / dt,
        "cpu_model": cpu_model(),
        "affinity_cpus": cpu_affinity(),
        "cgroup_cpu_quota": cpu_quota(),
        "single_thread": {"value": n1 / dt1 / 1e6, "unit": "Mrays/s", "cores": 1,
                          "cell_steps_per_s": steps1 / dt1,
                          "sample": f"1 ray in {stride1} ({n1} rays, {steps1} cell steps), "
                                    f"{dt1:.1f}s on one thread"},
    }


if __name__ == "__main__":
    sys.exit(main())
