"""Benchmark of the rasterizer hot path on one MI355X.

Default (`--workload step --config 2`): one step = one training forward+backward
of the reference's split rasterizer path on config 2 of BASELINE.json
(6,000,000 SH-degree-3 Gaussians, city-scale aerial scene, 1600x1066 camera):
preprocess forward -> binning + render forward -> render backward
(dL/dimage ~ N(0,1)) -> preprocess backward, driven through the drop-in
autograd API exactly as gaussian_renderer does.  Config 1 adds the reference's
training loss 0.8 * L1 + 0.2 * (1 - fused_ssim) against a seeded target; config
3 renders one rank's share (tile rows [43, 86) of 4096x2730).  Inputs are
generated once (seeded, synthetic) and stay resident in HBM.

`--workload knn`: distCUDA2 over config 4's 10M points.  `--workload ssim`:
fused_ssim forward+backward on config 4's 8 x 3 x 1080 x 1920 image pair.
`--workload adam`: the SparseGaussianAdam step over config 2's 6M Gaussians.
`--workload route`: one rank's routing + pack/unpack around the screen-space
all-to-all, config 3's 8M Gaussians split over four tile-row ranks.
`--workload full`: the full-image path (GaussianRasterizer.forward + backward,
and render_simp) on a config's scene.  `--workload ply`: the trained-scene PLY
layer (records <-> parameter tensors) at config 2's size, plus one file
save + load timed end to end.  `--workload geo`: the render forward with
render_geo (the five geometry maps and the plane depth) at a config's size,
fused into the colour's walk of the lists, against the colour-only forward and
a second walk.

Prints ONE JSON line.  For the step, `value` is Gaussians/s = P / step time.
`roofline` describes the dominant kernel, timed live with HIP events on the
launch stream inside the timed region; `cpu_baseline` times the CPU oracle
(oracle/, fp32 C with OpenMP) on a bounded sample of the same workload on this
host.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
STEP_METRIC = "rasterizer fwd+bwd ms/iter & Gaussians/s at 6M SH3 1600x1066; % HBM roofline"


# algorithmic bytes per unit of work, per stage (the scope table's per-unit figures)
def stage_bytes(P, P_vis, R, npx, E=None):
    """Algorithmic HBM bytes per launch (per step for binning and other): P
    Gaussians, P_vis of them visible (radius > 0; the listed ones, which touch
    a tile, are counted as P_vis), R tile instances, npx pixels, E region-list
    entries of the split path's binning (region_entries; None: the full-image
    path's per-tile binning)."""
    if E is None:
        # count: radius + means2D of all (12 B); scatter: the same again, compact index and out_observe (8 B)
        # of all, depth/conic/rgb (32 B) of the listed, their 64-byte record and id (68 B); per instance the
        # key written and read back (16 B) and the compact list written (4 B)
        binning = 32 * P + 100 * P_vis + 20 * R
    else:
        # count and scatter as above; per region-list entry 12 B written and read back, per instance the
        # compact list written (4 B)
        binning = 32 * P + 100 * P_vis + 24 * E + 4 * R
    return {
        # reads means3D, scales, rotations, opacity (44 B) of all, SH (192 B) of the visible; writes means2D,
        # depth, radius, conic+opacity, rgb (44 B) of all, the backward's 48-byte record of the visible and a
        # 64-bit mask per 64 Gaussians (cov3D is recomputed by the backward, the records hold the clamp flags)
        "preprocess_fwd_kernel": 88 * P + P // 8 + 240 * P_vis,
        # writes dL/dmeans3D, dL/dscales, dL/drotations, dL/dopacity (44 B) and reads dL/dopacity (4 B) of all
        # and the masks; reads the record, the rest of dL/dconic_opacity, dL/dmeans2D, dL/drgb and SH (272 B)
        # and writes the dL/dsh row (192 B) of the visible (the render backward cleared dL/dsh)
        "preprocess_bwd_kernel": 48 * P + P // 8 + 464 * P_vis,
        "binning": binning,
        "render_fwd_kernel": 40 * R + 24 * npx,
        # the blend's reads and writes, and the zeros of dL/dsh (192 B of every Gaussian) that it clears for
        # the preprocess backward while its VALU-bound walk runs
        "render_bwd_kernel": 40 * R + 32 * npx + 192 * P,
        # the accumulators cleared (64 B per listed), then the gradient unpack: compact index of all (4 B),
        # accumulators of the listed (48 B), four gradient rows of all written (48 B)
        "other": 64 * P_vis + 4 * P + 48 * P_vis + 48 * P,
    }


BINNING_KERNELS = ("localmap_kernel", "count_regions_kernel", "scan_regions_kernel", "ranges_kernel",
                   "scatter_regions_kernel", "regionsort_small_kernel",
                   "regionsort_kernel_8k", "regionsort_big_kernel",
                   # the full-image path's per-tile binning
                   "count_kernel", "tilescan_kernel", "scatter_kernel",
                   "tilesort_kernel_1k", "tilesort_kernel_2k", "tilesort_kernel_4k", "tilesort_kernel_8k")
# the library's stage mark around the whole binning on the caller's stream
# (first binning kernel -> end of the sorts)
BINNING_STAGE = "binning (wall)"
STEP_STAGES = ("preprocess_fwd_kernel", "render_fwd_kernel", "render_bwd_kernel", "preprocess_bwd_kernel")
# kernels timed under the name of the stage they implement (the preprocess
# backward's packed form, taken when the render backward has cleared dL/dsh)
STAGE_OF_KERNEL = {"preprocess_bwd_packed_kernel": "preprocess_bwd_kernel"}


def region_entries(means2D, radii, W, H, cl=None, side=0):
    """Entries of the split path's region lists: per listed Gaussian, the
    RS x RS-tile regions that its tile rect, clipped to the box of the local
    tiles, meets, regions tiling the box from its corner; RS is the larger of
    `side` (the forward's region_side argument) and the smallest of 2, 4, 8
    that gives at most 16384 regions.  Exact when the local tiles fill their
    box (no mask, or whole tile rows / columns), an upper bound otherwise."""
    import torch
    gx, gy = (W + 15) // 16, (H + 15) // 16
    rs = next((s for s in (2, 4, 8) if ((gx + s - 1) // s) * ((gy + s - 1) // s) <= 16384), 8)
    rs = max(rs, side)
    bx0, by0, bx1, by1 = 0, 0, gx, gy
    if cl is not None:
        cols = torch.nonzero(cl.reshape(gy, gx).any(0)).flatten()
        rows = torch.nonzero(cl.reshape(gy, gx).any(1)).flatten()
        if cols.numel() == 0:
            return 0
        bx0, bx1, by0, by1 = int(cols[0]), int(cols[-1]) + 1, int(rows[0]), int(rows[-1]) + 1
    r = radii.float()
    m = means2D.detach().float()
    tile = lambda v, n: torch.nan_to_num(torch.trunc(v / 16.0), nan=0.0).clamp(0, n).long()
    x0 = tile(m[:, 0] - r, gx).clamp(bx0, bx1)
    y0 = tile(m[:, 1] - r, gy).clamp(by0, by1)
    x1 = tile(m[:, 0] + r + 15.0, gx).clamp(bx0, bx1)
    y1 = tile(m[:, 1] + r + 15.0, gy).clamp(by0, by1)
    ok = (radii > 0) & (x1 > x0) & (y1 > y0)
    nx = torch.div(x1 - 1 - bx0, rs, rounding_mode="floor") - torch.div(x0 - bx0, rs, rounding_mode="floor") + 1
    ny = torch.div(y1 - 1 - by0, rs, rounding_mode="floor") - torch.div(y0 - by0, rs, rounding_mode="floor") + 1
    return int(torch.where(ok, nx * ny, torch.zeros_like(nx)).sum().item())


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["step", "knn", "ssim", "adam", "route", "full", "ply", "geo"],
                    default="step")
    ap.add_argument("--config", type=int, default=2, choices=[0, 1, 2, 3])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=float, default=1.0,
                    help="fraction of the Gaussians (step) or points (knn) the CPU baseline runs on")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run the library's plain copy kernel on MIB MiB (5 launches): the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE, then exit")
    ap.add_argument("--valu-probes", action="store_true",
                    help="only run the blend kernels' VALU probes (gs_diag_math ops 7 and 8, one launch each at "
                         "the iteration counts the bench times them at): the launches whose SQ_INSTS_VALU "
                         "profiles/valu_probes.json records, then exit")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def copy_peak(mib=1024, reps=5):
    """Measured stream-copy bandwidth (read + write bytes / time) of the library's copy kernel."""
    import torch
    from blitzgs_amd import _lib
    lib = _lib.load()
    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda:0")
    y = torch.empty_like(x)
    stream = _lib.stream_of(x.device)
    _lib.check(lib.gs_diag_math(4, n, _lib.ptr(x), _lib.ptr(y), stream), "gs_diag_math copy")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        _lib.check(lib.gs_diag_math(4, n, _lib.ptr(x), _lib.ptr(y), stream), "gs_diag_math copy")
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    assert bool((y == 1).all())
    del x, y
    return 2 * 4 * n / (ms * 1e-3) / 1e9


def calibrate_copy(mib):
    import torch
    from blitzgs_amd import _lib
    lib = _lib.load()
    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda:0")
    y = torch.empty_like(x)
    stream = _lib.stream_of(x.device)
    for _ in range(5):
        _lib.check(lib.gs_diag_math(4, n, _lib.ptr(x), _lib.ptr(y), stream), "gs_diag_math copy")
    torch.cuda.synchronize()
    assert bool((y == 1).all())
    print(json.dumps({"copy_kernel": "diag_copy_kernel", "bytes_read": 4 * n, "bytes_written": 4 * n,
                      "launches": 5}), flush=True)


STEP_TIMES = {}


def step_times(fn, steps):
    """`steps` calls of fn bracketed by synchronisation, a HIP event on the
    current stream before every call and after the last: (median ms of the
    per-call intervals, mean ms over the whole region)."""
    import torch
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    for i in range(steps):
        evs[i].record()
        fn()
    evs[steps].record()
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return float(np.median(per)), evs[0].elapsed_time(evs[steps]) / steps


def timed(fn, steps, warmup):
    """Run fn warmup times, then two timed regions of `steps` calls, each
    bracketed by synchronisation: the first without instrumentation (the step
    time: the median of the per-call intervals; the mean over the region is
    kept in STEP_TIMES), the second with the library's per-kernel HIP events
    recorded on the launch stream around every kernel (the per-kernel
    durations).  Returns (median ms per step, per-kernel {name: (total ms,
    launches)}, instrumented ms per step)."""
    import torch
    from blitzgs_amd import _lib
    for _ in range(warmup):
        fn()
    ms, ms_mean = step_times(fn, steps)
    STEP_TIMES["median_ms"], STEP_TIMES["mean_ms"] = ms, ms_mean
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _lib.timing_reset()
    _lib.timing_enable(True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(steps):
        fn()
    ev1.record()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    kt = _lib.timing_read()
    ms_instr = ev0.elapsed_time(ev1) / steps
    if BINNING_STAGE in kt:
        # the binning's wall time again, with the stage marks alone (per-kernel
        # events add a gap between the stage's launches)
        _lib.timing_reset()
        _lib.timing_enable(True, stages_only=True)
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        _lib.timing_enable(False)
        ks = _lib.timing_read()
        if BINNING_STAGE in ks:
            kt[BINNING_STAGE + " with kernel events"] = kt[BINNING_STAGE]
            kt[BINNING_STAGE] = ks[BINNING_STAGE]
    return ms, kt, ms_instr


def valu_peak(iters=2000, reps=5):
    """Measured VALU issue rate in G wave-instructions/s: the library's FMA
    probe (8192 blocks x 4 waves x 32 * iters independent-chain fp32 FMAs),
    best of `reps` launches."""
    import torch
    from blitzgs_amd import _lib
    lib = _lib.load()
    y = torch.zeros(1, device="cuda:0")
    stream = _lib.stream_of(y.device)
    _lib.check(lib.gs_diag_math(5, 10, None, _lib.ptr(y), stream), "gs_diag_math valu")
    best = float("inf")
    for _ in range(reps):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        _lib.check(lib.gs_diag_math(5, iters, None, _lib.ptr(y), stream), "gs_diag_math valu")
        ev1.record()
        torch.cuda.synchronize()
        best = min(best, ev0.elapsed_time(ev1))
    return 8192 * 4 * 32 * iters / (best * 1e-3) / 1e9


# the blend kernels' VALU probes: gs_diag_math op, kernel name, iterations
VALU_PROBES = {"render_fwd_kernel": (7, "valu_probe_fwd_kernel", 24),
               "render_bwd_kernel": (8, "valu_probe_bwd_kernel", 8),
               # the backward's 16x8 half-tile walk (two pixels per lane), which the kernel takes when the
               # Gaussians average 24 or more tile instances (R >= 24 L)
               "render_bwd_kernel_half_tiles": (9, "valu_probe_bwd2_kernel", 8)}
TWO_PX_MIN_INSTANCES = 24


def run_valu_probe(op, iters, reps=5):
    """Best-of-`reps` time (ms) of one VALU probe launch."""
    import torch
    from blitzgs_amd import _lib
    lib = _lib.load()
    y = torch.zeros(1, device="cuda:0")
    stream = _lib.stream_of(y.device)
    _lib.check(lib.gs_diag_math(op, 1, None, _lib.ptr(y), stream), "gs_diag_math probe")
    best = float("inf")
    for _ in range(reps):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        _lib.check(lib.gs_diag_math(op, iters, None, _lib.ptr(y), stream), "gs_diag_math probe")
        ev1.record()
        torch.cuda.synchronize()
        best = min(best, ev0.elapsed_time(ev1))
    return best


def valu_probes_only():
    for name, (op, pname, iters) in VALU_PROBES.items():
        ms = run_valu_probe(op, iters, reps=1)
        log(f"[bench] {pname}: {iters} iterations, {ms:.3f} ms")


def valu_of(name, avg_ms, config, probe=None):
    """VALU issue rate of kernel `name` per launch: SQ_INSTS_VALU per launch
    (profiles/valu_config<N>.json, rocprofv3 --pmc) over its live launch time,
    against the ceiling for its instruction mix: the issue rate of its VALU
    probe (the same per-entry arithmetic with no memory traffic; instructions
    per probe launch in profiles/valu_probes.json, the probe timed live)."""
    f = os.path.join(ROOT, "profiles", f"valu_config{config}.json")
    try:
        insts = json.load(open(f))[name]["SQ_INSTS_VALU"]
    except (OSError, ValueError, KeyError):
        return None
    achieved = insts / (avg_ms * 1e-3) / 1e9
    out = {"unit": "G wave-instructions/s", "insts_per_launch": int(insts), "achieved": round(achieved, 1),
           "fma_rate": round(valu_peak(), 1)}
    probe = probe or name
    if probe in VALU_PROBES:
        op, pname, iters = VALU_PROBES[probe]
        try:
            pj = json.load(open(os.path.join(ROOT, "profiles", "valu_probes.json")))[pname]
            assert int(pj["iters"]) == iters
            peak = pj["SQ_INSTS_VALU"] / (run_valu_probe(op, iters) * 1e-3) / 1e9
            out.update(peak=round(peak, 1), frac=round(achieved / peak, 4),
                       peak_is=f"measured VALU issue rate of the kernel's own per-entry arithmetic "
                               f"({pname}, gs_diag_math op {op}: no memory traffic, {iters} x 64 entries per wave)")
        except (OSError, ValueError, KeyError, AssertionError):
            pass
    return out


def roofline_of(name, alg_bytes, avg_ms, traffic=None):
    achieved = alg_bytes / (avg_ms * 1e-3) / 1e9
    return {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "avg_launch_ms": round(avg_ms, 4),
            "alg_bytes_per_launch": int(alg_bytes)}


def header(args, metric, value, unit, ms, dtype, workload, extra_cfg):
    return {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded PCG64)",
            "config": dict({"workload": workload, "parallelism": "single-gpu"}, **extra_cfg)}


# ------------------------------------------------------------------ step

def run_step(args):
    import torch
    from blitzgs_amd import _lib, synth
    from blitzgs_amd.rasterizer import GaussianRasterizationSettings, GaussianRasterizer
    dev = torch.device("cuda:0")
    peak_copy = copy_peak()

    t0 = time.time()
    gen = {0: synth.config0, 1: synth.config1, 2: synth.config2, 3: synth.config3}[args.config]
    scene, cam = gen()
    log(f"[bench] scene config {args.config} generated in {time.time() - t0:.1f}s")
    P = scene["means3D"].shape[0]
    W, H = cam["W"], cam["H"]
    T = ((W + 15) // 16) * ((H + 15) // 16)
    tt = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)
    params = {k: tt(scene[k]).requires_grad_(True) for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    dL_dimage = tt(scene.get("dL_dimage", np.random.default_rng(0).standard_normal((3, H, W)).astype(np.float32)))
    cl = tt(scene["compute_locally"]).bool() if "compute_locally" in scene else None
    rs = GaussianRasterizationSettings(
        image_height=H, image_width=W, tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
        bg=torch.zeros(3, device=dev), scale_modifier=1.0, viewmatrix=tt(cam["viewmatrix"]),
        projmatrix=tt(cam["projmatrix"]), sh_degree=3, campos=tt(cam["campos"]), prefiltered=False, debug=False)
    ras = GaussianRasterizer(rs)
    means2D_abs = torch.zeros((P, 3), device=dev, requires_grad=True)
    all_map = torch.zeros((P, 5), device=dev)
    # as gaussian_renderer passes them (its stats_collector makes every render
    # forward and backward wait on an event for its timers), and without the
    # collector (no host wait inside the step)
    cuda_args_train = {"avoid_pixel_all2all": False, "stats_collector": {}}
    cuda_args = {"avoid_pixel_all2all": False}
    info = {}
    loss_desc = "dL/dimage ~ N(0,1)"
    target = None
    if args.config == 1:
        from blitzgs_amd.ssim import fused_ssim
        target = tt(np.random.Generator(np.random.PCG64(101)).random((3, H, W), dtype=np.float32))
        loss_desc = "0.8 * L1 + 0.2 * (1 - fused_ssim) vs a seeded U[0,1] target (reference training loss)"

    def step(ca=cuda_args):
        for p in params.values():
            p.grad = None
        means2D_abs.grad = None
        means2D, rgb, conic_opacity, radii, depths = ras.preprocess_gaussians(
            params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], ca)
        color, n_render, n_consider, n_contrib, out_observe, _, _ = ras.render_gaussians(
            means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, cl, cl, ca)
        if target is None:
            torch.autograd.backward([color], [dL_dimage])
        else:
            loss = 0.8 * (color - target).abs().mean() + 0.2 * (1.0 - fused_ssim(color[None], target[None]))
            loss.backward()
        info["radii"] = radii
        info["means2D"] = means2D
        info["n_render"] = n_render
        info["n_consider"] = n_consider

    ms_per_step, kt, ms_instr = timed(step, args.steps, args.warmup)
    ms_mean = STEP_TIMES["mean_ms"]
    ms_train, ms_train_mean = step_times(lambda: step(cuda_args_train), args.steps)
    P_vis = int((info["radii"] > 0).sum().item())
    R = int(info["n_render"].sum().item())
    E = int(info["n_consider"].sum().item())
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step median ({ms_mean:.3f} mean; {ms_instr:.3f} with "
        f"per-kernel events; {ms_train:.3f} with cuda_args['stats_collector'])")

    for k, stage in STAGE_OF_KERNEL.items():
        if k in kt:
            t, n = kt.pop(k)
            t0, n0 = kt.get(stage, (0.0, 0))
            kt[stage] = (t0 + t, n0 + n)
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    stages = {k: per_kernel.get(k, 0.0) for k in STEP_STAGES}
    binning_kernels_ms = sum(per_kernel.get(k, 0.0) for k in BINNING_KERNELS)
    stages["binning"] = per_kernel.get(BINNING_STAGE, binning_kernels_ms)
    avg_launch["binning"] = avg_launch.get(BINNING_STAGE, binning_kernels_ms)
    stages["other"] = sum(v for k, v in per_kernel.items()
                          if k not in stages and k not in BINNING_KERNELS and not k.startswith(BINNING_STAGE))
    E_reg = region_entries(info["means2D"], info["radii"], W, H, cl, side=_lib.RESERVE.region_side(dev))
    sb = stage_bytes(P, P_vis, R, W * H, E_reg)
    stage_rows = {}
    for k, ms in stages.items():
        gbs = sb[k] / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        stage_rows[k] = {"ms": round(ms, 4), "alg_GB": round(sb[k] / 1e9, 4), "GB_per_s": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if args.verbose:
        for k, v in sorted(per_kernel.items(), key=lambda x: -x[1]):
            log(f"[bench]   {k:28s} {v:8.4f} ms/step  ({kt[k][1] // max(1, args.steps)} launches)")
    dom = max(STEP_STAGES + ("binning",), key=lambda k: stages.get(k, 0.0))
    traffic = None
    tf = os.path.join(ROOT, "profiles", f"traffic_config{args.config}.json")
    if os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get(dom)
        except (OSError, ValueError):
            traffic = None
    roofline = roofline_of(dom, sb[dom], avg_launch.get(dom, float("nan")), traffic)
    if dom == "binning":
        roofline["note"] = ("binning = tile count, scan, duplication and the per-tile sorts, timed as one stage on "
                            "the caller's stream (wall clock from the first binning kernel to the end of the sorts; "
                            "the forward is queued in one call, so no host round trip falls inside)")
    elif dom in VALU_PROBES:
        roofline["limiter"] = "valu"
        roofline["note"] = ("`bound` and `frac` are the HBM roofline (algorithmic bytes / launch time) the line format "
                            "asks for; this blend kernel is limited by VALU issue, not HBM: `valu.frac` is its VALU "
                            "instruction rate over that of its own per-entry arithmetic run with no memory traffic")
        # the backward's walk: 16x8 half tiles when R >= 24 L (L: the listed Gaussians, here those with a radius)
        half = dom == "render_bwd_kernel" and R >= TWO_PX_MIN_INSTANCES * P_vis
        roofline["valu"] = valu_of(dom, avg_launch.get(dom, float("nan")), args.config,
                                   "render_bwd_kernel_half_tiles" if half else None)
    else:
        roofline["note"] = "HBM roofline of the kernel (algorithmic bytes / launch time)"

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_step(scene, cam, args.cpu_sample, cl)

    metric = STEP_METRIC if args.config == 2 else f"rasterizer fwd+bwd ms/iter & Gaussians/s, config {args.config}"
    out = header(args, metric, P / (ms_per_step * 1e-3), "Gaussians/s", ms_per_step, "f32",
                 f"config{args.config}: {P} Gaussians SH3, {W}x{H}, fwd+bwd",
                 {"gaussians": P, "visible": P_vis, "instances": R, "region_entries": E_reg, "image": [W, H],
                  "tiles": T,
                  "local_tiles": int(cl.sum().item()) if cl is not None else T, "loss": loss_desc})
    out["stages_ms"] = stage_rows
    out["stages_note"] = ("per-kernel HIP-event times; `binning` is the wall time of the whole stage on the caller's "
                          "stream, timed in a run with only the stage's two marks (its kernels overlap on two side "
                          "streams; their summed times are binning_kernels_ms; binning_wall_with_kernel_events_ms is "
                          "the same wall in the run with an event pair around every kernel)")
    out["binning_kernels_ms"] = round(binning_kernels_ms, 4)
    if BINNING_STAGE + " with kernel events" in per_kernel:
        out["binning_wall_with_kernel_events_ms"] = round(per_kernel[BINNING_STAGE + " with kernel events"], 4)
    out["ms_per_step_note"] = ("median of the per-step intervals (HIP events between the steps) over the timed "
                               "steps after the warm-up steps; ms_per_step_mean is the whole timed region / steps")
    out["ms_per_step_mean"] = round(ms_mean, 4)
    out["ms_per_step_with_stats_collector"] = {
        "median": round(ms_train, 4), "mean": round(ms_train_mean, 4),
        "note": "the same step with cuda_args['stats_collector'] set, as gaussian_renderer/__init__.py:216 passes "
                "it: every render forward and backward then waits on the host for its timing event"}
    out["ms_per_step_with_kernel_events"] = round(ms_instr, 4)
    out["render_fwd_evaluations"] = E
    out["hbm_copy_GBs"] = round(peak_copy, 1)
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


def cpu_baseline_step(scene, cam, frac, cl):
    """The CPU oracle's full fwd+bwd chain on (a sample of) the same scene."""
    from oracle import oracle as O
    P = scene["means3D"].shape[0]
    n = max(1, int(round(P * frac)))
    sub = {k: scene[k][:n] for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    W, H = cam["W"], cam["H"]
    bg = np.zeros(3, np.float32)
    clm = None if cl is None else cl.detach().cpu().numpy().astype(np.uint8)
    dLd = scene.get("dL_dimage")
    if dLd is None:
        dLd = np.random.default_rng(0).standard_normal((3, H, W)).astype(np.float32)

    def once():
        t0 = time.perf_counter()
        pre, bn, rf = O.full_forward(cam, sub, bg=bg, compute_locally=clm)
        rb = O.render_bwd(W, H, bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"],
                          bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd, clm)
        O.preprocess_bwd(cam, sub["means3D"], sub["scales"], sub["rotations"], sub["sh"], pre["radii"],
                         pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic_opacity"], rb["dL_dcolors"])
        return time.perf_counter() - t0

    runs = cpu_runs(once)
    dt = float(np.median(runs))
    log(f"[bench] cpu oracle fwd+bwd on {n} Gaussians: {', '.join(f'{r:.2f}' for r in runs)} s")
    return {"value": round(n / dt, 1), "unit": "Gaussians/s", "cores": O.num_threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"CPU oracle fwd+bwd (fp32 C, OpenMP) on the first {n} of {P} Gaussians, same camera "
                      f"({W}x{H}): 1 warm-up, then the median of {len(runs)} timed runs, {dt * 1e3:.0f} ms "
                      f"(runs {', '.join(f'{r * 1e3:.0f}' for r in runs)} ms)"}


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_runs(once, timed_runs=3):
    """The CPU baseline protocol: one warm-up call of once(), then
    `timed_runs` timed calls; returns their durations (s)."""
    once()
    return [once() for _ in range(timed_runs)]


# ------------------------------------------------------------------- knn

def run_knn(args):
    import torch
    from blitzgs_amd import synth
    from blitzgs_amd.knn import distCUDA2
    t0 = time.time()
    pts_np = synth.config4_points()
    log(f"[bench] config 4 points generated in {time.time() - t0:.1f}s")
    P = pts_np.shape[0]
    pts = torch.as_tensor(pts_np, device="cuda:0")
    ms, kt, _ = timed(lambda: distCUDA2(pts), args.steps, args.warmup)
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    if args.verbose:
        for k, v in sorted(per_kernel.items(), key=lambda x: -x[1]):
            log(f"[bench]   {k:28s} {v:8.4f} ms/call")
    # compulsory traffic 12 P (points) + 4 P (output); the whole pipeline is the unit
    roofline = roofline_of("distCUDA2 (all kernels)", 16 * P, ms)
    roofline["query_kernel_ms"] = round(avg_launch.get("knn_query_kernel", float("nan")), 4)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        n = max(4, int(P * min(args.cpu_sample, 0.1)))
        sub = np.ascontiguousarray(pts_np[:n])

        def once():
            t1 = time.perf_counter()
            O.knn_meandist3(sub)
            return time.perf_counter() - t1
        runs = cpu_runs(once)
        dt = float(np.median(runs))
        cpu = {"value": round(n / dt, 1), "unit": "points/s", "cores": O.num_threads(), "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"CPU oracle exact 3-NN (grid) on the first {n} of the {P} points: 1 warm-up, then the "
                         f"median of {len(runs)} timed runs, {dt * 1e3:.0f} ms"}
    out = header(args, "distCUDA2 points/s (exact 3-NN mean squared distance)", P / (ms * 1e-3), "points/s", ms,
                 "f32", f"config4: distCUDA2 over {P} points", {"points": P})
    out["stages_ms"] = {k: round(v, 4) for k, v in per_kernel.items()}
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


# ------------------------------------------------------------------ ssim

def run_ssim(args):
    import torch
    from blitzgs_amd import synth
    from blitzgs_amd.ssim import fused_ssim
    a, b = synth.config4_images()
    B, C, H, W = a.shape
    img1 = torch.as_tensor(a, device="cuda:0").requires_grad_(True)
    img2 = torch.as_tensor(b, device="cuda:0")

    def step():
        img1.grad = None
        loss = 1.0 - fused_ssim(img1, img2)
        loss.backward()

    ms, kt, _ = timed(step, args.steps, args.warmup)
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    N = B * C * H * W
    fwd_bytes = 2 * 4 * N + 4 * 4 * N
    bwd_bytes = 5 * 4 * N + 4 * N
    rows = {}
    for k, nb in (("ssim_fwd_kernel", fwd_bytes), ("ssim_bwd_kernel", bwd_bytes)):
        t = per_kernel.get(k, 0.0)
        gbs = nb / (t * 1e-3) / 1e9 if t > 0 else 0.0
        rows[k] = {"ms": round(t, 4), "alg_GB": round(nb / 1e9, 4), "GB_per_s": round(gbs, 1),
                   "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    dom = max(rows, key=lambda k: rows[k]["ms"])
    roofline = roofline_of(dom, fwd_bytes if dom == "ssim_fwd_kernel" else bwd_bytes,
                           avg_launch.get(dom, float("nan")))
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        x, y = np.ascontiguousarray(a[:1]), np.ascontiguousarray(b[:1])

        def once():
            t1 = time.perf_counter()
            m, d1, d2, d3 = O.ssim_fwd(x, y)
            O.ssim_bwd(x, y, np.full(x.shape, -1.0 / N, np.float32), d1, d2, d3)
            return time.perf_counter() - t1
        runs = cpu_runs(once)
        dt = float(np.median(runs))
        cpu = {"value": round(x.size / dt, 1), "unit": "pixels/s", "cores": O.num_threads(), "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"CPU oracle SSIM fwd+bwd on image 1 of {B} (3x{H}x{W}): 1 warm-up, then the median of "
                         f"{len(runs)} timed runs, {dt * 1e3:.0f} ms"}
    out = header(args, "fused_ssim fwd+bwd pixels/s", N / (ms * 1e-3), "pixels/s", ms, "f32",
                 f"config4: fused_ssim fwd+bwd, {B}x{C}x{H}x{W}", {"shape": [B, C, H, W]})
    out["stages_ms"] = rows
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


# ------------------------------------------------------------------ adam

ADAM_GROUPS = {"xyz": 3, "f_dc": 3, "f_rest": 45, "opacity": 1, "scaling": 3, "rotation": 4}


def run_adam(args):
    """SparseGaussianAdam.step over config 2's 6M Gaussians (59 floats each, the
    reference's six parameter groups) with 18.8 % of them visible (config 2's
    visible fraction; a seeded random subset)."""
    import torch
    from blitzgs_amd.adam import SparseGaussianAdam
    N = 6_000_000
    rng = np.random.Generator(np.random.PCG64(5))
    vis = torch.as_tensor(rng.random(N) < 0.1877, device="cuda:0")
    params = {k: torch.zeros((N, m), device="cuda:0", requires_grad=True) for k, m in ADAM_GROUPS.items()}
    for k, p in params.items():
        p.grad = torch.randn_like(p)
    opt = SparseGaussianAdam([{"params": [params[k]], "lr": 1e-3, "name": k} for k in ADAM_GROUPS], lr=0.0,
                             eps=1e-15)
    ms, kt, _ = timed(lambda: opt.step(vis, N), args.steps, args.warmup)
    n_vis = int(vis.sum().item())
    floats = sum(ADAM_GROUPS.values())
    alg = n_vis * floats * 28 + N      # read param, grad, m, v and write param, m, v per visible element
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    roofline = roofline_of("adam_kernel", alg, avg_launch.get("adam_kernel", float("nan")))
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        n = 1_000_000
        vis_np = vis[:n].cpu().numpy().astype(np.uint8)
        arrs = {k: [np.zeros((n, m), np.float32) for _ in range(3)] + [rng.normal(0, 1, (n, m)).astype(np.float32)]
                for k, m in ADAM_GROUPS.items()}
        t1 = time.perf_counter()
        for k, (p, m, v, g) in arrs.items():
            O.adam_update(p, g, m, v, vis_np, 1e-3, 0.9, 0.999, 1e-15)
        dt = time.perf_counter() - t1
        cpu = {"value": round(n / dt, 1), "unit": "Gaussians/s", "cores": O.num_threads(), "kind": "port",
               "sample": f"CPU oracle sparse Adam, six groups, first {n} of {N} Gaussians; {dt * 1e3:.0f} ms"}
    out = header(args, "SparseGaussianAdam step Gaussians/s (59 floats per Gaussian)", N / (ms * 1e-3),
                 "Gaussians/s", ms, "f32", f"config2-size optimiser step: {N} Gaussians, {n_vis} visible",
                 {"gaussians": N, "visible": n_vis, "floats_per_gaussian": floats})
    out["stages_ms"] = {k: round(v, 4) for k, v in per_kernel.items()}
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


def run_full(args):
    """The full-image path (GaussianRasterizer.forward, the render_imp / eval
    rasterizer of diff-gaussian-rasterization_f) forward + backward through
    autograd on a scene config (default config 2): preprocess with SH, the
    tile-culled binning, the blend with accum_max_count, then dL/dimage ~ N(0,1)
    through the render and preprocess backward; plus render_simp (the pruning
    steps' importance pass) and render_depth timed separately."""
    import torch
    from blitzgs_amd import synth
    from blitzgs_amd.rasterizer import GaussianRasterizationSettings, GaussianRasterizer
    dev = torch.device("cuda:0")
    gen = {0: synth.config0, 1: synth.config1, 2: synth.config2, 3: synth.config3}[args.config]
    scene, cam = gen()
    P = scene["means3D"].shape[0]
    W, H = cam["W"], cam["H"]
    tt = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)
    sh = np.asarray(scene["sh"], np.float32)
    params = {"means3D": tt(scene["means3D"]), "scales": tt(scene["scales"]), "rotations": tt(scene["rotations"]),
              "opacities": tt(scene["opacities"]), "dc": tt(sh[:, :1]), "rest": tt(sh[:, 1:])}
    for v in params.values():
        v.requires_grad_(True)
    means2D = torch.zeros((P, 3), device=dev, requires_grad=True)
    culling = torch.zeros(P, dtype=torch.bool, device=dev)
    dL = tt(scene.get("dL_dimage", np.random.default_rng(0).standard_normal((3, H, W)).astype(np.float32)))
    rs = GaussianRasterizationSettings(
        image_height=H, image_width=W, tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
        bg=torch.zeros(3, device=dev), scale_modifier=1.0, viewmatrix=tt(cam["viewmatrix"]),
        projmatrix=tt(cam["projmatrix"]), sh_degree=3, campos=tt(cam["campos"]), prefiltered=False, debug=False)
    ras = GaussianRasterizer(rs)
    info = {}

    def step():
        for v in list(params.values()) + [means2D]:
            v.grad = None
        color, radii, amc = ras(means3D=params["means3D"], means2D=means2D, opacities=params["opacities"],
                                culling=culling, dc=params["dc"], shs=params["rest"], scales=params["scales"],
                                rotations=params["rotations"], flag_max_count=True)
        torch.autograd.backward([color], [dL])
        info["radii"] = radii

    ms, kt, _ = timed(step, args.steps, args.warmup)

    def simp():
        with torch.no_grad():
            ras.render_simp(means3D=params["means3D"], means2D=means2D, opacities=params["opacities"],
                            culling=culling, dc=params["dc"], shs=params["rest"], scales=params["scales"],
                            rotations=params["rotations"])

    ms_simp, kt_simp, _ = timed(simp, args.steps, args.warmup)

    def depth():
        ras.render_depth(means3D=params["means3D"], means2D=means2D, opacities=params["opacities"],
                         culling=culling, dc=params["dc"], shs=params["rest"], scales=params["scales"],
                         rotations=params["rotations"])

    ms_depth, kt_depth, _ = timed(depth, args.steps, args.warmup)
    P_vis = int((info["radii"] > 0).sum().item())
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    # instances after the tile test, from one direct forward (outside the timed regions)
    from blitzgs_amd import fullpath
    x = fullpath._inputs(rs, params["means3D"].detach(), params["dc"].detach(), params["rest"].detach(), None,
                         params["opacities"].detach(), params["scales"].detach(), params["rotations"].detach(), None)
    R = fullpath._forward(rs, x, culling, True, False)[-1]
    sb = stage_bytes(P, P_vis, R, W * H)
    sb["preprocess_fwd_full_kernel"] = sb["preprocess_fwd_kernel"]
    # the full-image path clears no dL/dsh in the render backward: its preprocess backward writes the SH
    # gradients of every Gaussian (zeros for the invisible ones)
    sb["preprocess_bwd_full_kernel"] = sb["preprocess_bwd_kernel"] + 192 * (P - P_vis)
    sb["render_bwd_kernel"] -= 192 * P
    dom = max((k for k in sb if k in per_kernel), key=lambda k: per_kernel[k])
    roofline = roofline_of(dom, sb[dom], avg_launch[dom])
    roofline["note"] = ("the blend kernels are VALU-bound (per-pixel exp and gradient arithmetic plus a 64-lane "
                        "reduction per Gaussian); their HBM fraction is low by nature")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        n = max(1, int(round(P * args.cpu_sample)))
        sub = {k: scene[k][:n] for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
        t1 = time.perf_counter()
        pre, bn, rf = O.full_path_forward(cam, sub)
        rb = O.render_bwd_full(W, H, np.zeros(3, np.float32), pre["means2D"], pre["conic_opacity"], pre["rgb"],
                               bn["ranges"], bn["point_list"], rf["final_T"], rf["n_contrib_px"], np.asarray(
                                   scene.get("dL_dimage", np.zeros((3, H, W), np.float32)), np.float32))
        shn = np.asarray(sub["sh"], np.float32)
        O.preprocess_bwd_full(cam, sub["means3D"], sub["scales"], sub["rotations"], shn[:, :1], shn[:, 1:],
                              pre["radii"], pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic"],
                              rb["dL_dcolors"])
        dt = time.perf_counter() - t1
        cpu = {"value": round(n / dt, 1), "unit": "Gaussians/s", "cores": O.num_threads(), "kind": "port",
               "sample": f"one full-path fwd+bwd of the CPU oracle on the first {n} of {P} Gaussians; "
                         f"{dt * 1e3:.0f} ms"}
    out = header(args, f"full-image path (GaussianRasterizer.forward) fwd+bwd Gaussians/s, config {args.config}",
                 P / (ms * 1e-3), "Gaussians/s", ms, "f32",
                 f"config{args.config} full-image path: {P} Gaussians SH3, {W}x{H}, fwd+bwd",
                 {"gaussians": P, "visible": P_vis, "image": [W, H]})
    out["stages_ms"] = {k: round(v, 4) for k, v in per_kernel.items()}
    out["render_simp_ms"] = round(ms_simp, 4)
    out["render_simp_stages_ms"] = {k: round(v[0] / max(1, args.steps), 4) for k, v in kt_simp.items()}
    out["render_depth_ms"] = round(ms_depth, 4)
    out["render_depth_stages_ms"] = {k: round(v[0] / max(1, args.steps), 4) for k, v in kt_depth.items()}
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    out["config"]["instances"] = R
    print(json.dumps(out), flush=True)


def run_route(args):
    """One rank's side of the screen-space exchange at config 3's shape: config
    3's 8M Gaussians (4096x2730) preprocessed once, then per step routed to
    the four tile-row ranks of the image (rows [0, 43), [43, 86), [86, 129),
    [129, 171): division_pos * TILE_X), every rank's send ids from one count
    and one write pass, the send rows of all four ranks packed (means2D 2, rgb
    3, conic_opacity 4, radii 1, depth 1, means3D 3, scales 3, rotation 4 =
    21 values per row) and one received buffer of rank 1's size unpacked into
    contiguous fields."""
    import torch
    from blitzgs_amd import rasterizer, routing, synth
    scene, cam = synth.config3()
    dev = torch.device("cuda:0")
    tt = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)
    rs = rasterizer.GaussianRasterizationSettings(
        image_height=int(cam["H"]), image_width=int(cam["W"]), tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
        bg=torch.zeros(3, device=dev), scale_modifier=1.0, viewmatrix=tt(cam["viewmatrix"]),
        projmatrix=tt(cam["projmatrix"]), sh_degree=3, campos=tt(cam["campos"]), prefiltered=False, debug=False)
    r = rasterizer._preprocess_forward_raw(tt(scene["means3D"]), tt(scene["scales"]), tt(scene["rotations"]),
                                           tt(scene["sh"]), tt(scene["opacities"]), rs)
    _, m2d, depths, radii, _, con, rgb, _ = r
    m3d, sc, rot = tt(scene["means3D"]), tt(scene["scales"]), tt(scene["rotations"])
    del scene["sh"]
    H, W = int(cam["H"]), int(cam["W"])
    gx, gy = (W + 15) // 16, (H + 15) // 16
    rows = [0, 43, 86, 129, gy]
    st = torch.tensor([v * gx for v in rows], dtype=torch.int32, device=dev)
    P = int(m2d.size(0))
    fields = [m2d, rgb, con, radii, depths, m3d, sc, rot]
    widths = [2, 3, 4, 1, 1, 3, 3, 4]
    types = [torch.float32] * 3 + [torch.int32] + [torch.float32] * 4
    info = {}

    def step():
        ids, cnt, _ = routing.local2j_ids_concat(m2d, radii, H, W, st, 4)
        buf = routing.pack_rows(ids, fields)
        s1 = cnt[0]
        routing.unpack_rows(buf[s1:s1 + cnt[1]], widths, types)
        info["cnt"] = cnt

    ms, kt, _ = timed(step, args.steps, args.warmup)
    cnt = info["cnt"]
    n_send = sum(cnt)
    row_bytes = 4 * sum(widths)
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    # algorithmic bytes: pack reads an id and a row and writes a row per sent
    # row; unpack reads and writes a row per received row
    pack_b = n_send * (8 + 2 * row_bytes)
    unpack_b = cnt[1] * 2 * row_bytes
    tot_ms, launches = kt.get("move_rows_kernel", (float("nan"), 1))
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_route_config3.json")
    if os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get("move_rows_kernel")
        except (OSError, ValueError):
            traffic = None
    roofline = roofline_of("move_rows_kernel", (pack_b + unpack_b) / 2, tot_ms / max(1, launches), traffic)
    roofline["note"] = ("two launches per step (pack of every send row, unpack of one rank's rows); achieved = "
                        "their algorithmic bytes over their time, per launch on average.  The pack gathers sparse "
                        "rows (20% of 8M) once per destination rank, so its HBM traffic is several times the "
                        "algorithmic bytes (traffic)")
    route_b = P * 12 * 2 + n_send * 8   # means2D + radii read by count and write passes; ids written
    rt_ms = sum(kt.get(k, (0.0, 1))[0] for k in ("route_count_kernel", "route_scan_kernel", "route_write_kernel"))
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        hm, hr = m2d.cpu().numpy(), radii.cpu().numpy()
        hf = [f.cpu().numpy().reshape(P, -1) for f in fields]
        t1 = time.perf_counter()
        b = O.local2j_ids_bool(H, W, hm, hr, st.cpu().numpy())
        hids = np.concatenate([np.flatnonzero(b[:, k]) for k in range(4)])
        hbuf = np.concatenate([f[hids].astype(np.float32) for f in hf], axis=1)
        dt = time.perf_counter() - t1
        assert hbuf.shape == (n_send, sum(widths))
        cpu = {"value": round(P / dt, 1), "unit": "Gaussians/s", "cores": O.num_threads(), "kind": "port",
               "sample": f"CPU oracle routing of all {P} Gaussians + numpy nonzero and row gather of the send "
                         f"rows (no unpack); {dt * 1e3:.0f} ms"}
    out = header(args, "exchange-side routing + pack/unpack Gaussians/s (one rank, 4 tile-row ranks)",
                 P / (ms * 1e-3), "Gaussians/s", ms, "f32/int32",
                 f"config3-shape routing: {P} Gaussians, 4096x2730, 4 ranks by tile rows",
                 {"gaussians": P, "ranks": 4, "rows_sent": n_send, "rows_per_rank": cnt,
                  "values_per_row": sum(widths)})
    out["stages_ms"] = {k: round(v, 4) for k, v in per_kernel.items()}
    out["routing_GBs"] = round(route_b / (rt_ms / max(1, args.steps) * 1e-3) / 1e9, 1) if rt_ms else None
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


def _ply_file_round_trip(plyio, t_, dev):
    import tempfile
    import torch
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "point_cloud.ply")
        t0 = time.perf_counter()
        plyio.save_ply(path, *t_)
        t1 = time.perf_counter()
        got = plyio.load_ply(path, 3, device=dev)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        ok = all(bool(torch.equal(a, b)) for a, b in zip(got[:6], t_))
        size = os.path.getsize(path)
        file_e2e = {"save_s": round(t1 - t0, 3), "load_s": round(t2 - t1, 3), "file_bytes": size,
                    "save_GBs": round(size / (t1 - t0) / 1e9, 2), "load_GBs": round(size / (t2 - t1) / 1e9, 2),
                    "round_trip_exact": ok}
        del got
    return file_e2e


def run_ply(args):
    """The trained-scene PLY layer at config 2's size (6M SH-3 Gaussians, 62
    float32 properties per vertex record): one step = gs_ply_unpack of the
    records resident in HBM into the six parameter tensors (load_ply's device
    part) + gs_ply_pack of the tensors back into records (save_ply's device
    part).  Outside the timed region one save_ply + load_ply through a file
    under the temp directory is timed end to end (file system and PCIe
    included)."""
    import tempfile
    import torch
    from blitzgs_amd import plyio
    P, n = 6_000_000, 62
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2)
    rec = torch.randn((P, n), device=dev, generator=g)
    names = plyio.construct_list_of_attributes(torch.empty(0, 1, 3), torch.empty(0, 15, 3), torch.empty(0, 3),
                                               torch.empty(0, 4))
    idx = {nm: i for i, nm in enumerate(names)}
    cm = [[0, 1, 2], [6, 7, 8], [idx["f_rest_{}".format(c * 15 + k)] for k in range(15) for c in range(3)], [54],
          [55, 56, 57], [58, 59, 60, 61]]
    shapes = [(3,), (1, 3), (15, 3), (1,), (3,), (4,)]
    state = {}

    def step():
        t = plyio.unpack_records(rec, cm, shapes)
        state["rec"], _ = plyio.pack_records(*t)

    ms, kt, _ = timed(step, args.steps, args.warmup)
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    # algorithmic bytes per launch: all 62 record columns one way, the 59
    # parameter columns (no normals) the other way
    alg = P * (n + 59) * 4
    dom = max(("ply_unpack_kernel", "ply_pack_kernel"), key=lambda k: avg_launch.get(k, 0.0))
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_ply_config2.json")
    if os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get(dom)
        except (OSError, ValueError):
            traffic = None
    roofline = roofline_of(dom, alg, avg_launch.get(dom, float("nan")), traffic)
    roofline["note"] = "per launch: {} B read + {} B written ({} Gaussians)".format(
        *((P * n * 4, P * 59 * 4) if dom == "ply_unpack_kernel" else (P * 59 * 4, P * n * 4)), P)
    t_ = plyio.unpack_records(rec, cm, shapes)
    torch.cuda.synchronize()
    file_e2e = {}
    try:
        file_e2e = _ply_file_round_trip(plyio, t_, dev)
    except OSError as e:      # no room for the 1.5 GB file: report, keep the kernel line
        file_e2e = {"error": str(e)}
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import o_ply
        m = 1_000_000
        h = [a[:m].cpu().numpy() for a in t_]
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "cpu.ply")
            t0 = time.perf_counter()
            o_ply.save_ply(path, *h)
            o_ply.load_ply(path, 3)
            dt = time.perf_counter() - t0
        cpu = {"value": round(m / dt, 1), "unit": "Gaussians/s", "cores": 1, "kind": "port",
               "sample": "numpy restatement of the reference's save_ply + load_ply (file I/O included) on the "
                         "first {} of {} Gaussians; {:.0f} ms; compare with file_e2e".format(m, P, dt * 1e3)}
    out = header(args, "PLY record <-> parameter tensors Gaussians/s (unpack + pack, 6M SH3 in HBM)",
                 P / (ms * 1e-3), "Gaussians/s", ms, "f32",
                 "config2-size PLY layer: {} Gaussians x {} properties".format(P, n),
                 {"gaussians": P, "properties": n})
    out["stages_ms"] = {k: round(v, 4) for k, v in per_kernel.items()}
    out["file_e2e"] = file_e2e
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


# ------------------------------------------------------------------ render_geo

def run_geo(args):
    """render_geo's forward (the _r render's five geometry maps and plane
    depth) at a config's size: the colour-only render forward, the fused
    forward (maps in the colour's walk of the lists) and the colour forward
    followed by a second walk for the maps, each from the preprocess outputs
    (binning included)."""
    import torch
    from blitzgs_amd import rasterizer as R
    from blitzgs_amd import synth
    gen = {0: synth.config0, 1: synth.config1, 2: synth.config2, 3: synth.config3}[args.config]
    scene, cam = gen()
    P = scene["means3D"].shape[0]
    W, H = cam["W"], cam["H"]
    dev = torch.device("cuda:0")
    tt = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)
    rs = R.GaussianRasterizationSettings(
        image_height=H, image_width=W, tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"], bg=torch.zeros(3, device=dev),
        scale_modifier=1.0, viewmatrix=tt(cam["viewmatrix"]), projmatrix=tt(cam["projmatrix"]), sh_degree=3,
        campos=tt(cam["campos"]), prefiltered=False, debug=False)
    pre = R._preprocess_forward_raw(tt(scene["means3D"]), tt(scene["scales"]), tt(scene["rotations"]),
                                    tt(scene["sh"]), tt(scene["opacities"]), rs)
    _, means2D, depths, radii, _, conic_opacity, rgb, _ = pre
    rng = np.random.default_rng(7)
    all_map = rng.uniform(-1.0, 1.0, (P, 5)).astype(np.float32)
    all_map[:, 2] = rng.uniform(-1.5, -0.5, P)
    amap = tt(all_map)
    cl = tt(scene["compute_locally"]).bool() if "compute_locally" in scene else None
    args_fwd = (rs.bg, H, W, means2D, depths, radii, conic_opacity, rgb, cl)
    geo = (cam["tanfovx"], cam["tanfovy"], amap)

    def two_walks():
        out = R._render_forward_raw(*args_fwd)
        R._render_geo_forward_raw(P, H, W, cam["tanfovx"], cam["tanfovy"], amap, cl, out[0], out[6], out[7], out[8])

    res = {}
    for name, fn in (("colour_only", lambda: R._render_forward_raw(*args_fwd)),
                     ("fused", lambda: R._render_forward_raw(*args_fwd, geo=geo)),
                     ("two_walks", two_walks)):
        ms, kt, _ = timed(fn, args.steps, args.warmup)
        per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
        res[name] = {"ms_per_forward": round(ms, 4),
                     "blend_kernels_ms": {k: round(v, 4) for k, v in per_kernel.items()
                                          if k in ("render_fwd_kernel", "render_fwd_geo_kernel", "render_geo_kernel")}}
        log(f"[bench] render_geo {name}: {ms:.3f} ms per forward")
    out = header(args, f"render_geo forward ms (colour + 5 maps + plane depth), config {args.config}",
                 1e3 / res["fused"]["ms_per_forward"], "forwards/s", res["fused"]["ms_per_forward"], "f32",
                 f"config{args.config}: {P} Gaussians, {W}x{H}, render forward with render_geo",
                 {"gaussians": P, "image": [W, H]})
    out["higher_is_better"] = True
    out["variants"] = res
    out["roofline"] = None
    out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path shards by "
              "Gaussians for preprocess and by tile rows for render, with an all-to-all between them, which is "
              "not built here", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.valu_probes:
        valu_probes_only()
        return
    import torch
    from blitzgs_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    {"step": run_step, "knn": run_knn, "ssim": run_ssim, "adam": run_adam, "route": run_route,
     "full": run_full, "ply": run_ply, "geo": run_geo}[args.workload](args)


if __name__ == "__main__":
    main()
