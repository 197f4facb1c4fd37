"""Benchmark of the rasterizer hot path on one MI355X.

One step = one training forward+backward of the reference's split rasterizer
path on config 2 of BASELINE.json (6,000,000 SH-degree-3 Gaussians, city-scale
aerial scene, 1600x1066 camera): preprocess forward -> binning + render forward
-> render backward (dL/dimage ~ N(0,1)) -> preprocess backward, driven through
the drop-in autograd API exactly as gaussian_renderer does.  Inputs are
generated once (seeded, synthetic) and stay resident in HBM.

Prints ONE JSON line (rank 0).  `value` is Gaussians/s = P / step time.
`roofline` describes the dominant kernel, timed live with HIP events inside the
timed region; `cpu_baseline` times the CPU oracle (oracle/, fp32 C with OpenMP)
on a bounded sample of the same workload on this host.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

# algorithmic bytes per unit of work, per stage
def stage_bytes(P, P_vis, R, npx, T):
    return {
        "preprocess_fwd_kernel": 115 * P + 192 * P_vis,
        "preprocess_bwd_kernel": 240 * P + 295 * P_vis,
        "binning": 16 * P + 44 * R,
        "render_fwd_kernel": 40 * R + 24 * npx,
        "render_bwd_kernel": 40 * R + 32 * npx,
        # out_observe clear (4P) and the gradient unpack (1P flag + 48 P_vis read + 48 P_vis clear + 48 P written)
        "other": 4 * P + P + 96 * P_vis + 48 * P,
    }


BINNING_KERNELS = ("localmap_kernel", "count_kernel", "tilescan_kernel", "ranges_kernel", "scatter_kernel",
                   "tilesort_kernel_s", "tilesort_kernel_m", "tilesort_kernel_l", "tilesort_big_kernel")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=[0, 1, 2, 3])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=float, default=1.0,
                    help="fraction of the Gaussians the CPU baseline runs on")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run the library's plain copy kernel on MIB MiB (5 launches): the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE, then exit")
    return ap.parse_args()


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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding of this path is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    import torch
    from blitzgs_amd import _lib, synth
    from blitzgs_amd.rasterizer import GaussianRasterizationSettings, GaussianRasterizer

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda:0")

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
    cuda_args = {"avoid_pixel_all2all": False}
    info = {}

    def step():
        for p in params.values():
            p.grad = None
        means2D_abs.grad = None
        means2D, rgb, conic_opacity, radii, depths = ras.preprocess_gaussians(
            params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], cuda_args)
        color, n_render, n_consider, n_contrib, out_observe, _, _ = ras.render_gaussians(
            means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, cl, cl, cuda_args)
        torch.autograd.backward([color], [dL_dimage])
        info["radii"] = radii
        info["n_render"] = n_render

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    P_vis = int((info["radii"] > 0).sum().item())
    R = int(info["n_render"].sum().item())

    # timed region: K steps bracketed by synchronisation; per-kernel HIP events on
    # the launch stream accumulate each kernel's launch durations
    _lib.timing_reset()
    _lib.timing_enable(True)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    _lib.timing_enable(False)
    kt = _lib.timing_read()
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step (wall {1e3 * wall / args.steps:.3f} ms)")

    # per-stage durations (ms per step) and algorithmic bandwidth
    per_kernel = {k: v[0] / max(1, args.steps) for k, v in kt.items()}
    avg_launch = {k: v[0] / max(1, v[1]) for k, v in kt.items()}
    stages = {k: per_kernel.get(k, 0.0) for k in ("preprocess_fwd_kernel", "render_fwd_kernel",
                                                  "render_bwd_kernel", "preprocess_bwd_kernel")}
    stages["binning"] = sum(per_kernel.get(k, 0.0) for k in BINNING_KERNELS)
    stages["other"] = sum(v for k, v in per_kernel.items() if k not in stages and k not in BINNING_KERNELS)
    sb = stage_bytes(P, P_vis, R, W * H, T)
    stage_rows = {}
    for k, ms in stages.items():
        gbs = sb[k] / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        stage_rows[k] = {"ms": round(ms, 4), "alg_GB": round(sb[k] / 1e9, 4), "GB_per_s": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if args.verbose:
        for k, v in sorted(per_kernel.items(), key=lambda x: -x[1]):
            log(f"[bench]   {k:28s} {v:8.4f} ms/step  ({kt[k][1] // max(1, args.steps)} launches)")
    dom = max(("preprocess_fwd_kernel", "render_fwd_kernel", "render_bwd_kernel", "preprocess_bwd_kernel"),
              key=lambda k: per_kernel.get(k, 0.0))
    dom_ms = avg_launch.get(dom, float("nan"))
    dom_bytes = sb[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "avg_launch_ms": round(dom_ms, 4), "alg_bytes_per_launch": int(dom_bytes)}
    traffic = os.path.join(ROOT, "profiles", "traffic_config2.json")
    if os.path.exists(traffic):
        try:
            roofline["traffic"] = json.load(open(traffic)).get(dom)
        except Exception:
            pass

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(scene, cam, args.cpu_sample, cl)

    gs_per_s = P / (ms_per_step * 1e-3)
    out = {
        "metric": "rasterizer fwd+bwd ms/iter & Gaussians/s at 6M SH3 1600x1066; % HBM roofline",
        "value": round(gs_per_s, 1), "unit": "Gaussians/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded PCG64 scene)",
        "config": {"workload": f"config{args.config}: {P} Gaussians SH3, {W}x{H}, fwd+bwd", "gaussians": P,
                   "visible": P_vis, "instances": R, "image": [W, H], "tiles": T, "parallelism": "single-gpu"},
        "stages_ms": stage_rows,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def cpu_baseline(scene, cam, frac, cl):
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
    t0 = time.perf_counter()
    pre, bn, rf = O.full_forward(cam, sub, bg=bg, compute_locally=clm)
    rb = O.render_bwd(W, H, bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"], bn["point_list"],
                      rf["final_T"], rf["n_contrib_px"], dLd, clm)
    O.preprocess_bwd(cam, sub["means3D"], sub["scales"], sub["rotations"], sub["sh"], pre["radii"], pre["cov3D"],
                     pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic_opacity"], rb["dL_dcolors"])
    dt = time.perf_counter() - t0
    log(f"[bench] cpu oracle fwd+bwd on {n} Gaussians: {dt:.2f}s")
    return {"value": round(n / dt, 1), "unit": "Gaussians/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"one fwd+bwd iteration of the CPU oracle on the first {n} of {P} Gaussians, "
                      f"same camera ({W}x{H}); {dt * 1e3:.0f} ms"}


if __name__ == "__main__":
    main()
