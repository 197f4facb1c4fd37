"""Parity at BASELINE.json's full sizes, through properties that do not depend
on size or against the oracle where it finishes in seconds:

* config 1 (1M Gaussians, 1920x1080): the whole forward against the CPU
  oracle -- preprocess and binning bit-exact, the blend within 1e-4 max-abs;
* config 3 (8M Gaussians, 4096x2730, tile rows [43, 86) local): the rank's
  share against the full-image render of the same scene on the GPU -- ranges
  are the full ranges shifted by a constant, the local pixel rows are
  bit-identical, every other tile is empty;
* config 4: distCUDA2 over all 10M points, checked bit for bit at 2048 sampled
  points against a brute force over all points (torch, the reference's
  distance expression with separately rounded operations) and at every point
  against the CPU oracle; fused_ssim on the 8 x 3 x 1080 x 1920 pair (map, the
  three partial derivatives and the backward) against the oracle on two of
  the images.
"""
import numpy as np
import pytest
import torch

from blitzgs_amd import synth
from oracle import oracle as O
from tests.gpu_helpers import (assert_blend_counts, assert_close_abs, gpu_preprocess, gpu_render_forward, np_,
                               settings_for, to_dev)

pytestmark = pytest.mark.gpu


def _bitexact(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, what
    if a.dtype.kind == "f":
        a, b = a.view(np.uint32), b.view(np.uint32)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}"


def test_config1_forward_vs_oracle(gpu):
    scene, cam = synth.config1()
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    pre, bn, rf = O.full_forward(cam, scene, bg=np.zeros(3, np.float32))
    for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]:
        _bitexact(np_(g[k]), pre[k], k)
    out = gpu_render_forward(rs, g["means2D"], g["depths"], g["radii"], g["conic_opacity"], g["rgb"])
    assert out["R"] == bn["R"]
    _bitexact(np_(out["point_list"]).view(np.uint32), bn["point_list"], "point_list")
    _bitexact(np_(out["ranges"]).view(np.uint32), bn["ranges"], "ranges")
    assert_close_abs(np_(out["color"]), rf["color"], "color")
    assert_close_abs(np_(out["final_T"]), rf["final_T"], "final_T")
    assert_blend_counts(dict(n_contrib_px=np_(out["n_contrib_px"]).view(np.uint32),
                             n_contrib2loss_px=np_(out["n_contrib2loss_px"]).view(np.uint32),
                             out_observe=np_(out["out_observe"]), n_consider=np_(out["n_consider"]),
                             n_contrib=np_(out["n_contrib"])), rf, "config 1 forward")


def test_config3_share_matches_full_image(gpu):
    scene, cam = synth.config3()
    cl = scene["compute_locally"]
    gy, gx = cl.shape
    rows = np.flatnonzero(cl.any(axis=1))
    lo, hi = int(rows[0]), int(rows[-1]) + 1
    assert (lo, hi) == (43, 86)
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    args = (g["means2D"], g["depths"], g["radii"], g["conic_opacity"], g["rgb"])
    full = gpu_render_forward(rs, *args)
    sub = gpu_render_forward(rs, *args, compute_locally=cl)
    fr, sr = np_(full["ranges"]).astype(np.int64), np_(sub["ranges"]).astype(np.int64)
    t0, t1 = lo * gx, hi * gx
    nonempty = fr[t0:t1, 1] > fr[t0:t1, 0]
    assert nonempty.any()
    off = int(fr[t0:t1][nonempty][0, 0])                  # the share's list starts at 0
    assert sub["R"] == int((fr[t0:t1, 1] - fr[t0:t1, 0]).sum())
    assert (sr[t0:t1][nonempty] == fr[t0:t1][nonempty] - off).all()
    assert not sr[t0:t1][~nonempty].any()
    assert not sr[:t0].any() and not sr[t1:].any()
    # the instances of the local tiles are the same, in the same order
    fpl, spl = np_(full["point_list"]), np_(sub["point_list"])
    _bitexact(spl[:sub["R"]], fpl[off:off + sub["R"]], "point_list of the local rows")
    fc, sc = np_(full["color"]), np_(sub["color"])
    py0, py1 = lo * 16, min(hi * 16, cam["H"])
    _bitexact(sc[:, py0:py1], fc[:, py0:py1], "local rows of the image")
    assert not sc[:, :py0].any() and not sc[:, py1:].any()


def test_config4_knn_10m_sampled_bruteforce(gpu):
    from blitzgs_amd.knn import distCUDA2
    pts = synth.config4_points()
    P = pts.shape[0]
    dev = to_dev(pts)
    out = np_(distCUDA2(dev))
    rng = np.random.default_rng(4)
    idx = np.sort(rng.choice(P, 2048, replace=False))
    x, y, z = dev[:, 0], dev[:, 1], dev[:, 2]
    ref = np.empty(len(idx), np.float32)
    for b0 in range(0, len(idx), 32):
        q = torch.as_tensor(idx[b0:b0 + 32], device="cuda")
        dx = x[None, :] - x[q][:, None]
        dy = y[None, :] - y[q][:, None]
        dz = z[None, :] - z[q][:, None]
        d = (dx * dx + dy * dy) + dz * dz          # separately rounded, as in the reference
        d[torch.arange(len(q), device="cuda"), q] = float("inf")   # self excluded by index
        best = np_(torch.topk(d, 3, dim=1, largest=False).values)  # ascending
        # final sum and division in numpy float32: torch divides by a Python
        # scalar as a multiplication by its reciprocal, which is not the
        # reference's IEEE division
        ref[b0:b0 + 32] = ((best[:, 0] + best[:, 1]) + best[:, 2]) / np.float32(3.0)
        del dx, dy, dz, d
    _bitexact(out[idx], ref, "distCUDA2 at sampled points")


def test_config4_knn_10m_vs_oracle(gpu):
    # every one of the 10M outputs against the CPU oracle (exact 3-NN, the
    # reference's distance expression): bit-exact
    from blitzgs_amd.knn import distCUDA2
    pts = synth.config4_points()
    out = np_(distCUDA2(to_dev(pts)))
    _bitexact(out, O.knn_meandist3(pts), "distCUDA2 over all 10M points")


def test_config4_ssim_batch_vs_oracle(gpu):
    from blitzgs_amd.ssim import fusedssim, fusedssim_backward
    a, b = synth.config4_images()
    C1, C2 = 0.01 ** 2, 0.03 ** 2
    da, db = to_dev(a), to_dev(b)
    m, d1, d2, d3 = fusedssim(C1, C2, da, db, True)
    dL = np.random.default_rng(44).standard_normal(a.shape).astype(np.float32)
    g = fusedssim_backward(C1, C2, da, db, to_dev(dL), d1, d2, d3)
    for i in (0, 7):
        om, od1, od2, od3 = O.ssim_fwd(a[i:i + 1], b[i:i + 1])
        _bitexact(np_(m[i:i + 1]), om, f"ssim map image {i}")
        _bitexact(np_(d1[i:i + 1]), od1, f"dm_dmu1 image {i}")
        _bitexact(np_(d2[i:i + 1]), od2, f"dm_dsigma1_sq image {i}")
        _bitexact(np_(d3[i:i + 1]), od3, f"dm_dsigma12 image {i}")
        og = O.ssim_bwd(a[i:i + 1], b[i:i + 1], dL[i:i + 1], od1, od2, od3)
        _bitexact(np_(g[i:i + 1]), og, f"dL_dimg1 image {i}")
