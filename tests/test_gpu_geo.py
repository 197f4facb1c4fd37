"""render_geo of the split render (the _r rasterizer's five geometry maps and
plane depth, _r/cuda_rasterizer/forward.cu:381-384,407-412, backward.cu:393-405,
427-432,476-490) on the GPU against the oracle.

Bar: out_all_map within the image's 1e-4 max-abs (the maps take the colour's
blend weights, and the blend evaluates exp with the hardware exp2 away from
the alpha cut-off); out_plane_depth within that bound carried through its
formula; every gradient, dL/dall_map included, within 1e-3 relative L2;
through the C ABI (unmasked and with a compute_locally mask), the autograd
operator with a loss on all three outputs, and the drop-in's raw _C ops.  The
operators render the maps in the colour's own walk of the lists (the fused
forward); it is checked bit for bit against the plain forward (every colour
output) followed by the second walk (gs_render_geo_forward: the maps)."""
import os
import sys
import importlib

import numpy as np
import pytest
import torch

from blitzgs_amd import rasterizer, synth
from oracle import oracle as O
from tests.gpu_helpers import (BLEND_ATOL, assert_bitexact, assert_close_abs, buffer_views, gpu_render_forward, np_,
                               rel_l2, settings_for, to_dev)

pytestmark = pytest.mark.gpu

DROPIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "blitzgs_amd", "dropin")
GRADS = ["dL_dmeans2D", "dL_dmeans2D_abs", "dL_dconic_opacity", "dL_dcolors", "dL_dall_map"]


def _case(seed, masked, P=4000, W=203, H=147):
    scene, cam = synth.small_scene(P, seed=seed, W=W, H=H, extent=1.3, log_mu=-2.3)
    pre = O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                           scene["opacities"])
    gx, gy = O.tile_grid(W, H)
    rng = np.random.default_rng(seed)
    cl = (rng.random((gy, gx)) < 0.6).astype(np.uint8) if masked else np.ones((gy, gx), np.uint8)
    all_map = rng.uniform(-1.0, 1.0, (P, 5)).astype(np.float32)
    all_map[:, 2] = rng.uniform(-1.5, -0.5, P)   # the blended n . ray stays away from 0
    grads = dict(dpix=rng.normal(size=(3, H, W)).astype(np.float32),
                 dmaps=rng.normal(size=(5, H, W)).astype(np.float32),
                 dplane=(0.1 * rng.normal(size=(1, H, W))).astype(np.float32))
    return scene, cam, pre, cl, all_map, grads


def assert_plane_depth_close(got, ref, ref_maps, cam, name):
    """D = M4 / -(M0 rx + M1 ry + M2 + 1e-8): an error of at most BLEND_ATOL in
    each map moves D by at most BLEND_ATOL (1 + |rx| + |ry|)(1/|s| + |M4|/s^2)
    to first order (s the dot product); pixels with no contribution give 0
    (-0 on local tiles, as 0 / -(0 + 1e-8))."""
    W, H = cam["W"], cam["H"]
    fx, fy = (float(v) for v in O.focal(W, H, cam["tanfovx"], cam["tanfovy"]))
    y, x = np.mgrid[0:H, 0:W].astype(np.float64)
    rx, ry = (x - 0.5 * W) / fx, (y - 0.5 * H) / fy
    M = ref_maps.astype(np.float64)
    s = M[0] * rx + M[1] * ry + M[2]
    g, r = got.reshape(H, W).astype(np.float64), ref.reshape(H, W).astype(np.float64)
    empty = ~M.any(axis=0)
    assert (g[empty] == 0).all() and (np.signbit(g) == np.signbit(r))[empty].all(), name
    ok = ~empty & (np.abs(s) > 1e-3)
    assert ok.sum() > 0.5 * (~empty).sum(), name
    so = s[ok]
    bound = 2 * BLEND_ATOL * (1 + np.abs(rx[ok]) + np.abs(ry[ok])) * (1 / np.abs(so) + np.abs(M[4][ok]) / so ** 2)
    bad = np.flatnonzero(np.abs(g - r)[ok] > bound)
    assert bad.size == 0, (name, bad.size, float(np.abs(g - r)[ok].max()))


def _oracle(cam, pre, cl, all_map, bg, grads, cl_bwd=None):
    """Forward (binning, colour, maps) over the tiles of cl; backward over
    those of cl_bwd (default cl), as avoid_pixel_all2all splits them."""
    W, H = cam["W"], cam["H"]
    cl_bwd = cl if cl_bwd is None else cl_bwd
    bn = O.binning(W, H, pre["means2D"], pre["depths"], pre["radii"], cl)
    rf = O.render_fwd(W, H, bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"], bn["point_list"], cl)
    geo = O.render_geo_fwd(W, H, cam["tanfovx"], cam["tanfovy"], pre["means2D"], pre["conic_opacity"], all_map,
                           bn["ranges"], bn["point_list"], cl)
    rb = O.render_bwd_geo(W, H, cam["tanfovx"], cam["tanfovy"], bg, pre["means2D"], pre["conic_opacity"], pre["rgb"],
                          all_map, geo["out_all_map"], bn["ranges"], bn["point_list"], rf["final_T"],
                          rf["n_contrib_px"], grads["dpix"], grads["dmaps"], grads["dplane"], cl_bwd)
    return bn, rf, geo, rb


@pytest.mark.parametrize("masked", [False, True])
def test_geo_forward_within_tolerance_and_backward_vs_oracle(gpu, masked):
    scene, cam, pre, cl, all_map, grads = _case(17 + masked, masked)
    bg = np.array([0.2, 0.5, 0.1], np.float32)
    W, H = cam["W"], cam["H"]
    P = len(all_map)
    print(f"render_geo C ABI: P={P} W={W} H={H} masked={masked}", flush=True)
    rs = settings_for(cam, bg=bg)
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    f = gpu_render_forward(rs, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], cl)
    amap = to_dev(all_map)
    maps, plane = rasterizer._render_geo_forward_raw(P, H, W, cam["tanfovx"], cam["tanfovy"], amap, to_dev(cl),
                                                     f["R"], f["geom"], f["binning"], f["img"])
    bn, rf, geo, rb = _oracle(cam, pre, cl, all_map, bg, grads)
    assert f["R"] == bn["R"]
    assert_close_abs(np_(f["color"]), rf["color"], "color")
    assert_close_abs(np_(maps), geo["out_all_map"], "out_all_map")
    assert_plane_depth_close(np_(plane), geo["out_plane_depth"], geo["out_all_map"], cam, "out_plane_depth")
    out = rasterizer._render_backward_raw(
        rs.bg, f["R"], H, W, dev["means2D"], dev["conic_opacity"], dev["rgb"], to_dev(cl), f["geom"], f["binning"],
        f["img"], to_dev(grads["dpix"]), 3,
        geo=(cam["tanfovx"], cam["tanfovy"], maps, amap, to_dev(grads["dmaps"]), to_dev(grads["dplane"])))
    got = dict(zip(GRADS, out[:4] + (out[5],)))
    assert not np_(got["dL_dmeans2D"])[:, 2].any()
    for k in GRADS:
        e = rel_l2(np_(got[k]), rb[k])
        assert e < 1e-3, (k, e)
    assert np.abs(rb["dL_dall_map"]).max() > 0
    # the plane depth's gradient reaches the maps: without it dL/dall_map changes
    assert rel_l2(np_(got["dL_dall_map"]), _oracle(cam, pre, cl, all_map, bg,
                                                    dict(grads, dplane=0 * grads["dplane"]))[3]["dL_dall_map"]) > 1e-2


def _fused_vs_two_walks(cam, pre, cl, all_map, bg):
    """The fused forward (colour and maps in one walk) against the plain
    forward followed by the second walk: every colour output, statistic and
    buffer, and the maps and plane depth, bit for bit."""
    import torch
    W, H = cam["W"], cam["H"]
    P = len(all_map)
    rs = settings_for(cam, bg=bg)
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    amap = to_dev(all_map)
    args = (rs.bg, H, W, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], to_dev(cl))
    plain = rasterizer._render_forward_raw(*args)
    R = plain[0]
    maps2, plane2 = rasterizer._render_geo_forward_raw(P, H, W, cam["tanfovx"], cam["tanfovy"], amap, to_dev(cl), R,
                                                       plain[6], plain[7], plain[8])
    fused = rasterizer._render_forward_raw(*args, geo=(cam["tanfovx"], cam["tanfovy"], amap))
    torch.cuda.synchronize()
    assert fused[0] == R
    for k, name in ((1, "color"), (2, "n_render"), (3, "n_consider"), (4, "n_contrib"), (5, "out_observe")):
        assert_bitexact(np_(fused[k]), np_(plain[k]), name)
    vf = buffer_views(R, W, H, fused[7], fused[8], P, dev["depths"], fused[6])
    vp = buffer_views(R, W, H, plain[7], plain[8], P, dev["depths"], plain[6])
    for k in ("point_list", "keys", "ranges", "final_T", "n_contrib_px", "n_contrib2loss_px"):
        assert_bitexact(np_(vf[k]), np_(vp[k]), k)
    assert_bitexact(np_(fused[10]), np_(maps2), "out_all_map")
    assert_bitexact(np_(fused[11]), np_(plane2), "out_plane_depth")
    return fused


@pytest.mark.parametrize("masked", [False, True])
def test_geo_fused_forward_equals_plain_forward_and_second_walk(gpu, masked):
    scene, cam, pre, cl, all_map, grads = _case(23 + masked, masked)
    bg = np.array([0.3, 0.2, 0.1], np.float32)
    print(f"render_geo fused forward: P={len(all_map)} W={cam['W']} H={cam['H']} masked={masked}", flush=True)
    fused = _fused_vs_two_walks(cam, pre, cl, all_map, bg)
    _, _, geo, _ = _oracle(cam, pre, cl, all_map, bg, grads)
    assert_close_abs(np_(fused[10]), geo["out_all_map"], "out_all_map")
    assert_plane_depth_close(np_(fused[11]), geo["out_plane_depth"], geo["out_all_map"], cam, "out_plane_depth")


def test_geo_autograd_and_raw_ops(gpu, monkeypatch):
    monkeypatch.syspath_prepend(DROPIN)
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)
    R_pkg = importlib.import_module("diff_gaussian_rasterization_r")
    try:
        scene, cam, pre, cl, all_map, grads = _case(29, True, P=3000, W=160, H=128)
        bg = np.array([0.0, 0.3, 0.6], np.float32)
        W, H = cam["W"], cam["H"]
        P = len(all_map)
        print(f"render_geo autograd: P={P} W={W} H={H}", flush=True)
        rs = R_pkg.GaussianRasterizationSettings(**dict(settings_for(cam, bg=bg)._asdict(), render_geo=True))
        ras = R_pkg.GaussianRasterizer(raster_settings=rs)
        leaf = {k: to_dev(pre[k]).requires_grad_(k in ("means2D", "conic_opacity", "rgb"))
                for k in ["means2D", "conic_opacity", "rgb"]}
        m2_abs = torch.zeros((P, 3), device="cuda", requires_grad=True)
        amap = to_dev(all_map).requires_grad_(True)
        clt = to_dev(cl).bool()
        color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth = ras.render_gaussians(
            leaf["means2D"], m2_abs, leaf["conic_opacity"], leaf["rgb"], amap, to_dev(pre["depths"]),
            to_dev(pre["radii"]), clt, clt, {"stats_collector": {}, "avoid_pixel_all2all": False})
        loss = ((color * to_dev(grads["dpix"])).sum() + (out_all_map * to_dev(grads["dmaps"])).sum()
                + (out_plane_depth * to_dev(grads["dplane"])).sum())
        loss.backward()
        bn, rf, geo, rb = _oracle(cam, pre, cl, all_map, bg, grads)
        assert_close_abs(np_(out_all_map), geo["out_all_map"], "out_all_map (autograd)")
        assert_plane_depth_close(np_(out_plane_depth), geo["out_plane_depth"], geo["out_all_map"], cam,
                                 "out_plane_depth (autograd)")
        for got, ref, nm in ((leaf["means2D"].grad, rb["dL_dmeans2D"][:, :2], "means2D"),
                             (m2_abs.grad, rb["dL_dmeans2D_abs"], "means2D_abs"),
                             (leaf["conic_opacity"].grad, rb["dL_dconic_opacity"], "conic_opacity"),
                             (leaf["rgb"].grad, rb["dL_dcolors"], "rgb"),
                             (amap.grad, rb["dL_dall_map"], "all_map")):
            e = rel_l2(np_(got), ref)
            assert e < 1e-3, (nm, e)
        # the raw _C ops with the reference's positional signatures (_r/ext.cpp:18-22)
        C = R_pkg._C
        t = lambda a: to_dev(np.asarray(a, np.float32))
        args = {"stats_collector": {}}
        r = C.render_gaussians(t(bg), H, W, to_dev(pre["means2D"]), to_dev(pre["depths"]), to_dev(pre["radii"]),
                               to_dev(pre["conic_opacity"]), to_dev(pre["rgb"]), clt, t(cam["viewmatrix"]),
                               t(cam["campos"]), cam["tanfovx"], cam["tanfovy"], to_dev(all_map), True, False, args)
        Rn, col, _, _, _, _, oam, opd, geom, binning, img = r
        assert_close_abs(np_(oam), geo["out_all_map"], "out_all_map (raw)")
        assert_plane_depth_close(np_(opd), geo["out_plane_depth"], geo["out_all_map"], cam, "out_plane_depth (raw)")
        g = C.render_gaussians_backward(t(bg), cam["tanfovx"], cam["tanfovy"], oam, to_dev(all_map), Rn, geom,
                                        binning, img, clt, to_dev(grads["dpix"]), to_dev(grads["dmaps"]),
                                        to_dev(grads["dplane"]), to_dev(pre["means2D"]), to_dev(pre["conic_opacity"]),
                                        to_dev(pre["rgb"]), True, False, args)
        for got, k in zip(g, GRADS):
            e = rel_l2(np_(got), rb[k])
            assert e < 1e-3, (k, e)
    finally:
        for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
            sys.modules.pop(m, None)


def test_geo_autograd_avoid_pixel_all2all(gpu, monkeypatch):
    # avoid_pixel_all2all: the forward (colour, maps, plane depth) renders the
    # tiles of extended_compute_locally, the backward differentiates only those
    # of compute_locally (a narrower block of tile rows inside them)
    monkeypatch.syspath_prepend(DROPIN)
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)
    R_pkg = importlib.import_module("diff_gaussian_rasterization_r")
    try:
        scene, cam, pre, _, all_map, grads = _case(31, False, P=3500, W=176, H=160)
        bg = np.array([0.3, 0.1, 0.2], np.float32)
        W, H = cam["W"], cam["H"]
        P = len(all_map)
        gx, gy = O.tile_grid(W, H)
        cl = np.zeros((gy, gx), np.uint8)
        cl[3:6] = 1
        ext = np.zeros((gy, gx), np.uint8)
        ext[2:8] = 1
        print(f"render_geo avoid_pixel_all2all: P={P} W={W} H={H}", flush=True)
        rs = R_pkg.GaussianRasterizationSettings(**dict(settings_for(cam, bg=bg)._asdict(), render_geo=True))
        ras = R_pkg.GaussianRasterizer(raster_settings=rs)
        leaf = {k: to_dev(pre[k]).requires_grad_(True) for k in ["means2D", "conic_opacity", "rgb"]}
        m2_abs = torch.zeros((P, 3), device="cuda", requires_grad=True)
        amap = to_dev(all_map).requires_grad_(True)
        color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth = ras.render_gaussians(
            leaf["means2D"], m2_abs, leaf["conic_opacity"], leaf["rgb"], amap, to_dev(pre["depths"]),
            to_dev(pre["radii"]), to_dev(cl).bool(), to_dev(ext).bool(),
            {"stats_collector": {}, "avoid_pixel_all2all": True})
        loss = ((color * to_dev(grads["dpix"])).sum() + (out_all_map * to_dev(grads["dmaps"])).sum()
                + (out_plane_depth * to_dev(grads["dplane"])).sum())
        loss.backward()
        bn, rf, geo, rb = _oracle(cam, pre, ext, all_map, bg, grads, cl_bwd=cl)
        assert_close_abs(np_(color), rf["color"], "color (extended rows)")
        assert np_(color)[:, 2 * 16:3 * 16].any()                       # an extended-only row is rendered
        assert_close_abs(np_(out_all_map), geo["out_all_map"], "out_all_map (extended rows)")
        assert_plane_depth_close(np_(out_plane_depth), geo["out_plane_depth"], geo["out_all_map"], cam,
                                 "out_plane_depth (extended rows)")
        # the backward over compute_locally differs from one over the extended mask
        rb_ext = _oracle(cam, pre, ext, all_map, bg, grads)[3]
        assert rel_l2(rb_ext["dL_dall_map"], rb["dL_dall_map"]) > 1e-2
        for got, ref, nm in ((leaf["means2D"].grad, rb["dL_dmeans2D"][:, :2], "means2D"),
                             (m2_abs.grad, rb["dL_dmeans2D_abs"], "means2D_abs"),
                             (leaf["conic_opacity"].grad, rb["dL_dconic_opacity"], "conic_opacity"),
                             (leaf["rgb"].grad, rb["dL_dcolors"], "rgb"),
                             (amap.grad, rb["dL_dall_map"], "all_map")):
            e = rel_l2(np_(got), ref)
            assert e < 1e-3, (nm, e)
    finally:
        for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
            sys.modules.pop(m, None)


def test_geo_config2_full_size_vs_oracle(gpu):
    # the headline size (6M SH3 Gaussians, 1600x1066, > 8M instances): the maps'
    # staging and the Gaussian ids the geometry passes read, at full list lengths
    scene, cam = synth.config2()
    W, H = cam["W"], cam["H"]
    pre = O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                           scene["opacities"])
    P = len(pre["radii"])
    rng = np.random.default_rng(2)
    all_map = rng.uniform(-1.0, 1.0, (P, 5)).astype(np.float32)
    all_map[:, 2] = rng.uniform(-1.5, -0.5, P)
    grads = dict(dpix=scene["dL_dimage"].astype(np.float32),
                 dmaps=rng.normal(size=(5, H, W)).astype(np.float32),
                 dplane=(0.1 * rng.normal(size=(1, H, W))).astype(np.float32))
    cl = np.ones(O.tile_grid(W, H)[::-1], np.uint8)
    bg = np.zeros(3, np.float32)
    print(f"render_geo config 2: P={P} W={W} H={H}", flush=True)
    _fused_vs_two_walks(cam, pre, cl, all_map, bg)
    rs = settings_for(cam, bg=bg)
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    f = gpu_render_forward(rs, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], cl)
    amap = to_dev(all_map)
    maps, plane = rasterizer._render_geo_forward_raw(P, H, W, cam["tanfovx"], cam["tanfovy"], amap, to_dev(cl),
                                                     f["R"], f["geom"], f["binning"], f["img"])
    out = rasterizer._render_backward_raw(
        rs.bg, f["R"], H, W, dev["means2D"], dev["conic_opacity"], dev["rgb"], to_dev(cl), f["geom"], f["binning"],
        f["img"], to_dev(grads["dpix"]), 3,
        geo=(cam["tanfovx"], cam["tanfovy"], maps, amap, to_dev(grads["dmaps"]), to_dev(grads["dplane"])))
    bn, rf, geo, rb = _oracle(cam, pre, cl, all_map, bg, grads)
    assert f["R"] == bn["R"] and f["R"] > 8_000_000
    assert_close_abs(np_(maps), geo["out_all_map"], "out_all_map")
    assert_plane_depth_close(np_(plane), geo["out_plane_depth"], geo["out_all_map"], cam, "out_plane_depth")
    got = dict(zip(GRADS, out[:4] + (out[5],)))
    errs = {k: rel_l2(np_(got[k]), rb[k]) for k in GRADS}
    print("render_geo config 2 gradient errors:", errs)
    assert max(errs.values()) < 1e-3, errs
