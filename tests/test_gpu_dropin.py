"""The split drop-in as BlitzGS imports and calls it, against the CPU oracle.

* gaussian_renderer's keyword call sequence (gaussian_renderer/__init__.py:
  205-217 cuda_args with string values, 311-327 settings / rasterizer /
  preprocess_gaussians / means2D.retain_grad, 795-824 means2D_abs leaf and
  render_gaussians) through `diff_gaussian_rasterization_f` imported from the
  drop-in directory, once with avoid_pixel_all2all off and once on with an
  extended mask wider than compute_locally;
* the raw `_C` ops with the reference's positional signatures and tuples
  (_f/ext.cpp:25-28, _r/ext.cpp:18-22), reached through
  `_get_split_op_backend` (render ops from the _r package), with the
  reference's (P,3) dL/dmeans2D on both sides of the preprocess backward.
Bar: preprocess outputs bit-exact, the image within 1e-4 max-abs (counts up
to rare threshold cases), gradients within 1e-3 relative L2.
"""
import importlib
import os
import sys

import numpy as np
import pytest
import torch

from blitzgs_amd import synth
from tests.gpu_helpers import (GRAD_NAMES, PARAM_KEYS, assert_bitexact, assert_blend_counts, assert_close_abs, np_,
                               oracle_step, rel_l2, to_dev)

pytestmark = pytest.mark.gpu

DROPIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "blitzgs_amd", "dropin")


@pytest.fixture()
def f_pkg(gpu, monkeypatch):
    monkeypatch.syspath_prepend(DROPIN)
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)
    yield importlib.import_module("diff_gaussian_rasterization_f")
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)


def _cuda_args(avoid):
    # get_cuda_args_final (gaussian_renderer/__init__.py:205-217)
    return {"mode": "train", "world_size": "1", "global_rank": "0", "local_rank": "0", "mp_world_size": "1",
            "mp_rank": "0", "log_folder": "/tmp/blitzgs_amd_test", "log_interval": "10", "iteration": "1",
            "avoid_pixel_all2all": avoid, "stats_collector": {}}


def _scene(wide=False):
    # wide: Gaussians with ~67 tile instances each, for which the backward
    # walks 16x8 half tiles, two pixels per lane
    if wide:
        scene, cam = synth.small_scene(2500, seed=64, W=287, H=213, extent=1.4, log_mu=-1.2)
    else:
        scene, cam = synth.small_scene(7000, seed=64, W=287, H=213, extent=1.4, log_mu=-2.4)
    gx, gy = (287 + 15) // 16, (213 + 15) // 16
    cl = np.zeros((gy, gx), np.uint8)
    cl[3:9, :] = 1                                   # a tile-row block, as the strategy builds
    ext = cl.copy()
    ext[2:10, :] = 1                                 # one extra tile row on each side
    return scene, cam, cl, ext


@pytest.mark.parametrize("avoid,wide", [(False, False), (True, False), (True, True)])
def test_gaussian_renderer_call_sequence(f_pkg, avoid, wide):
    F = f_pkg
    scene, cam, cl_np, ext_np = _scene(wide)
    bg = (0.1, 0.3, 0.2)
    t = lambda a: to_dev(np.asarray(a, np.float32))
    raster_settings = F.GaussianRasterizationSettings(
        image_height=int(cam["H"]), image_width=int(cam["W"]), tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
        bg=t(bg), scale_modifier=1.0, viewmatrix=t(cam["viewmatrix"]), projmatrix=t(cam["projmatrix"]),
        sh_degree=3, campos=t(cam["campos"]), prefiltered=False, debug=False)
    rasterizer = F.GaussianRasterizer(raster_settings=raster_settings)
    params = {k: to_dev(scene[k]).requires_grad_(True) for k in PARAM_KEYS}
    cuda_args = _cuda_args(avoid)
    means2D, rgb_precomp, conic_opacity, radii, depths = rasterizer.preprocess_gaussians(
        means3D=params["means3D"], scales=params["scales"], rotations=params["rotations"], shs=params["sh"],
        opacities=params["opacities"], cuda_args=cuda_args)
    means2D.retain_grad()
    P = means2D.shape[0]
    input_all_map = torch.zeros((P, 5)).cuda().float()
    screenspace_points_abs = torch.zeros_like(params["means3D"], dtype=means2D.dtype, requires_grad=True,
                                              device="cuda") + 0
    screenspace_points_abs.retain_grad()
    compute_locally = to_dev(cl_np).bool()
    extended_compute_locally = to_dev(ext_np).bool()
    rendered_image, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth = (
        rasterizer.render_gaussians(means2D=means2D, means2D_abs=screenspace_points_abs, conic_opacity=conic_opacity,
                                    rgb=rgb_precomp, all_map=input_all_map, depths=depths, radii=radii,
                                    compute_locally=compute_locally, extended_compute_locally=extended_compute_locally,
                                    cuda_args=cuda_args))
    assert out_all_map.shape == (5, cam["H"], cam["W"]) and out_plane_depth.shape == (1, cam["H"], cam["W"])
    assert not out_all_map.any() and not out_plane_depth.any()
    assert radii.dtype == torch.int32 and not radii.requires_grad and not depths.requires_grad
    torch.autograd.backward([rendered_image], [to_dev(scene["dL_dimage"])])
    assert set(cuda_args["stats_collector"]) >= {"forward_render_time", "backward_render_time"}

    fwd_mask = ext_np if avoid else cl_np
    pre, bn, rf, rb, pb = oracle_step(scene, cam, bg=bg, cl_fwd=fwd_mask, cl_bwd=cl_np,
                                      dL_dimage=scene["dL_dimage"])
    assert_close_abs(np_(rendered_image), rf["color"], "rendered_image")
    assert_bitexact(np_(n_render), rf["n_render"], "n_render")
    assert_blend_counts(dict(out_observe=np_(out_observe), n_consider=np_(n_consider), n_contrib=np_(n_contrib)), rf,
                        f"avoid_pixel_all2all={avoid}")
    if avoid:
        # the extended rows are rendered
        assert np_(rendered_image)[:, 2 * 16:3 * 16].any()
    assert means2D.grad.shape == (P, 2)
    assert rel_l2(np_(means2D.grad), rb["dL_dmeans2D"][:, :2]) < 1e-3
    assert rel_l2(np_(screenspace_points_abs.grad), rb["dL_dmeans2D_abs"]) < 1e-3
    for k in PARAM_KEYS:
        e = rel_l2(np_(params[k].grad), pb[GRAD_NAMES[k]])
        assert e < 1e-3, (k, e)


def test_raw_split_ops_positional(f_pkg):
    F = f_pkg
    scene, cam, cl_np, _ = _scene()
    bg = np.array([0.4, 0.0, 0.7], np.float32)
    H, W = int(cam["H"]), int(cam["W"])
    t = lambda a: to_dev(np.asarray(a, np.float32))
    args = {"stats_collector": {}, "avoid_pixel_all2all": False}
    pre_op = F._get_split_op_backend("preprocess_gaussians")
    dev = {k: to_dev(scene[k]) for k in PARAM_KEYS}
    out = pre_op.preprocess_gaussians(dev["means3D"], dev["scales"], dev["rotations"], dev["sh"], dev["opacities"],
                                      1.0, t(cam["viewmatrix"]), t(cam["projmatrix"]), cam["tanfovx"],
                                      cam["tanfovy"], H, W, 3, t(cam["campos"]), False, False, args)
    assert len(out) == 8
    num_rendered, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped = out
    cl = to_dev(cl_np).bool()
    P = means2D.shape[0]
    all_map = torch.zeros((P, 5), device="cuda")
    ren_op = F._get_split_op_backend("render_gaussians")
    r = ren_op.render_gaussians(t(bg), H, W, means2D, depths, radii, conic_opacity, rgb, cl, t(cam["viewmatrix"]),
                                t(cam["campos"]), cam["tanfovx"], cam["tanfovy"], all_map, False, False, args)
    assert len(r) == 11
    R, color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth, geom, binning, img = r
    pre, bn, rf, rb, pb = oracle_step(scene, cam, bg=bg, cl_fwd=cl_np, cl_bwd=cl_np, dL_dimage=scene["dL_dimage"])
    assert R == bn["R"]
    for k, v in (("means2D", means2D), ("depths", depths), ("radii", radii), ("cov3D", cov3D),
                 ("conic_opacity", conic_opacity), ("rgb", rgb)):
        assert_bitexact(np_(v), pre[k], k)
    assert_bitexact(np_(clamped).astype(np.uint8), pre["clamped"], "clamped")
    assert_close_abs(np_(color), rf["color"], "color")
    bwd_op = F._get_split_op_backend("render_gaussians_backward")
    g = bwd_op.render_gaussians_backward(t(bg), cam["tanfovx"], cam["tanfovy"], out_all_map, all_map, R, geom,
                                         binning, img, cl, to_dev(scene["dL_dimage"]),
                                         torch.zeros_like(out_all_map), torch.zeros((H, W), device="cuda"),
                                         means2D, conic_opacity, rgb, False, False, args)
    assert len(g) == 5
    dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, dL_dall_map = g
    assert dL_dmeans2D.shape == (P, 3) and not dL_dmeans2D[:, 2].any()
    assert dL_dall_map.shape == (P, 5) and not dL_dall_map.any()
    for got, ref, nm in ((dL_dmeans2D, rb["dL_dmeans2D"], "dL_dmeans2D"),
                         (dL_dmeans2D_abs, rb["dL_dmeans2D_abs"], "dL_dmeans2D_abs"),
                         (dL_dconic_opacity, rb["dL_dconic_opacity"], "dL_dconic_opacity"),
                         (dL_dcolors, rb["dL_dcolors"], "dL_dcolors")):
        assert rel_l2(np_(got), ref) < 1e-3, nm
    assert set(args["stats_collector"]) >= {"forward_render_time", "backward_render_time"}
    pbw_op = F._get_split_op_backend("preprocess_gaussians_backward")
    out = pbw_op.preprocess_gaussians_backward(radii, cov3D, clamped, dev["means3D"], dev["scales"],
                                               dev["rotations"], dev["sh"], 1.0, t(cam["viewmatrix"]),
                                               t(cam["projmatrix"]), cam["tanfovx"], cam["tanfovy"], H, W, 3,
                                               t(cam["campos"]), dL_dmeans2D, dL_dconic_opacity, dL_dcolors, R, False,
                                               args)
    assert len(out) == 5
    for got, k in zip(out, PARAM_KEYS):
        e = rel_l2(np_(got), pb[GRAD_NAMES[k]])
        assert e < 1e-3, (k, e)


def test_debug_mode_synchronises(f_pkg):
    # debug=True: every call waits for the device and raises on a failure
    # (CHECK_CUDA with debug); a healthy call returns the same results
    F = f_pkg
    scene, cam, _, _ = _scene()
    t = lambda a: to_dev(np.asarray(a, np.float32))
    outs = []
    for debug in (False, True):
        rs = F.GaussianRasterizationSettings(
            image_height=int(cam["H"]), image_width=int(cam["W"]), tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
            bg=t((0, 0, 0)), scale_modifier=1.0, viewmatrix=t(cam["viewmatrix"]), projmatrix=t(cam["projmatrix"]),
            sh_degree=3, campos=t(cam["campos"]), prefiltered=False, debug=debug)
        ras = F.GaussianRasterizer(raster_settings=rs)
        dev = {k: to_dev(scene[k]) for k in PARAM_KEYS}
        m2, rgb, co, radii, depths = ras.preprocess_gaussians(dev["means3D"], dev["scales"], dev["rotations"],
                                                              dev["sh"], dev["opacities"], _cuda_args(False))
        P = m2.shape[0]
        color = ras.render_gaussians(m2, torch.zeros((P, 3), device="cuda"), co, rgb, torch.zeros((P, 5), device="cuda"),
                                     depths, radii, None, None, _cuda_args(False))[0]
        outs.append(np_(color))
    assert_bitexact(outs[1], outs[0], "debug-mode image")
