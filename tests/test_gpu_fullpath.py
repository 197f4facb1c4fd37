"""GPU parity of the full-image rasterize path (GaussianRasterizer.forward /
render_simp / backward / markVisible of diff-gaussian-rasterization_f)
against the CPU oracle (oracle/o_preprocess.c, oracle/o_render.c), through
the C ABI.

* preprocess (all degrees, culling mask, precomputed colours, precomputed 3D
  covariances) and the tile-culled binning (sorted ids, ranges): bit-exact;
  the image and final T within 1e-4 max-abs, contributor counts and
  accum_max_count equal up to rare threshold cases (the blend's exp is the
  hardware exp2; tests/gpu_helpers.py);
* render_simp: accum_weights_count and accum_max_count as the counts above,
  accum_weights within 1e-4;
* gradients (also with active alpha clamps, precomputed colours and
  covariances): relative L2 below 1e-3 of the oracle;
* the autograd module, the raw _C ops and markVisible.
"""
import numpy as np
import pytest
import torch

from blitzgs_amd import fullpath, synth
from blitzgs_amd.rasterizer import GaussianRasterizer
from oracle import oracle as O
from tests.gpu_helpers import (assert_bitexact, assert_close_abs, assert_counts_close, buffer_views, np_, rel_l2,
                               settings_for, to_dev)

pytestmark = pytest.mark.gpu


def _split_sh(scene):
    sh = np.asarray(scene["sh"], np.float32)
    return np.ascontiguousarray(sh[:, :1]), np.ascontiguousarray(sh[:, 1:])


def _run(scene, cam, bg=(0.0, 0.0, 0.0), culling=None, colors_precomp=None, cov3D_precomp=None, deg=3,
         flag_max_count=True, simp=False):
    rs = settings_for(cam, bg=bg, sh_degree=deg)
    dc, rest = _split_sh(scene)
    x = fullpath._inputs(rs, to_dev(scene["means3D"]), to_dev(dc), to_dev(rest),
                         None if colors_precomp is None else to_dev(colors_precomp),
                         to_dev(scene["opacities"]), to_dev(scene["scales"]), to_dev(scene["rotations"]),
                         None if cov3D_precomp is None else to_dev(cov3D_precomp))
    cull = None if culling is None else to_dev(culling.astype(bool))
    color, radii, amc, aw, awc, geom, binning, img, R = fullpath._forward(rs, x, cull, flag_max_count, simp)
    W, H = cam["W"], cam["H"]
    g = fullpath._Geom(x["P"], W, H).views(geom)
    views = buffer_views(R, W, H, binning, img, x["P"], g["depths"], fullpath._Geom(x["P"], W, H).render_ws(geom))
    return dict(rs=rs, x=x, color=color, radii=radii, amc=amc, aw=aw, awc=awc, geom=geom, binning=binning, img=img,
                R=R, g=g, **views)


def _oracle(scene, cam, bg=(0.0, 0.0, 0.0), culling=None, colors_precomp=None, cov3D_precomp=None, deg=3,
            flag_max_count=True, simp=False):
    return O.full_path_forward(cam, scene, bg=np.asarray(bg, np.float32), culling=culling,
                               colors_precomp=colors_precomp, cov3D_precomp=cov3D_precomp,
                               flag_max_count=flag_max_count, simp=simp, sh_degree=deg)


def _check_forward(got, pre, bn, rf):
    g = got["g"]
    assert_bitexact(np_(g["means2D"]), pre["means2D"], "means2D")
    assert_bitexact(np_(got["radii"]), pre["radii"], "radii")
    assert_bitexact(np_(g["conic"]), pre["conic_opacity"], "conic_opacity")
    assert_bitexact(np_(g["depths"]), pre["depths"], "depths")
    assert_bitexact(np_(g["rects"]), pre["rects"], "rects")
    assert_bitexact(np_(g["tiles"]).view(np.uint32), pre["tiles_touched"], "tiles_touched")
    assert got["R"] == bn["valid"]
    assert_bitexact(np_(got["point_list"]).view(np.uint32), bn["point_list"][:bn["valid"]], "point_list")
    assert_bitexact(np_(got["ranges"]).view(np.uint32), bn["ranges"], "ranges")
    assert_close_abs(np_(got["color"]), rf["color"], "color")
    assert_close_abs(np_(got["final_T"]), rf["final_T"], "final_T")
    assert_counts_close(np_(got["n_contrib_px"]).view(np.uint32), rf["n_contrib_px"], "n_contrib")
    assert_counts_close(np_(got["amc"]), rf["accum_max_count"], "accum_max_count")


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_forward_bitexact_config0(gpu, deg):
    scene, cam = synth.config0()
    bg = (0.1, 0.2, 0.3)
    got = _run(scene, cam, bg=bg, deg=deg)
    pre, bn, rf = _oracle(scene, cam, bg=bg, deg=deg)
    assert_bitexact(np_(got["g"]["rgb"]), pre["rgb"], "rgb")
    assert_bitexact(np_(got["g"]["clamped"]), pre["clamped"], "clamped")
    assert_bitexact(np_(got["g"]["cov3D"]), pre["cov3D"], "cov3D")
    _check_forward(got, pre, bn, rf)
    assert bn["valid"] < bn["R"]     # the tile test did cull instances


def test_forward_culling_and_precomputed_inputs(gpu):
    scene, cam = synth.small_scene(3000, seed=11, W=200, H=150, log_mu=-2.2)
    P = scene["means3D"].shape[0]
    rng = np.random.default_rng(11)
    cull = rng.random(P) < 0.3
    got = _run(scene, cam, culling=cull)
    _check_forward(got, *_oracle(scene, cam, culling=cull))
    cols = rng.random((P, 3)).astype(np.float32)
    got = _run(scene, cam, colors_precomp=cols)
    _check_forward(got, *_oracle(scene, cam, colors_precomp=cols))
    pre0, _, _ = _oracle(scene, cam)
    got = _run(scene, cam, cov3D_precomp=pre0["cov3D"])
    _check_forward(got, *_oracle(scene, cam, cov3D_precomp=pre0["cov3D"]))
    got = _run(scene, cam, flag_max_count=False)
    assert not np_(got["amc"]).any()


def test_render_simp(gpu):
    scene, cam = synth.config0()
    got = _run(scene, cam, simp=True)
    pre, bn, rf = _oracle(scene, cam, simp=True)
    _check_forward(got, pre, bn, rf)
    assert_counts_close(np_(got["awc"]), rf["accum_weights_count"], "accum_weights_count")
    np.testing.assert_allclose(np_(got["aw"]), rf["accum_weights"], rtol=1e-4, atol=1e-4)
    # the public entry point returns the reference's tuple order
    rs = settings_for(cam)
    dc, rest = _split_sh(scene)
    ras = GaussianRasterizer(rs)
    color, radii, aw, awc, amc = ras.render_simp(
        means3D=to_dev(scene["means3D"]), means2D=None, opacities=to_dev(scene["opacities"]),
        culling=torch.zeros(len(pre["radii"]), dtype=torch.bool, device="cuda"), dc=to_dev(dc), shs=to_dev(rest),
        scales=to_dev(scene["scales"]), rotations=to_dev(scene["rotations"]))
    assert_close_abs(np_(color), rf["color"], "render_simp color")
    assert_counts_close(np_(awc), rf["accum_weights_count"], "render_simp counts")


def _grads_oracle(scene, cam, bg, dLd, pre, bn, rf, colors_precomp=None, cov3D_precomp=None):
    W, H = cam["W"], cam["H"]
    colors = pre["rgb"] if colors_precomp is None else colors_precomp
    rb = O.render_bwd_full(W, H, np.asarray(bg, np.float32), pre["means2D"], pre["conic_opacity"], colors,
                           bn["ranges"], bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd)
    dc, rest = _split_sh(scene)
    pb = O.preprocess_bwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], dc, rest, pre["radii"],
                               pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic"], rb["dL_dcolors"],
                               colors_precomp=colors_precomp, cov3D_precomp=cov3D_precomp)
    return rb, pb


def _check_grads(got_tuple, rb, pb, what):
    (g_m2d, g_col, g_op, g_m3d, g_cov, g_dc, g_sh, g_sc, g_rot) = [np_(t) for t in got_tuple]
    pairs = [("dL_dmeans2D", g_m2d, rb["dL_dmeans2D"]), ("dL_dcolors", g_col, rb["dL_dcolors"]),
             ("dL_dopacity", g_op.reshape(-1), rb["dL_dopacity"]), ("dL_dmeans3D", g_m3d, pb["dL_dmeans3D"]),
             ("dL_dcov3D", g_cov, pb["dL_dcov3D"]), ("dL_ddc", g_dc, pb["dL_ddc"]), ("dL_dsh", g_sh, pb["dL_dsh"]),
             ("dL_dscales", g_sc, pb["dL_dscales"]), ("dL_drotations", g_rot, pb["dL_drotations"])]
    for name, g, r in pairs:
        assert g.shape == r.shape, (what, name, g.shape, r.shape)
        if np.abs(r).max() == 0:
            assert np.abs(g).max() == 0, (what, name)
            continue
        e = rel_l2(g, r)
        assert e < 1e-3, (what, name, e)


@pytest.mark.parametrize("case", ["plain", "clamped", "colors", "cov3D"])
def test_backward_vs_oracle(gpu, case):
    scene, cam = synth.small_scene(2500, seed=13, W=160, H=128, log_mu=-1.8)
    if case == "clamped":
        scene["opacities"][::3] = 0.9995
    bg = (0.3, 0.1, 0.2)
    dLd = np.random.default_rng(13).standard_normal((3, cam["H"], cam["W"])).astype(np.float32)
    kw = {}
    if case == "colors":
        kw["colors_precomp"] = np.random.default_rng(1).random((2500, 3)).astype(np.float32)
    if case == "cov3D":
        kw["cov3D_precomp"] = _oracle(scene, cam)[0]["cov3D"]
    got = _run(scene, cam, bg=bg, **kw)
    pre, bn, rf = _oracle(scene, cam, bg=bg, **kw)
    _check_forward(got, pre, bn, rf)
    grads = fullpath._backward(got["rs"], got["x"], got["radii"], got["geom"], got["R"], got["binning"],
                               got["img"], to_dev(dLd))
    rb, pb = _grads_oracle(scene, cam, bg, dLd, pre, bn, rf, **kw)
    _check_grads(grads, rb, pb, case)


def test_autograd_module_and_raw_ops(gpu):
    scene, cam = synth.small_scene(2000, seed=17, W=128, H=96, log_mu=-1.9)
    rs = settings_for(cam, bg=(0.2, 0.2, 0.2))
    dc, rest = _split_sh(scene)
    leaves = {k: to_dev(v).requires_grad_() for k, v in
              dict(means3D=scene["means3D"], opacities=scene["opacities"], scales=scene["scales"],
                   rotations=scene["rotations"], dc=dc, rest=rest).items()}
    means2D = torch.zeros_like(leaves["means3D"], requires_grad=True)
    ras = GaussianRasterizer(rs)
    culling = torch.zeros(2000, dtype=torch.bool, device="cuda")
    color, radii, amc = ras(means3D=leaves["means3D"], means2D=means2D, opacities=leaves["opacities"],
                            culling=culling, dc=leaves["dc"], shs=leaves["rest"], scales=leaves["scales"],
                            rotations=leaves["rotations"], flag_max_count=True)
    dLd = torch.randn_like(color)
    (color * dLd).sum().backward()
    pre, bn, rf = _oracle(scene, cam, bg=(0.2, 0.2, 0.2))
    assert_close_abs(np_(color), rf["color"], "module color")
    assert_counts_close(np_(amc), rf["accum_max_count"], "module accum_max_count")
    rb, pb = _grads_oracle(scene, cam, (0.2, 0.2, 0.2), np_(dLd), pre, bn, rf)
    assert rel_l2(np_(means2D.grad), rb["dL_dmeans2D"]) < 1e-3
    assert rel_l2(np_(leaves["means3D"].grad), pb["dL_dmeans3D"]) < 1e-3
    assert rel_l2(np_(leaves["opacities"].grad).reshape(-1), rb["dL_dopacity"]) < 1e-3
    assert rel_l2(np_(leaves["dc"].grad), pb["dL_ddc"]) < 1e-3
    assert rel_l2(np_(leaves["rest"].grad), pb["dL_dsh"]) < 1e-3
    assert rel_l2(np_(leaves["scales"].grad), pb["dL_dscales"]) < 1e-3
    assert rel_l2(np_(leaves["rotations"].grad), pb["dL_drotations"]) < 1e-3
    # the raw _C ops, as the reference's autograd function calls them
    from blitzgs_amd import compat_ops as _C
    e = torch.Tensor([])
    out = _C.rasterize_gaussians(rs.bg, leaves["means3D"].detach(), e, leaves["opacities"].detach(),
                                 leaves["scales"].detach(), leaves["rotations"].detach(), 1.0, e, rs.viewmatrix,
                                 rs.projmatrix, rs.tanfovx, rs.tanfovy, rs.image_height, rs.image_width,
                                 leaves["dc"].detach(), leaves["rest"].detach(), 3, rs.campos, False, True, culling,
                                 False)
    num_rendered, num_buckets, color2, amc2, radii2, geomB, binB, imgB, sampB = out
    assert num_rendered == bn["R"] and num_buckets == bn["num_buckets"]
    assert torch.equal(color2, color) and torch.equal(amc2, amc) and torch.equal(radii2, radii)
    g2 = _C.rasterize_gaussians_backward(rs.bg, leaves["means3D"].detach(), radii2, e, leaves["scales"].detach(),
                                         leaves["rotations"].detach(), 1.0, e, rs.viewmatrix, rs.projmatrix,
                                         rs.tanfovx, rs.tanfovy, dLd, leaves["dc"].detach(),
                                         leaves["rest"].detach(), 3, rs.campos, geomB, num_rendered, binB, imgB,
                                         num_buckets, sampB, False)
    _check_grads(g2, rb, pb, "raw ops")


def test_mark_visible(gpu):
    scene, cam = synth.config0()
    pts = scene["means3D"].copy()
    pts[::5, 2] = -5.0            # behind the camera
    rs = settings_for(cam)
    vis = np_(GaussianRasterizer(rs).markVisible(to_dev(pts)))
    V = np.asarray(cam["viewmatrix"], np.float32).reshape(-1)
    z = (V[2] * pts[:, 0] + V[6] * pts[:, 1]) + V[10] * pts[:, 2] + V[14]
    assert np.array_equal(vis, z > np.float32(0.2))
    assert vis.any() and not vis.all()


def test_config1_full_path_forward_vs_oracle(gpu):
    scene, cam = synth.config1()
    got = _run(scene, cam)
    pre, bn, rf = _oracle(scene, cam)
    _check_forward(got, pre, bn, rf)


def _tile_buckets_scene(specs, seed, n_bg=1500):
    """A 256x256 scene (camera at (0, 0, -4) looking down +z, FoV 60, R = I)
    whose tiles (tx, ty, n, ties) each receive n Gaussians projected onto the
    tile centre with a small isotropic precomputed covariance (the tile test
    keeps only that tile); with ties, half of them lie on the plane z = 0
    (view depth exactly 4.0: one run of equal depths), the rest at depths in
    [3, 7].  n_bg small Gaussians fill the lower half of the image."""
    import math
    rng = np.random.default_rng(seed)
    W = H = 256
    fov = math.radians(60.0)
    cam = synth.make_camera(np.eye(3), (0.0, 0.0, -4.0), W, H, fov, fov)
    tx_, ty_ = float(cam["tanfovx"]), float(cam["tanfovy"])
    pts = []
    for tx, ty, n, ties in specs:
        zw = rng.uniform(-1.0, 3.0, n)
        if ties:
            zw[: n // 2] = 0.0
        zv = zw + 4.0
        px, py = 16 * tx + 8.0, 16 * ty + 8.0
        x = ((2 * px + 1) / W - 1) * tx_ * zv
        y = ((2 * py + 1) / H - 1) * ty_ * zv
        pts.append(np.stack([x, y, zw], 1))
    zb = rng.uniform(-1.0, 1.0, n_bg)
    pyb = rng.uniform(140.0, 250.0, n_bg)
    pxb = rng.uniform(4.0, 252.0, n_bg)
    pts.append(np.stack([((2 * pxb + 1) / W - 1) * tx_ * (zb + 4), ((2 * pyb + 1) / H - 1) * ty_ * (zb + 4), zb], 1))
    means = np.concatenate(pts)
    P = means.shape[0]
    order = rng.permutation(P)
    means = means[order].astype(np.float32)
    scene = synth._finish(rng, means, -4.0, 0.3, 1.0, 0.5, P)
    var = np.float32(0.004 ** 2)
    cov = np.zeros((P, 6), np.float32)
    cov[:, 0] = cov[:, 3] = cov[:, 5] = var
    cols = rng.random((P, 3)).astype(np.float32)
    return scene, cam, cov, cols


def test_full_path_tile_sort_classes_and_tie_runs(gpu):
    # one tile per sort class of the full-image path's per-tile sort: <= 512
    # keys (per-wave register network), 1k, 2k, 4k and 8k (LDS radix sort),
    # > 8192 (EXTRA_BIG: bitonic network in global memory); the radix classes
    # also with a run of more than 32 equal depths (the fallback to the full
    # 64-bit sort in global memory); ties order by ascending id everywhere
    specs = [(1, 1, 300, True), (3, 1, 700, False), (5, 1, 700, True), (7, 1, 1500, False), (9, 1, 1500, True),
             (11, 1, 3000, False), (13, 1, 3000, True), (1, 3, 6000, False), (3, 3, 6000, True),
             (5, 3, 9000, False), (7, 3, 9000, True)]
    scene, cam, cov, cols = _tile_buckets_scene(specs, 51)
    got = _run(scene, cam, colors_precomp=cols, cov3D_precomp=cov)
    pre, bn, rf = _oracle(scene, cam, colors_precomp=cols, cov3D_precomp=cov)
    _check_forward(got, pre, bn, rf)
    n = np.diff(bn["ranges"].reshape(16, 16, 2), axis=2)[..., 0]
    for tx, ty, cnt, ties in specs:
        assert n[ty, tx] == cnt, (tx, ty, n[ty, tx], cnt)
        ids = bn["point_list"][bn["ranges"][ty * 16 + tx, 0]:bn["ranges"][ty * 16 + tx, 1]]
        d = pre["depths"][ids]
        run = np.diff(np.flatnonzero(np.diff(np.r_[-1.0, d, -1.0]) != 0)).max()
        assert (run > 32) == ties, (tx, ty, run)


# ------------------------------------------------------------------ render_depth

def _depth_gpu(scene, cam, bg=(0.0, 0.0, 0.0), culling=None, colors_precomp=None, deg=3):
    rs = settings_for(cam, bg=bg, sh_degree=deg)
    dc, rest = _split_sh(scene)
    ras = GaussianRasterizer(rs)
    cull = torch.zeros(len(scene["means3D"]), dtype=torch.bool, device="cuda") if culling is None \
        else to_dev(culling.astype(bool))
    return ras.render_depth(means3D=to_dev(scene["means3D"]), means2D=None, opacities=to_dev(scene["opacities"]),
                            culling=cull, dc=None if colors_precomp is not None else to_dev(dc),
                            shs=None if colors_precomp is not None else to_dev(rest),
                            colors_precomp=None if colors_precomp is None else to_dev(colors_precomp),
                            scales=to_dev(scene["scales"]), rotations=to_dev(scene["rotations"]))


def _check_depth(res, rd):
    """Colour and transmittance within 1e-4; the per-pixel Gaussian of the
    largest weight (gidx) equal up to rare near-ties; where it is equal, the
    depth, hit point and discriminant (which do not depend on the falloff exp)
    bit-identical."""
    assert_close_abs(np_(res["render"]), rd["color"], "depth render colour")
    assert_close_abs(np_(res["accum_alpha"]), rd["accum_alpha"], "accum_alpha")
    g, r = np_(res["gidx"]), rd["gidx"]
    assert_counts_close(g, r, "gidx")
    same = (g == r)
    for k, rk in (("rendered_depth", "depth"), ("discriminants", "discriminants")):
        assert_bitexact(np_(res[k])[same], rd[rk][same], k)
    assert_bitexact(np_(res["out_pts"])[:, same[0]], rd["out_pts"][:, same[0]], "out_pts")


@pytest.mark.parametrize("case", ["config0", "culling_colors", "negative_depth", "anisotropic"])
def test_render_depth_vs_oracle(gpu, case):
    print(f"render_depth {case}", flush=True)
    bg = (0.1, 0.2, 0.3)
    culling = colors = None
    if case == "config0":
        scene, cam = synth.config0()
    elif case == "culling_colors":
        scene, cam = synth.small_scene(3000, seed=21, W=96, H=80, log_mu=-2.0)
        rng = np.random.default_rng(1)
        culling = rng.random(3000) < 0.3
        colors = rng.random((3000, 3)).astype(np.float32)
    else:
        scene, cam = synth.small_scene(1, seed=9, W=48, H=40)
        if case == "negative_depth":
            mu, q, s = [-3.0, 0.0, -3.5], [1, 0, 0, 0], [2.0, 2.0, 2.0]
        else:
            mu, q, s = [0.1, -0.05, 0.5], [0.8, 0.3, -0.4, 0.2], [1.2, 0.5, 0.3]
        scene["means3D"] = np.array([mu], np.float32)
        scene["rotations"] = np.array([q], np.float32)
        scene["scales"] = np.array([s], np.float32)
        scene["opacities"] = np.array([[0.9]], np.float32)
    res = _depth_gpu(scene, cam, bg=bg, culling=culling, colors_precomp=colors)
    pre, bn, rd = O.full_path_depth(cam, scene, bg=np.asarray(bg, np.float32), culling=culling,
                                    colors_precomp=colors)
    _check_depth(res, rd)
    assert (np_(res["accum_alpha"]) < 1).any()


def test_render_depth_raw_op_and_config1(gpu):
    """The raw _C.rasterize_gaussians_depth tuple, and config 1's 1M Gaussians
    at 1920x1080 against the oracle."""
    from blitzgs_amd import compat_ops as _C
    scene, cam = synth.config1()
    print("render_depth config1", flush=True)
    rs = settings_for(cam)
    dc, rest = _split_sh(scene)
    e = torch.Tensor([])
    out = _C.rasterize_gaussians_depth(rs.bg, to_dev(scene["means3D"]), e, to_dev(scene["opacities"]),
                                       to_dev(scene["scales"]), to_dev(scene["rotations"]), 1.0, e, rs.viewmatrix,
                                       rs.projmatrix, rs.tanfovx, rs.tanfovy, rs.image_height, rs.image_width,
                                       to_dev(dc), to_dev(rest), 3, rs.campos, False,
                                       torch.zeros(len(scene["means3D"]), dtype=torch.bool, device="cuda"), False)
    assert len(out) == 11
    num_rendered, color, out_pts, depth, accum_alpha, gidx, disc, radii = out[:8]
    pre, bn, rd = O.full_path_depth(cam, scene)
    assert num_rendered == bn["R"]
    assert_bitexact(np_(radii), pre["radii"], "radii")
    _check_depth(dict(render=color, out_pts=out_pts, rendered_depth=depth, accum_alpha=accum_alpha, gidx=gidx,
                      discriminants=disc), rd)


def test_render_depth_needs_scales_and_rotations(gpu):
    scene, cam = synth.small_scene(10, seed=1)
    rs = settings_for(cam)
    ras = GaussianRasterizer(rs)
    dc, rest = _split_sh(scene)
    cov = torch.zeros((10, 6), device="cuda")
    with pytest.raises(RuntimeError, match="scales and rotations"):
        ras.render_depth(means3D=to_dev(scene["means3D"]), means2D=None, opacities=to_dev(scene["opacities"]),
                         culling=torch.zeros(10, dtype=torch.bool, device="cuda"), dc=to_dev(dc), shs=to_dev(rest),
                         cov3D_precomp=cov)


def test_repeated_backward_of_one_forward(gpu):
    """GaussianRasterizer.forward differentiated twice (retain_graph): the
    second backward gives the first one's gradients."""
    scene, cam = synth.small_scene(2000, seed=19, W=128, H=96, log_mu=-1.9)
    rs = settings_for(cam, bg=(0.1, 0.1, 0.1))
    dc, rest = _split_sh(scene)
    leaves = {k: to_dev(v).requires_grad_() for k, v in
              dict(means3D=scene["means3D"], opacities=scene["opacities"], scales=scene["scales"],
                   rotations=scene["rotations"], dc=dc, rest=rest).items()}
    means2D = torch.zeros_like(leaves["means3D"], requires_grad=True)
    culling = torch.zeros(2000, dtype=torch.bool, device="cuda")
    color, radii, amc = GaussianRasterizer(rs)(means3D=leaves["means3D"], means2D=means2D,
                                               opacities=leaves["opacities"], culling=culling, dc=leaves["dc"],
                                               shs=leaves["rest"], scales=leaves["scales"],
                                               rotations=leaves["rotations"], flag_max_count=True)
    loss = (color * torch.randn_like(color)).sum()
    loss.backward(retain_graph=True)
    first = {k: v.grad.detach().clone() for k, v in leaves.items()}
    first_m2d = means2D.grad.detach().clone()
    for v in list(leaves.values()) + [means2D]:
        v.grad = None
    loss.backward()
    for k, v in leaves.items():
        assert rel_l2(np_(v.grad), np_(first[k])) < 1e-5, k
    assert rel_l2(np_(means2D.grad), np_(first_m2d)) < 1e-5
