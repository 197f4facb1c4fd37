"""Pin the oracle's render_geo (the _r render's five geometry maps and plane
depth, _r/cuda_rasterizer/forward.cu:381-384,407-412 and backward.cu:393-405,
427-432,476-490) against the colour render it shares its blend with, the
ray-plane intersection the plane depth stands for, and finite differences of
the plane depth's formula."""
import numpy as np
import pytest

from blitzgs_amd import synth
from oracle import oracle as O


def _setup(seed=3, P=600, W=80, H=64, masked=False):
    scene, cam = synth.small_scene(P, seed=seed, W=W, H=H, extent=1.2, log_mu=-2.2)
    pre, bn, _ = O.full_forward(cam, scene)
    rng = np.random.default_rng(seed)
    gx, gy = O.tile_grid(W, H)
    cl = (rng.random(gx * gy) < 0.7).astype(np.uint8) if masked else np.ones(gx * gy, np.uint8)
    if masked:
        bn = O.binning(W, H, pre["means2D"], pre["depths"], pre["radii"], cl)
    all_map = rng.uniform(-1.0, 1.0, (P, 5)).astype(np.float32)
    return cam, pre, bn, cl, all_map, rng


def _fwd(cam, pre, bn, cl, rgb, bg=None):
    bg = np.zeros(3, np.float32) if bg is None else bg
    return O.render_fwd(cam["W"], cam["H"], bg, pre["means2D"], pre["conic_opacity"], rgb, bn["ranges"],
                        bn["point_list"], cl)


@pytest.mark.parametrize("masked", [False, True])
def test_geo_maps_are_the_colour_blend_of_the_map_channels(masked):
    # the maps take the colour's weights alpha T: channel c of out_all_map is
    # the colour render (bg = 0) of a Gaussian colour equal to all_map[:, c]
    cam, pre, bn, cl, all_map, _ = _setup(masked=masked)
    geo = O.render_geo_fwd(cam["W"], cam["H"], cam["tanfovx"], cam["tanfovy"], pre["means2D"],
                           pre["conic_opacity"], all_map, bn["ranges"], bn["point_list"], cl)
    lo = _fwd(cam, pre, bn, cl, all_map[:, 0:3])
    hi = _fwd(cam, pre, bn, cl, np.concatenate([all_map[:, 3:5], np.zeros((len(all_map), 1), np.float32)], 1))
    np.testing.assert_array_equal(geo["out_all_map"][0:3], lo["color"])
    np.testing.assert_array_equal(geo["out_all_map"][3:5], hi["color"][0:2])
    if masked:   # non-local tiles: zeros
        H, W = cam["H"], cam["W"]
        gx = (W + 15) // 16
        px_local = np.repeat(np.repeat(cl.reshape(-1, gx), 16, 0), 16, 1)[:H, :W].astype(bool)
        assert not geo["out_plane_depth"][0][~px_local].any()
        assert not geo["out_all_map"][:, ~px_local].any()


def test_geo_plane_depth_is_the_ray_plane_intersection():
    # every Gaussian carries one plane n . p + d = 0 (maps n0, n1, n2, -, d):
    # the blended maps are (n, d) times the pixel's opacity S = 1 - T, so the
    # plane depth S d / -(S n . ray + 1e-8) is the depth z = -d / (n . ray) at
    # which the ray (rx z, ry z, z) meets the plane, wherever S is not small
    cam, pre, bn, cl, _, _ = _setup(seed=5, P=900)
    W, H = cam["W"], cam["H"]
    n = np.array([0.1, -0.2, -1.0]); d = 3.0
    all_map = np.tile(np.array([[n[0], n[1], n[2], 0.0, d]], np.float32), (len(pre["means2D"]), 1))
    geo = O.render_geo_fwd(W, H, cam["tanfovx"], cam["tanfovy"], pre["means2D"], pre["conic_opacity"], all_map,
                           bn["ranges"], bn["point_list"], cl)
    T = _fwd(cam, pre, bn, cl, np.zeros((len(all_map), 3), np.float32))["final_T"]
    fx = W / (2.0 * cam["tanfovx"]); fy = H / (2.0 * cam["tanfovy"])
    y, x = np.mgrid[0:H, 0:W].astype(np.float64)
    z = -d / (n[0] * (x - 0.5 * W) / fx + n[1] * (y - 0.5 * H) / fy + n[2])
    dense = (1.0 - T) > 0.5
    assert dense.mean() > 0.3
    np.testing.assert_allclose(geo["out_plane_depth"][0][dense], z[dense], rtol=2e-5)
    # no contribution: 0 / -(0 + 1e-8) = -0
    empty = T == 1.0
    assert empty.any()
    dz = geo["out_plane_depth"][0][empty]
    assert (dz == 0).all() and np.signbit(dz).all()


def _bwd_geo(cam, pre, bn, cl, fwd, geo_px, all_map, rgb, bg, dpix, dmaps, dplane):
    return O.render_bwd_geo(cam["W"], cam["H"], cam["tanfovx"], cam["tanfovy"], bg, pre["means2D"],
                            pre["conic_opacity"], rgb, all_map, geo_px, bn["ranges"], bn["point_list"],
                            fwd["final_T"], fwd["n_contrib_px"], dpix, dmaps, dplane, cl)


def _bwd(cam, pre, bn, cl, fwd, rgb, bg, dpix):
    return O.render_bwd(cam["W"], cam["H"], bg, pre["means2D"], pre["conic_opacity"], rgb, bn["ranges"],
                        bn["point_list"], fwd["final_T"], fwd["n_contrib_px"], dpix, cl)


def _close(a, b, rtol=2e-5):
    scale = max(np.abs(b).max(), 1e-30)
    np.testing.assert_allclose(a, b, rtol=rtol, atol=rtol * scale)


KEYS = ["dL_dmeans2D", "dL_dmeans2D_abs", "dL_dconic_opacity"]


@pytest.mark.parametrize("masked", [False, True])
def test_geo_backward_map_terms_are_the_colour_backward_of_the_map_channels(masked):
    # dL/dalpha sums (c - acc) dL/dc over the 3 colours and the 5 maps alike,
    # so with dL/dpixel = 0 and two map gradients zero, the backward of the
    # other three maps is the colour backward of a colour equal to those map
    # channels -- dL/dmean2D_abs (a sum of absolute values) included
    cam, pre, bn, cl, all_map, rng = _setup(seed=7, masked=masked)
    W, H = cam["W"], cam["H"]
    P = len(all_map)
    rgb = rng.random((P, 3)).astype(np.float32)
    bg = np.array([0.3, 0.1, 0.2], np.float32)
    fwd = _fwd(cam, pre, bn, cl, rgb, bg)
    geo_px = O.render_geo_fwd(W, H, cam["tanfovx"], cam["tanfovy"], pre["means2D"], pre["conic_opacity"],
                              all_map, bn["ranges"], bn["point_list"], cl)["out_all_map"]
    g = rng.normal(size=(5, H, W)).astype(np.float32)
    zero3 = np.zeros((3, H, W), np.float32)
    zplane = np.zeros((1, H, W), np.float32)
    for chans in ([0, 1, 2], [3, 4]):
        dmaps = np.zeros_like(g)
        dmaps[chans] = g[chans]
        got = _bwd_geo(cam, pre, bn, cl, fwd, geo_px, all_map, rgb, bg, zero3, dmaps, zplane)
        as_rgb = np.zeros((P, 3), np.float32)
        as_rgb[:, :len(chans)] = all_map[:, chans]
        dpix = np.zeros((3, H, W), np.float32)
        dpix[:len(chans)] = g[chans]
        ref = _bwd(cam, pre, bn, cl, fwd, as_rgb, np.zeros(3, np.float32), dpix)   # maps: no background term
        for k in KEYS:
            _close(got[k], ref[k])
        _close(got["dL_dall_map"][:, chans], ref["dL_dcolors"][:, :len(chans)])
        assert not got["dL_dcolors"].any()
    # all at once: every output but the absolute values is linear in the
    # pixel gradients, so it is the sum of the three separate backwards
    dpix = rng.normal(size=(3, H, W)).astype(np.float32)
    both = _bwd_geo(cam, pre, bn, cl, fwd, geo_px, all_map, rgb, bg, dpix, g, zplane)
    col = _bwd(cam, pre, bn, cl, fwd, rgb, bg, dpix)
    parts = [_bwd_geo(cam, pre, bn, cl, fwd, geo_px, all_map, rgb, bg, zero3,
                      np.where(np.isin(np.arange(5), c)[:, None, None], g, 0).astype(np.float32), zplane)
             for c in ([0, 1, 2], [3, 4])]
    for k in ["dL_dmeans2D", "dL_dconic_opacity"]:
        _close(both[k], col[k] + parts[0][k] + parts[1][k], rtol=1e-4)
    _close(both["dL_dcolors"], col["dL_dcolors"])
    _close(both["dL_dall_map"], parts[0]["dL_dall_map"] + parts[1]["dL_dall_map"])
    # Gaussians with no instance on a local tile: no map gradient
    unlisted = np.setdiff1d(np.arange(P), bn["point_list"])
    assert not both["dL_dall_map"][unlisted].any()
    assert len(unlisted) > 0 or not masked


@pytest.mark.parametrize("band", ["away_from_pole", "near_pole"])
def test_geo_backward_plane_depth_chain_matches_finite_differences(band):
    # dL/dplane_depth enters through the maps: per pixel the backward adds
    # dL/dD * dD/dM to the map gradients, D(M) = M4 / -(M0 rx + M1 ry + M2 + 1e-8);
    # the same backward with that product given directly as map gradients,
    # dD/dM by central differences in float64, must agree -- where the blended
    # n . ray is far from 0, and where it is small (0.003 < |n . ray| < 0.05,
    # D and its derivatives large: the float32 chain's cancellation there)
    cam, pre, bn, cl, all_map, rng = _setup(seed=11, P=700)
    W, H = cam["W"], cam["H"]
    P = len(all_map)
    if band == "away_from_pole":
        all_map[:, 2] = rng.uniform(-1.5, -0.5, P).astype(np.float32)   # n . ray away from 0
    else:
        all_map[:, 2] = rng.uniform(-0.3, 0.3, P).astype(np.float32)    # n . ray crosses 0 in the image
    rgb = rng.random((P, 3)).astype(np.float32)
    bg = np.zeros(3, np.float32)
    fwd = _fwd(cam, pre, bn, cl, rgb, bg)
    geo = O.render_geo_fwd(W, H, cam["tanfovx"], cam["tanfovy"], pre["means2D"], pre["conic_opacity"], all_map,
                           bn["ranges"], bn["point_list"], cl)
    M = geo["out_all_map"].astype(np.float64)
    fx, fy = (float(v) for v in O.focal(W, H, cam["tanfovx"], cam["tanfovy"]))
    y, x = np.mgrid[0:H, 0:W].astype(np.float64)
    rx, ry = (x - 0.5 * W) / fx, (y - 0.5 * H) / fy

    def depth(M):
        return M[4] / -(M[0] * rx + M[1] * ry + M[2] + 1e-8)
    J = np.zeros_like(M)
    for c in (0, 1, 2, 4):
        h = 1e-6 * np.maximum(np.abs(M[c]), 1e-3)
        Mp, Mm = M.copy(), M.copy()
        Mp[c] += h; Mm[c] -= h
        J[c] = (depth(Mp) - depth(Mm)) / (2 * h)
    g = rng.normal(size=(1, H, W))
    dot = np.abs(M[0] * rx + M[1] * ry + M[2])
    # keep pixels whose blended maps are not at a pole of D
    ok = (dot > 0.05) if band == "away_from_pole" else ((dot > 0.003) & (dot < 0.05))
    assert ok.sum() > (50 if band == "near_pole" else 500), int(ok.sum())
    g = np.where(ok[None], g, 0.0)
    zero3 = np.zeros((3, H, W), np.float32)
    via_depth = _bwd_geo(cam, pre, bn, cl, fwd, geo["out_all_map"], all_map, rgb, bg, zero3,
                         np.zeros((5, H, W), np.float32), g.astype(np.float32))
    via_maps = _bwd_geo(cam, pre, bn, cl, fwd, geo["out_all_map"], all_map, rgb, bg, zero3,
                        (J * g).astype(np.float32), np.zeros((1, H, W), np.float32))
    for k in KEYS + ["dL_dall_map"]:
        _close(via_depth[k], via_maps[k], rtol=1e-3)
    assert np.abs(via_depth["dL_dall_map"]).max() > 0
