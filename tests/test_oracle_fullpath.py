"""Pinning the full-image path's oracle (GaussianRasterizer.forward /
render_simp / backward of diff-gaussian-rasterization_f).

* preprocess: with the split path's arguments (no culling, no precomputed
  colours or covariances, SH split into dc + rest) the outputs equal the split
  path's oracle bit for bit; culled rows are empty; precomputed colours leave
  everything but rgb unchanged; the precomputed 3D covariance equal to the
  computed one changes nothing; tiles_touched equals the float-rect area
  worked out in numpy.
* the tile test of duplicateWithKeys: a mean inside the tile keeps the tile
  iff opacity >= 1/255; for axis-aligned conics (b = 0) it keeps exactly the
  tiles whose pixel rect reaches exponent <= log(255 o) (closed form in
  float64); for any conic a kept tile truly reaches it somewhere in the rect.
* binning: keys, ids, ranges, valid count and bucket count equal a Python
  enumeration (padding, stable order, invalid tile skipped).
* render: colour, final T and contributor counts equal the split path's
  render on the same lists; accum_max_count sums to the number of covered
  pixels; render_simp's weights sum to sum(1 - T_final) and its counts to the
  number of contributions (the split oracle's independent counter).
* backward: without alpha clamping it equals the split path's backward; with
  clamping, the whole chain matches central finite differences of the float64
  twin (which differentiates min(0.99, o G) exactly); dL/dcov3D is consistent
  with dL/dscales through the covariance Jacobian.
"""
import numpy as np
import pytest

from blitzgs_amd import synth
from oracle import oracle as O
from oracle import ref64


def _split(sh):
    sh = np.asarray(sh, np.float32)
    return sh[:, :1], sh[:, 1:]


def _frect_area(m2d, ex, W, H):
    gx, gy = (W + 15) // 16, (H + 15) // 16
    f = np.float32
    c = lambda v, g: np.clip(v, 0, g)
    with np.errstate(invalid="ignore"):
        x0 = c(np.floor((m2d[:, 0] - ex[:, 0]) / f(16)), gx)
        y0 = c(np.floor((m2d[:, 1] - ex[:, 1]) / f(16)), gy)
        x1 = c(np.ceil((m2d[:, 0] + ex[:, 0]) / f(16)), gx)
        y1 = c(np.ceil((m2d[:, 1] + ex[:, 1]) / f(16)), gy)
    return ((x1 - x0) * (y1 - y0)).astype(np.int64)


@pytest.mark.parametrize("deg", [0, 1, 3])
def test_preprocess_full_equals_split_path(deg):
    scene, cam = synth.config0()
    dc, rest = _split(scene["sh"])
    a = O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                         scene["opacities"], sh_degree=deg)
    b = O.preprocess_fwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], dc, rest,
                              scene["opacities"], sh_degree=deg)
    for k in ["means2D", "depths", "radii", "cov3D", "conic_opacity", "rgb", "clamped"]:
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k
    vis = b["radii"] > 0
    assert vis.sum() > 1000
    area = _frect_area(b["means2D"], b["rects"], cam["W"], cam["H"])
    assert np.array_equal(b["tiles_touched"][vis].astype(np.int64), area[vis])
    assert not b["tiles_touched"][~vis].any() and not b["rects"][~vis].any()
    assert (b["rects"][vis] > 0).all()


def test_preprocess_full_culling_and_precomputed_inputs():
    scene, cam = synth.config0()
    dc, rest = _split(scene["sh"])
    args = (cam, scene["means3D"], scene["scales"], scene["rotations"], dc, rest, scene["opacities"])
    base = O.preprocess_fwd_full(*args)
    cull = np.zeros(len(base["radii"]), np.uint8)
    cull[::3] = 1
    c = O.preprocess_fwd_full(*args, culling=cull)
    keys = ["means2D", "depths", "radii", "cov3D", "conic_opacity", "rgb", "rects", "tiles_touched"]
    for k in keys:
        assert not c[k][cull == 1].any(), k
        assert np.array_equal(c[k][cull == 0], base[k][cull == 0]), k
    cols = np.random.default_rng(0).random((len(base["radii"]), 3)).astype(np.float32)
    p = O.preprocess_fwd_full(*args, colors_precomp=cols)
    assert not p["rgb"].any()
    for k in ["means2D", "depths", "radii", "cov3D", "conic_opacity", "rects", "tiles_touched"]:
        assert np.array_equal(p[k], base[k]), k
    q = O.preprocess_fwd_full(*args, cov3D_precomp=base["cov3D"])
    for k in ["means2D", "depths", "radii", "conic_opacity", "rgb", "rects", "tiles_touched"]:
        assert np.array_equal(q[k], base[k]), k


def _rect_min_exponent(xy, co, tx, ty):
    """Exact minimum over the continuous pixel rect of the tile of
    0.5 (a dx^2 + c dy^2) + b dx dy, float64 (convex: inside -> 0, else on an edge)."""
    a, b, c = (float(v) for v in co[:3])
    x0, x1 = 16.0 * tx, 16.0 * tx + 15.0
    y0, y1 = 16.0 * ty, 16.0 * ty + 15.0
    mx, my = float(xy[0]), float(xy[1])
    if x0 <= mx <= x1 and y0 <= my <= y1:
        return 0.0
    q = lambda x, y: 0.5 * (a * (mx - x) ** 2 + c * (my - y) ** 2) + b * (mx - x) * (my - y)
    best = np.inf
    for X in (x0, x1):   # vertical edges: minimise over y
        y = min(max(my + b * (mx - X) / c, y0), y1)
        best = min(best, q(X, y))
    for Y in (y0, y1):
        x = min(max(mx + b * (my - Y) / a, x0), x1)
        best = min(best, q(x, Y))
    return best


def test_tile_keep_closed_forms():
    rng = np.random.default_rng(3)
    checked_axis, checked_any = 0, 0
    for it in range(4000):
        tx, ty = int(rng.integers(0, 6)), int(rng.integers(0, 6))
        xy = rng.uniform(-20, 120, 2).astype(np.float32)
        a, c = np.exp(rng.uniform(-6, 0, 2))
        b = 0.0 if it % 2 == 0 else rng.uniform(-0.9, 0.9) * np.sqrt(a * c)
        o = np.float32(rng.uniform(0.001, 1.0))
        co = np.array([a, b, c, o], np.float32)
        keep = O.full_tile_keep(xy, co, tx, ty)
        thr = np.log(255.0 * float(o))
        m = _rect_min_exponent(xy, co, tx, ty)
        inside = 16 * tx <= xy[0] <= 16 * tx + 15 and 16 * ty <= xy[1] <= 16 * ty + 15
        if inside:
            assert keep == (thr >= -1e-6) or abs(thr) < 1e-5
        if abs(m - thr) < 1e-3 * (1.0 + abs(thr)):
            continue   # float rounding decides
        if b == 0.0:
            assert keep == (m <= thr), (xy, co, tx, ty, m, thr)
            checked_axis += 1
        elif keep:
            assert m <= thr, (xy, co, tx, ty, m, thr)
            checked_any += 1
    assert checked_axis > 1500 and checked_any > 200


def test_binning_full_matches_enumeration():
    scene, cam = synth.small_scene(300, seed=5, W=96, H=80, log_mu=-2.0)
    W, H = cam["W"], cam["H"]
    gx, gy = (W + 15) // 16, (H + 15) // 16
    dc, rest = _split(scene["sh"])
    pre = O.preprocess_fwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], dc, rest,
                                scene["opacities"])
    bn = O.binning_full(W, H, pre["means2D"], pre["depths"], pre["radii"], pre["rects"], pre["conic_opacity"],
                        pre["tiles_touched"])
    entries, pads = [], 0
    for i in range(len(pre["radii"])):
        if pre["radii"][i] <= 0:
            continue
        p, e = pre["means2D"][i], pre["rects"][i]
        x0 = int(np.clip(np.floor((p[0] - e[0]) / np.float32(16)), 0, gx))
        y0 = int(np.clip(np.floor((p[1] - e[1]) / np.float32(16)), 0, gy))
        x1 = int(np.clip(np.ceil((p[0] + e[0]) / np.float32(16)), 0, gx))
        y1 = int(np.clip(np.ceil((p[1] + e[1]) / np.float32(16)), 0, gy))
        n = 0
        for y in range(y0, y1):
            for x in range(x0, x1):
                if O.full_tile_keep(p, pre["conic_opacity"][i], x, y):
                    entries.append(((y * gx + x) << 32 | int(pre["depths"][i:i + 1].view(np.uint32)[0]), i))
                    n += 1
        pads += int(pre["tiles_touched"][i]) - n
    assert pads > 0 and len(entries) > 500
    entries.sort(key=lambda kv: kv[0])      # stable: Gaussian order breaks ties
    R = len(entries) + pads
    assert bn["R"] == R and bn["valid"] == len(entries)
    assert np.array_equal(bn["keys"][:len(entries)], np.array([k for k, _ in entries], np.uint64))
    assert np.array_equal(bn["point_list"][:len(entries)], np.array([v for _, v in entries], np.uint32))
    assert (bn["keys"][len(entries):] == np.uint64(0xFFFFFFFF7F7FFFFF)).all()
    assert (bn["point_list"][len(entries):] == 0xFFFFFFFF).all()
    ranges = np.zeros((gx * gy, 2), np.int64)
    tiles = np.array([k >> 32 for k, _ in entries])
    for t in range(gx * gy):
        idx = np.flatnonzero(tiles == t)
        if idx.size:
            ranges[t] = (idx[0], idx[-1] + 1)
    assert np.array_equal(bn["ranges"].astype(np.int64), ranges)
    assert bn["num_buckets"] == int(((ranges[:, 1] - ranges[:, 0] + 31) // 32).sum())


def test_render_full_matches_split_render_and_counters():
    scene, cam = synth.config0()
    bg = np.array([0.2, 0.3, 0.1], np.float32)
    pre, bn, rf = O.full_path_forward(cam, scene, bg=bg)
    W, H = cam["W"], cam["H"]
    rs = O.render_fwd(W, H, bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"], bn["point_list"])
    for a, b in [("color", "color"), ("final_T", "final_T"), ("n_contrib_px", "n_contrib_px")]:
        assert np.array_equal(rf[a].view(np.uint32), rs[b].view(np.uint32)), a
    covered = int((rf["n_contrib_px"] > 0).sum())
    assert rf["accum_max_count"].sum() == covered
    assert np.isin(np.flatnonzero(rf["accum_max_count"]), bn["point_list"][:bn["valid"]]).all()
    gx = (W + 15) // 16
    mc = np.zeros_like(rf["max_contrib"])
    for t in range(len(mc)):
        tx, ty = t % gx, t // gx
        mc[t] = rf["n_contrib_px"][ty * 16:ty * 16 + 16, tx * 16:tx * 16 + 16].max()
    assert np.array_equal(rf["max_contrib"], mc)
    _, _, off = O.full_path_forward(cam, scene, bg=bg, flag_max_count=False)
    assert not off["accum_max_count"].any()
    _, _, sp = O.full_path_forward(cam, scene, bg=bg, simp=True)
    assert np.array_equal(sp["color"], rf["color"]) and np.array_equal(sp["accum_max_count"], rf["accum_max_count"])
    assert sp["accum_weights_count"].sum() == int(rs["n_contrib2loss_px"].astype(np.int64).sum())
    np.testing.assert_allclose(sp["accum_weights"].astype(np.float64).sum(),
                               (1.0 - rf["final_T"].astype(np.float64)).sum(), rtol=1e-5)


def test_single_gaussian_max_count_is_its_footprint():
    scene, cam = synth.small_scene(1, seed=2, W=64, H=64, extent=0.0, log_mu=-1.5, log_sd=0.0)
    pre, bn, rf = O.full_path_forward(cam, scene)
    assert rf["accum_max_count"][0] == int((rf["n_contrib_px"] > 0).sum()) > 50


def _fd_scene(seed):
    scene, cam = synth.small_scene(14, seed=seed, W=32, H=32, extent=0.6, log_mu=-2.3, log_sd=0.3)
    scene["opacities"] = np.clip(scene["opacities"], 0.05, 0.85)
    return scene, cam


def _full_chain(cam, scene, bg, dLd, **kw):
    pre, bn, rf = O.full_path_forward(cam, scene, bg=bg, **kw)
    W, H = cam["W"], cam["H"]
    colors = pre["rgb"] if kw.get("colors_precomp") is None else kw["colors_precomp"]
    rb = O.render_bwd_full(W, H, bg, pre["means2D"], pre["conic_opacity"], colors, bn["ranges"], bn["point_list"],
                           rf["final_T"], rf["n_contrib_px"], dLd)
    dc, rest = _split(scene["sh"])
    pb = O.preprocess_bwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], dc, rest, pre["radii"],
                               pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic"], rb["dL_dcolors"],
                               colors_precomp=kw.get("colors_precomp"), cov3D_precomp=kw.get("cov3D_precomp"))
    return pre, bn, rf, rb, pb


def test_backward_full_equals_split_without_clamping():
    scene, cam = _fd_scene(1)
    bg = np.array([0.3, 0.1, 0.2], np.float32)
    dLd = np.random.default_rng(1).standard_normal((3, cam["H"], cam["W"])).astype(np.float32)
    pre, bn, rf, rb, pb = _full_chain(cam, scene, bg, dLd)
    rs = O.render_bwd(cam["W"], cam["H"], bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"],
                      bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd)
    for k in ["dL_dmeans2D", "dL_dconic", "dL_dopacity", "dL_dcolors"]:
        np.testing.assert_allclose(rb[k], rs[k], rtol=1e-5, atol=1e-7, err_msg=k)
    ps = O.preprocess_bwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"], pre["radii"],
                          pre["cov3D"], pre["clamped"], rs["dL_dmeans2D"], rs["dL_dconic_opacity"], rs["dL_dcolors"])
    np.testing.assert_allclose(pb["dL_dmeans3D"], ps["dL_dmeans3D"], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(pb["dL_dscales"], ps["dL_dscales"], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(pb["dL_drotations"], ps["dL_drotations"], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(pb["dL_ddc"][:, 0], ps["dL_dsh"][:, 0], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(pb["dL_dsh"], ps["dL_dsh"][:, 1:], rtol=1e-4, atol=1e-7)


def _loss64(cam, sc, bg, ranges, plist, dLd):
    pr = ref64.project(cam, sc["means3D"], sc["scales"], sc["rotations"], sc["opacities"], sc["sh"])
    img, _, sig = ref64.render(cam["W"], cam["H"], bg, pr["means2D"], pr["conic"], pr["opacity"], pr["rgb"],
                               ranges, plist, signature=True)
    return float((img * dLd).sum()), sig


@pytest.mark.parametrize("seed", [3, 5])
def test_backward_full_with_clamping_matches_finite_differences(seed):
    scene, cam = synth.small_scene(12, seed=seed, W=32, H=32, extent=0.5, log_mu=-1.2, log_sd=0.3)
    scene["opacities"] = np.clip(scene["opacities"], 0.05, 0.85)
    scene["opacities"][::2] = 0.9995        # o * G > 0.99 near these means: alpha clamps
    bg = np.array([0.3, 0.1, 0.2], np.float32)
    dLd = np.random.default_rng(seed).standard_normal((3, cam["H"], cam["W"]))
    pre, bn, rf, rb, pb = _full_chain(cam, scene, bg, dLd.astype(np.float32))
    assert (pre["radii"] > 0).all()
    valid = bn["valid"]
    ranges, plist = bn["ranges"], bn["point_list"][:valid]
    # the conic / opacity / colour paths; the mean's screen-space gradient keeps
    # the clamped pixels' terms by the reference's rule (backward.cu:548-557
    # come before the clamp test), so means3D is not a finite-difference case here
    groups = {"opacities": ("dL_dopacity", 1e-5), "scales": ("dL_dscales", 1e-6),
              "rotations": ("dL_drotations", 1e-5), "sh": ("dL_dsh_all", 1e-4)}
    base = {k: np.asarray(v, np.float64) for k, v in scene.items() if k in ("means3D", "scales", "rotations",
                                                                           "opacities", "sh")}
    ana_all = {"dL_dscales": pb["dL_dscales"], "dL_dopacity": rb["dL_dopacity"],
               "dL_drotations": pb["dL_drotations"],
               "dL_dsh_all": np.concatenate([pb["dL_ddc"], pb["dL_dsh"]], axis=1)}
    skipped = 0
    for name, (gname, h) in groups.items():
        ana = ana_all[gname].reshape(-1).astype(np.float64)
        fd = np.zeros_like(ana)
        keep = np.ones_like(ana, bool)
        flat = base[name].reshape(-1)
        for i in range(flat.size):
            sc = dict(base)
            p = flat.copy(); p[i] += h
            sc[name] = p.reshape(base[name].shape)
            lp, sp = _loss64(cam, sc, bg, ranges, plist, dLd)
            p[i] -= 2 * h
            sc[name] = p.reshape(base[name].shape)
            lm, sm = _loss64(cam, sc, bg, ranges, plist, dLd)
            fd[i] = (lp - lm) / (2 * h)
            keep[i] = sp == sm
        skipped += int((~keep).sum())
        err = np.linalg.norm(ana[keep] - fd[keep]) / max(np.linalg.norm(fd[keep]), 1e-12)
        assert err < 1e-3, (name, err)
    assert skipped < 10
    # Gaussians whose opacity * G exceeds 0.99 at the pixel centre nearest the mean
    m2d, co = pre["means2D"].astype(np.float64), pre["conic_opacity"].astype(np.float64)
    d = m2d - np.round(m2d)
    G = np.exp(-0.5 * (co[:, 0] * d[:, 0] ** 2 + co[:, 2] * d[:, 1] ** 2) - co[:, 1] * d[:, 0] * d[:, 1])
    clamped = co[:, 3] * G > 0.99
    assert clamped.any()
    # where the clamp acts, the split path's rule (no clamp skip) gives other opacity gradients
    rs = O.render_bwd(cam["W"], cam["H"], bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], ranges,
                      bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd.astype(np.float32))
    assert not np.allclose(rs["dL_dopacity"][clamped], rb["dL_dopacity"][clamped], rtol=1e-3)


def test_dL_dcov3D_consistent_with_scale_gradient():
    scene, cam = _fd_scene(6)
    bg = np.zeros(3, np.float32)
    dLd = np.random.default_rng(6).standard_normal((3, cam["H"], cam["W"])).astype(np.float32)
    pre, bn, rf, rb, pb = _full_chain(cam, scene, bg, dLd)
    q = O.preprocess_bwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], *_split(scene["sh"]),
                              pre["radii"], pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic"],
                              rb["dL_dcolors"], cov3D_precomp=pre["cov3D"])
    assert np.array_equal(q["dL_dcov3D"], pb["dL_dcov3D"])
    assert not q["dL_dscales"].any() and not q["dL_drotations"].any()
    # d cov3D / d scale in float64 (cov = R diag(s^2) R^T, six unique entries, off-diagonals once)
    R = ref64.quat_to_rot(np.asarray(scene["rotations"], np.float64))
    s = np.asarray(scene["scales"], np.float64)
    iu = [(0, 0), (0, 1), (0, 2), (1, 1), (1, 2), (2, 2)]
    for i in range(len(s)):
        J = np.zeros((6, 3))
        for k in range(3):
            dS = np.zeros(3); dS[k] = 2 * s[i, k]
            dcov = R[i] @ np.diag(dS) @ R[i].T
            J[:, k] = [dcov[a, b] for a, b in iu]
        expect = J.T @ pb["dL_dcov3D"][i].astype(np.float64)
        np.testing.assert_allclose(pb["dL_dscales"][i], expect, rtol=2e-3, atol=1e-6)


# ------------------------------------------------------------------ render_depth

def _proj_colmajor(cam):
    """The matrix the kernels see: element (r, c) is projmatrix's flat entry 4c + r."""
    return np.asarray(cam["projmatrix"], np.float64).reshape(4, 4).T


def test_inverse_projection_matches_numpy():
    for cam in (synth.small_scene(1, seed=0)[1], synth.config0()[1], synth.aerial_camera(1600, 1066)):
        got = O.inv4_colmajor(cam["projmatrix"]).astype(np.float64).reshape(4, 4).T
        ref = np.linalg.inv(_proj_colmajor(cam))
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6 * np.abs(ref).max())


def _rays64(cam):
    """Per-pixel rays in float64: the point inv(M) (ndc.x, ndc.y, z, 1) (no
    division by w) minus the camera centre.  For znear 0.01 / zfar 100 the
    reference's z constant is the NDC depth of view depth 1, where w = 1."""
    W, H = int(cam["W"]), int(cam["H"])
    Minv = np.linalg.inv(_proj_colmajor(cam))
    ys, xs = np.mgrid[0:H, 0:W].astype(np.float64)
    ndx = (2 * xs + 1) / W - 1
    ndy = (2 * ys + 1) / H - 1
    h = np.stack([ndx * 1.0000001, ndy * 1.0000001, np.full_like(ndx, 99.0 / 99.99), np.ones_like(ndx)], -1)
    p = h @ Minv.T
    np.testing.assert_allclose(p[..., 3], 1.0, atol=1e-5)
    return p[..., :3] - np.asarray(cam["campos"], np.float64)


def _ellipsoid_hit64(cam, mu, q, s):
    """Closest approach of every pixel ray to the Gaussian's 3-sigma ellipsoid,
    from the quadric x^T A x = 1 with A = R diag(1/(3 s)^2) R^T (R the
    textbook rotation of q): t = -b / 2a along the unit ray, depth = t / |ray|,
    discriminant b^2 - 4ac, hit point c + t n."""
    d = _rays64(cam)
    L = np.linalg.norm(d, axis=-1)
    n = d / L[..., None]
    R = ref64.quat_to_rot(np.asarray(q, np.float64))
    A = R @ np.diag(1.0 / (3.0 * np.asarray(s, np.float64)) ** 2) @ R.T
    o = np.asarray(cam["campos"], np.float64) - np.asarray(mu, np.float64)
    a = np.einsum("hwi,ij,hwj->hw", n, A, n)
    b = 2 * np.einsum("hwi,ij,j->hw", n, A, o)
    c = o @ A @ o - 1
    t = -b / (2 * a)
    return t / L, b * b - 4 * a * c, np.asarray(cam["campos"], np.float64) + t[..., None] * n, b * b + abs(4 * a * c)


def _one_gaussian(mu, q, s, opacity, W=32, H=24):
    scene, cam = synth.small_scene(1, seed=9, W=W, H=H)
    scene["means3D"] = np.array([mu], np.float32)
    scene["rotations"] = np.array([q], np.float32)
    scene["scales"] = np.array([s], np.float32)
    scene["opacities"] = np.array([[opacity]], np.float32)
    return scene, cam


def test_depth_single_anisotropic_gaussian_closed_form():
    q = np.array([0.8, 0.3, -0.4, 0.2])                    # unnormalised on purpose
    s = [1.2, 0.5, 0.3]
    scene, cam = _one_gaussian([0.1, -0.05, 0.5], q, s, 0.9)
    pre, bn, rd = O.full_path_depth(cam, scene)
    hit = rd["accum_alpha"][0] < 1.0
    assert hit.sum() > 100
    depth, disc, pts, scale = _ellipsoid_hit64(cam, scene["means3D"][0], scene["rotations"][0].astype(np.float64),
                                               s)
    # The ray's float construction cancels terms of size ~1/znear = 100 (the
    # inverse projection applied at NDC depth 0.990099 to give w = 1), so a
    # float32 ray carries relative errors of a few 1e-5 against this float64
    # one -- as the reference's float glm::inverse does.  A formula mistake
    # (transposed rotation, missing factor 3, wrong ray normalisation) moves
    # the depths by far more (checked below for the rotation).
    np.testing.assert_allclose(rd["depth"][0][hit], depth[hit], rtol=1e-4)
    np.testing.assert_allclose(rd["out_pts"][:, hit].T, pts[hit], rtol=1e-4, atol=1e-4)
    assert np.all(np.abs(rd["discriminants"][0][hit] - disc[hit]) <= 1e-3 * scale[hit])
    assert np.all(rd["gidx"][0] == 0)
    assert np.all(rd["depth"][0][~hit] == 0) and np.all(rd["out_pts"][:, ~hit] == 0)
    # a wrongly transposed rotation gives another ellipsoid
    bad, _, _, _ = _ellipsoid_hit64(cam, scene["means3D"][0], q * np.array([1, -1, -1, -1]), s)
    assert np.abs(bad[hit] - depth[hit]).max() > 1e-2


def test_depth_negative_ray_parameter_keeps_transmittance():
    """A large Gaussian off to the side: on the right of the image the ray's
    closest approach lies behind the camera (depth < 0).  There its colour is
    added but T, depth, id and hit point stay untouched."""
    scene, cam = _one_gaussian([-3.0, 0.0, -3.5], [1, 0, 0, 0], [2.0, 2.0, 2.0], 0.9)
    pre, bn, rd = O.full_path_depth(cam, scene)
    rf = O.full_path_forward(cam, scene)[2]
    depth, _, _, _ = _ellipsoid_hit64(cam, scene["means3D"][0], [1, 0, 0, 0], [2.0, 2.0, 2.0])
    contributed = rf["n_contrib_px"] > 0
    neg = contributed & (depth < -1e-4)
    pos = contributed & (depth > 1e-4)
    assert neg.sum() > 50 and pos.sum() > 50
    assert np.all(rd["accum_alpha"][0][neg] == 1.0) and np.all(rd["depth"][0][neg] == 0)
    assert np.all(rd["out_pts"][:, neg] == 0)
    # colour = rgb * alpha with T = 1: the forward's colour there (one contribution, T = 1 before it)
    np.testing.assert_allclose(rd["color"][:, neg], rf["color"][:, neg], rtol=1e-6, atol=1e-7)
    assert np.all(rd["accum_alpha"][0][pos] == rf["final_T"][pos]) and np.all(rd["depth"][0][pos] > 0)


def test_depth_render_agrees_with_forward_on_a_scene():
    """On a scene in front of the camera (every depth positive) the depth
    render's T equals the forward's final T bit for bit, its colour to
    rounding, and counting each covered pixel's gidx reproduces the forward's
    accum_max_count (the same arg-max of alpha * T)."""
    scene, cam = synth.small_scene(400, seed=4, W=64, H=48, extent=0.8, log_mu=-2.2)
    pre, bn, rd = O.full_path_depth(cam, scene)
    rf = O.full_path_forward(cam, scene, flag_max_count=True)[2]
    assert np.array_equal(rd["accum_alpha"][0], rf["final_T"])
    np.testing.assert_allclose(rd["color"], rf["color"], rtol=1e-5, atol=1e-6)
    covered = rf["n_contrib_px"] > 0
    counts = np.bincount(rd["gidx"][0][covered], minlength=400).astype(np.float32)
    assert np.array_equal(counts, rf["accum_max_count"])
    assert np.all(rd["depth"][0][covered] > 0)
