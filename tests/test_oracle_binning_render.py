"""Pin the oracle's binning against a brute-force restatement and its render
forward against the float64 twin and closed forms."""
import math

import numpy as np

from blitzgs_amd import synth
from oracle import oracle as O
from oracle import ref64


def brute_force_binning(W, H, means2D, depths, radii, compute_locally):
    """Enumerate each Gaussian's square tile rect (getRect with an integer
    radius, _r auxiliary.h:66-76) and sort the instances by
    (tile, depth bits, Gaussian index) -- the order a stable sort of the
    duplicated keys produces."""
    gx, gy = (W + 15) // 16, (H + 15) // 16
    cl = compute_locally.reshape(-1)
    inst = []
    f32 = np.float32
    for i in range(len(radii)):
        r = int(radii[i])
        if r <= 0:
            continue
        px, py = f32(means2D[i, 0]), f32(means2D[i, 1])
        rf = f32(r)

        def clampi(v, g):
            v = int(np.trunc(v)) if np.isfinite(v) else 0
            return min(g, max(0, v))
        x0 = clampi((px - rf) / f32(16), gx)
        y0 = clampi((py - rf) / f32(16), gy)
        x1 = clampi(((px + rf) + f32(16) - f32(1)) / f32(16), gx)
        y1 = clampi(((py + rf) + f32(16) - f32(1)) / f32(16), gy)
        db = int(np.float32(depths[i]).view(np.uint32))
        for y in range(y0, y1):
            for x in range(x0, x1):
                t = y * gx + x
                if cl[t]:
                    inst.append((t, db, i))
    inst.sort()
    keys = np.array([(t << 32) | d for t, d, _ in inst], np.uint64)
    vals = np.array([i for _, _, i in inst], np.uint32)
    ranges = np.zeros((gx * gy, 2), np.uint32)
    for k, (t, _, _) in enumerate(inst):
        if k == 0 or inst[k - 1][0] != t:
            ranges[t, 0] = k
        ranges[t, 1] = k + 1
    return keys, vals, ranges


def _pre(scene, cam):
    return O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                            scene["opacities"])


def test_binning_matches_brute_force_full_and_masked():
    scene, cam = synth.small_scene(1500, seed=21, W=150, H=100, extent=1.5)
    pre = _pre(scene, cam)
    # force depth ties: equal depth bits must keep ascending Gaussian index
    pre["depths"][10:20] = pre["depths"][10]
    gx, gy = (cam["W"] + 15) // 16, (cam["H"] + 15) // 16
    rng = np.random.default_rng(0)
    for cl in [np.ones(gx * gy, np.uint8), (rng.random(gx * gy) < 0.5).astype(np.uint8),
               np.zeros(gx * gy, np.uint8)]:
        bn = O.binning(cam["W"], cam["H"], pre["means2D"], pre["depths"], pre["radii"], cl)
        k, v, r = brute_force_binning(cam["W"], cam["H"], pre["means2D"], pre["depths"], pre["radii"], cl)
        assert bn["R"] == len(k)
        np.testing.assert_array_equal(bn["keys"], k)
        np.testing.assert_array_equal(bn["point_list"], v)
        np.testing.assert_array_equal(bn["ranges"], r)


def test_binning_edge_cases():
    W, H = 40, 33   # ragged last tile row/column
    gx, gy = 3, 3
    means2D = np.array([[-1000.0, 5.0], [5.0, 5.0], [39.5, 32.9], [np.nan, 1.0], [1e12, 1e12],
                        [20.0, 20.0], [20.0, 20.0]], np.float32)
    radii = np.array([5, 0, 3, 4, 7, 100, 1], np.int32)
    depths = np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 6.0], np.float32)
    cl = np.ones(gx * gy, np.uint8)
    bn = O.binning(W, H, means2D, depths, radii, cl)
    k, v, r = brute_force_binning(W, H, means2D, depths, radii, cl)
    np.testing.assert_array_equal(bn["keys"], k)
    np.testing.assert_array_equal(bn["point_list"], v)
    np.testing.assert_array_equal(bn["ranges"], r)
    # empty input
    bn = O.binning(W, H, np.zeros((0, 2), np.float32), np.zeros(0, np.float32), np.zeros(0, np.int32), cl)
    assert bn["R"] == 0 and not bn["ranges"].any()


def test_sub_image_ranges_equal_full_image_restricted():
    # one rank's contiguous block of tile rows renders exactly the full image's
    # instances for those tiles, shifted by a constant offset
    scene, cam = synth.small_scene(3000, seed=8, W=128, H=160, extent=1.5)
    pre = _pre(scene, cam)
    gx, gy = 8, 10
    full = O.binning(cam["W"], cam["H"], pre["means2D"], pre["depths"], pre["radii"])
    lo, hi = synth.tile_row_block(gy, 4, 1)
    cl = np.zeros((gy, gx), np.uint8)
    cl[lo:hi] = 1
    sub = O.binning(cam["W"], cam["H"], pre["means2D"], pre["depths"], pre["radii"], cl)
    t0, t1 = lo * gx, hi * gx
    off = full["ranges"][t0, 0]
    np.testing.assert_array_equal(sub["ranges"][t0:t1], full["ranges"][t0:t1] - off)
    assert not sub["ranges"][:t0].any() and not sub["ranges"][t1:].any()
    np.testing.assert_array_equal(sub["point_list"], full["point_list"][full["ranges"][t0, 0]:full["ranges"][t1 - 1, 1]])


def test_render_matches_float64_twin_and_invariants():
    scene, cam = synth.small_scene(800, seed=4, W=96, H=64, extent=1.2, log_mu=-2.2)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    pre, bn, rf = O.full_forward(cam, scene, bg=bg)
    proj = ref64.project(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["opacities"],
                         scene["sh"])
    img, T = ref64.render(cam["W"], cam["H"], bg, proj["means2D"], proj["conic"], proj["opacity"],
                          proj["rgb"], bn["ranges"], bn["point_list"])
    diff = np.abs(rf["color"] - img)
    # float64 vs fp32: thresholds (alpha < 1/255, T < 1e-4) may flip at a few pixels
    assert np.quantile(diff, 0.999) < 1e-4
    assert (diff > 1e-4).mean() < 0.002
    assert (rf["final_T"] > 0).all() and (rf["final_T"] <= 1).all()
    # colour <= max rgb * (1 - T) + T * bg
    cmax = pre["rgb"].max()
    assert (rf["color"] <= cmax * (1 - rf["final_T"]) + rf["final_T"] * bg[:, None, None] + 1e-5).all()
    # stats: n_render = range length; n_consider / n_contrib = per-tile sums
    np.testing.assert_array_equal(rf["n_render"], (bn["ranges"][:, 1] - bn["ranges"][:, 0]).astype(np.int32))
    gx = (cam["W"] + 15) // 16
    t = 5
    ty, tx = divmod(t, gx)
    blk = (slice(ty * 16, ty * 16 + 16), slice(tx * 16, tx * 16 + 16))
    assert rf["n_consider"][t] == rf["n_contrib_px"][blk].sum()
    assert rf["n_contrib"][t] == rf["n_contrib2loss_px"][blk].sum()
    assert (rf["n_contrib2loss_px"] <= rf["n_contrib_px"]).all()


def test_render_single_gaussian_closed_form():
    # one Gaussian, bg = 0: C(p) = rgb * min(0.99, o exp(power(p))) wherever alpha >= 1/255
    W, H = 48, 48
    means2D = np.array([[20.3, 25.7]], np.float32)
    conic = np.array([[0.05, 0.01, 0.08, 0.7]], np.float32)
    rgb = np.array([[0.2, 0.5, 0.9]], np.float32)
    ranges = np.zeros((9, 2), np.uint32)
    ranges[:] = [0, 1]
    point_list = np.zeros(9, np.uint32)
    rf = O.render_fwd(W, H, np.zeros(3, np.float32), means2D, conic, rgb, ranges, point_list)
    y, x = np.mgrid[0:H, 0:W].astype(np.float64)
    dx, dy = 20.3 - x, 25.7 - y
    power = -0.5 * (0.05 * dx * dx + 0.08 * dy * dy) - 0.01 * dx * dy
    alpha = np.minimum(0.99, 0.7 * np.exp(power))
    alpha[alpha < 1 / 255] = 0
    np.testing.assert_allclose(rf["color"], rgb[0][:, None, None] * alpha[None], atol=2e-6)
    np.testing.assert_allclose(rf["final_T"], 1 - alpha, atol=2e-6)
    assert rf["out_observe"][0] == (alpha > 0).sum()   # T = 1 > 0.5 at every blended pixel


def test_render_early_termination():
    # a stack of opaque Gaussians: each pixel stops when T would drop below 1e-4
    W, H = 16, 16
    n = 8
    means2D = np.tile(np.array([[7.5, 7.5]], np.float32), (n, 1))
    conic = np.tile(np.array([[1e-4, 0.0, 1e-4, 0.95]], np.float32), (n, 1))
    rgb = np.random.default_rng(0).random((n, 3)).astype(np.float32)
    ranges = np.array([[0, n]], np.uint32)
    rf = O.render_fwd(W, H, np.zeros(3, np.float32), means2D, conic, rgb, ranges, np.arange(n, dtype=np.uint32))
    # alpha ~0.95 at the centre: T = 0.05^k; 0.05^3 = 1.25e-4, 0.05^4 < 1e-4 -> 3 blended
    c = (7, 7)
    assert rf["n_contrib2loss_px"][c] == 3 and rf["n_contrib_px"][c] == 3
    assert 1e-4 <= rf["final_T"][c] < 2e-4
