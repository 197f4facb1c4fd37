"""HIP path vs CPU oracle, through the C ABI, on seeded synthetic scenes.

Bar: bit-exact for the per-Gaussian preprocess outputs and the tile instance
lists (sorted ids, keys, ranges); the blend's image and transmittance within
1e-4 max-abs and its counts equal up to rare threshold cases (the blend's exp
is the hardware exp2, see gpu_helpers); gradients within 1e-3 relative L2 of
the oracle (float atomics reorder the sums)."""
import numpy as np
import pytest
import torch

from blitzgs_amd import synth, _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu

from tests.gpu_helpers import (assert_bitexact, assert_blend_counts, assert_close_abs, gpu_preprocess,
                               gpu_render_forward, np_, rel_l2, settings_for, to_dev)


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    _lib.load()
    yield


def _oracle_pre(scene, cam, deg=3):
    return O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                            scene["opacities"], sh_degree=deg)


def test_device_math_bitexact():
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-87.5, 0.0, 400_001), rng.uniform(-100, 90, 200_000),
                        [0.0, -0.0, -87.0, -87.00001, 88.5, 89.0, np.nan, -np.inf]]).astype(np.float32)
    xt = to_dev(x)
    for op, ref in ((0, O.vec_expf(x)), (2, O.vec_expf(x))):
        y = torch.empty_like(xt)
        _lib.check(_lib.load().gs_diag_math(op, x.size, _lib.ptr(xt), _lib.ptr(y), None), "diag")
        torch.cuda.synchronize()
        assert_bitexact(np_(y), ref, f"exp op{op}")
    xl = np.concatenate([rng.uniform(1.0, 256.0, 300_000), np.exp(rng.uniform(-80, 80, 100_000)),
                         [0.0, 1.0, -1.0, np.inf, np.nan, 1e-40]]).astype(np.float32)
    xt = to_dev(xl)
    y = torch.empty_like(xt)
    _lib.check(_lib.load().gs_diag_math(1, xl.size, _lib.ptr(xt), _lib.ptr(y), None), "diag")
    torch.cuda.synchronize()
    assert_bitexact(np_(y), O.vec_logf(xl), "log")


def test_valu_probes_run_and_write_nothing():
    """The blend kernels' VALU probes (gs_diag_math ops 7, 8 and 9: forward,
    quadrant backward, half-tile backward) run, and the float they could
    write stays untouched (the work is kept alive by a test that never
    holds)."""
    y = torch.zeros(1, device="cuda")
    for op in (7, 8, 9):
        _lib.check(_lib.load().gs_diag_math(op, 1, None, _lib.ptr(y), None), f"probe op {op}")
    torch.cuda.synchronize()
    assert float(y[0]) == 0.0


def test_blend_falloff_exp_bound_and_guard():
    """The blend's G (op 6, opacity 1): within 2e-5 relative of exp(x) in
    double over [-87, 0], and bit-equal to the oracle's exact exp for every x
    within 2.5e-5 of the alpha cut-off log(1/255) (the guard window is 3e-5
    around -logf(255)), so the alpha >= 1/255 decision is the exact one."""
    rng = np.random.default_rng(6)
    c = np.log(1.0 / 255.0)
    x = np.concatenate([np.linspace(-87.0, 0.0, 300_001), rng.uniform(-20, 0, 200_000),
                        c + rng.uniform(-5e-5, 5e-5, 100_000)]).astype(np.float32)
    xt = to_dev(x)
    y = torch.empty_like(xt)
    _lib.check(_lib.load().gs_diag_math(6, x.size, _lib.ptr(xt), _lib.ptr(y), None), "diag blend G")
    torch.cuda.synchronize()
    g = np_(y).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert (np.abs(g - ref) <= 2e-5 * ref + 1e-38).all()
    inside = np.abs(x.astype(np.float64) - c) <= 2.5e-5
    assert inside.sum() > 1000
    assert_bitexact(np_(y)[inside], O.vec_expf(x)[inside], "exact exp around the alpha cut-off")


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_preprocess_forward_bitexact(deg):
    scene, cam = synth.small_scene(20000, seed=31 + deg, W=320, H=200, extent=2.0, cam_dist=3.0)
    rs = settings_for(cam, sh_degree=deg)
    g = gpu_preprocess(scene, rs)
    o = _oracle_pre(scene, cam, deg)
    for k in ["means2D", "depths", "radii", "cov3D", "conic_opacity", "rgb"]:
        assert_bitexact(np_(g[k]), o[k], k)
    assert_bitexact(np_(g["clamped"]).astype(np.uint8), o["clamped"], "clamped")
    vis = o["radii"] > 0
    assert 0 < vis.sum() < len(vis)   # both culled and visible Gaussians covered


def test_preprocess_forward_config0_and_edge_inputs():
    scene, cam = synth.config0()
    # edge inputs: behind the camera, zero / tiny / >1 opacity, degenerate scale, huge scale
    scene["means3D"][:4] = [[0, 0, -5.0], [0, 0, -3.9], [0.1, 0.1, 0.0], [0.0, 0.0, 1.0]]
    scene["opacities"][4:8, 0] = [0.0, 1e-4, 1.0 / 255.0, 1.5]
    scene["scales"][8] = 0.0
    scene["scales"][9] = 1e3
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    o = _oracle_pre(scene, cam)
    for k in ["means2D", "depths", "radii", "cov3D", "conic_opacity", "rgb"]:
        assert_bitexact(np_(g[k]), o[k], k)


def _check_binning_and_render(cam, pre, bg, cl=None):
    rs = settings_for(cam, bg=bg)
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    g = gpu_render_forward(rs, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], cl)
    ob = O.binning(cam["W"], cam["H"], pre["means2D"], pre["depths"], pre["radii"], cl)
    assert g["R"] == ob["R"]
    assert_bitexact(np_(g["point_list"]).view(np.uint32), ob["point_list"], "point_list")
    assert_bitexact(np_(g["keys"]).view(np.uint64), ob["keys"], "point_list_keys")
    assert_bitexact(np_(g["ranges"]).view(np.uint32), ob["ranges"], "ranges")
    orf = O.render_fwd(cam["W"], cam["H"], np.asarray(bg, np.float32), pre["means2D"], pre["conic_opacity"],
                       pre["rgb"], ob["ranges"], ob["point_list"], cl)
    assert_bitexact(np_(g["n_render"]), orf["n_render"], "n_render")
    assert_close_abs(np_(g["color"]), orf["color"], "color")
    assert_close_abs(np_(g["final_T"]), orf["final_T"], "final_T")
    assert_blend_counts(dict(n_contrib_px=np_(g["n_contrib_px"]).view(np.uint32),
                             n_contrib2loss_px=np_(g["n_contrib2loss_px"]).view(np.uint32),
                             out_observe=np_(g["out_observe"]), n_consider=np_(g["n_consider"]),
                             n_contrib=np_(g["n_contrib"])), orf)
    return g, ob, orf


def test_binning_and_render_forward_bitexact_config0():
    scene, cam = synth.config0()
    pre = _oracle_pre(scene, cam)
    _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))


def test_binning_render_ragged_masked_and_ties():
    scene, cam = synth.small_scene(6000, seed=77, W=250, H=170, extent=1.8, log_mu=-2.0)
    pre = _oracle_pre(scene, cam)
    pre["depths"][100:160] = pre["depths"][100]          # depth ties -> ascending id order
    gx, gy = (250 + 15) // 16, (170 + 15) // 16
    rng = np.random.default_rng(5)
    for cl in [None, (rng.random((gy, gx)) < 0.4).astype(np.uint8), np.zeros((gy, gx), np.uint8)]:
        _check_binning_and_render(cam, pre, (0.2, 0.5, 0.9), cl)


def test_binning_every_sort_size_class():
    # A Gaussian of radius 1 at a tile centre lands in exactly that tile, so the
    # bucket sizes below are exact: they straddle every boundary of the on-chip
    # sort classes (512 / 1024 / 2048 / 4096 / 8192 keys) and exceed the largest
    # (the global-memory path).  Depths are drawn from a small set (many ties ->
    # ascending id order) plus a continuous range.
    sizes = [1, 2, 63, 64, 65, 511, 512, 513, 1023, 1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097,
             8191, 8192, 8193, 10000]
    gx = 8
    W, H = gx * 16, ((len(sizes) + gx - 1) // gx) * 16
    rng = np.random.default_rng(21)
    xs, ys = [], []
    for t, n in enumerate(sizes):
        xs.append(np.full(n, (t % gx) * 16 + 8.0))
        ys.append(np.full(n, (t // gx) * 16 + 8.0))
    P = sum(sizes)
    order = rng.permutation(P)          # interleave the tiles' Gaussians in id order
    means2D = np.stack([np.concatenate(xs)[order], np.concatenate(ys)[order]], 1).astype(np.float32)
    radii = np.ones(P, np.int32)
    depths = np.where(rng.random(P) < 0.5, rng.integers(1, 6, P).astype(np.float32),
                      rng.uniform(0.3, 40.0, P)).astype(np.float32)
    conic = np.tile(np.array([[0.3, 0.0, 0.3, 0.02]], np.float32), (P, 1))
    rgb = rng.random((P, 3)).astype(np.float32)
    cam = dict(W=W, H=H, tanfovx=1.0, tanfovy=1.0, viewmatrix=np.eye(4, dtype=np.float32),
               projmatrix=np.eye(4, dtype=np.float32), campos=np.zeros(3, np.float32))
    pre = dict(means2D=means2D, depths=depths, radii=radii, conic_opacity=conic, rgb=rgb)
    g, ob, _ = _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))
    counts = np.diff(ob["ranges"].reshape(-1, 2), axis=1).ravel()
    assert sorted(counts[counts > 0].tolist()) == sorted(sizes)


def test_binning_large_bucket_and_global_mode():
    # one tile receiving > 4096 instances and an image with more than 16384
    # local tiles (the global-atomics count path)
    rng = np.random.default_rng(9)
    P = 9000
    W, H = 2304, 2048   # 144 x 128 = 18432 tiles
    means2D = np.stack([rng.uniform(0, W, P), rng.uniform(0, H, P)], 1).astype(np.float32)
    means2D[:5000] = rng.uniform(30, 34, (5000, 2))
    radii = rng.integers(1, 12, P).astype(np.int32)
    radii[::97] = 0
    depths = rng.uniform(0.5, 50, P).astype(np.float32)
    depths[:300] = 2.0
    conic = np.tile(np.array([[0.05, 0.0, 0.05, 0.5]], np.float32), (P, 1))
    rgb = rng.random((P, 3)).astype(np.float32)
    cam = dict(W=W, H=H, tanfovx=1.0, tanfovy=1.0, viewmatrix=np.eye(4, dtype=np.float32),
               projmatrix=np.eye(4, dtype=np.float32), campos=np.zeros(3, np.float32))
    pre = dict(means2D=means2D, depths=depths, radii=radii, conic_opacity=conic, rgb=rgb)
    g, ob, _ = _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))
    assert (np.diff(ob["ranges"], axis=1) > 4096).any()


def _big_region_branch(depths):
    """Which branch sort_filter_big takes for a region list longer than 8192
    entries with these depths: "global" (bitonic network in global memory +
    per-tile filter) when every depth is equal or one 12-bit digit (from the
    highest bit on which the depths differ) holds more than 4096 entries,
    else "split" (depth ranges sorted on chip)."""
    b = np.asarray(depths, np.float32).view(np.uint32).astype(np.uint64)
    vary = int(np.bitwise_or.reduce(b)) ^ int(np.bitwise_and.reduce(b))
    if vary == 0:
        return "global", len(b)
    shift = max(vary.bit_length() - 1 - 11, 0)
    mx = int(np.bincount(((b >> np.uint64(shift)) & np.uint64(4095)).astype(np.int64), minlength=4096).max())
    return ("global" if mx > 4096 else "split"), mx


def _one_big_region_scene(n_big, big_depths, seed):
    """A 256x128 image (16x8 tiles, 8x4 regions of 2x2 tiles) whose region
    (3, 1) -- tiles x 6..7, y 2..3 -- receives n_big Gaussians (rects of 1..4
    tiles inside the region, so the filter splits each entry over its tiles),
    and 3000 others confined to tile columns 0..4, interleaved in id order."""
    rng = np.random.default_rng(seed)
    W, H = 256, 128
    nb = 3000
    big = np.stack([rng.uniform(109, 115, n_big), rng.uniform(45, 51, n_big)], 1)
    other = np.stack([rng.uniform(0, 60, nb), rng.uniform(0, H, nb)], 1)
    P = n_big + nb
    order = rng.permutation(P)
    means2D = np.concatenate([big, other])[order].astype(np.float32)
    radii = np.concatenate([rng.integers(1, 13, n_big), rng.integers(1, 17, nb)])[order].astype(np.int32)
    depths = np.concatenate([np.asarray(big_depths, np.float32), rng.uniform(0.5, 50, nb)])[order].astype(np.float32)
    conic = np.tile(np.array([[0.3, 0.0, 0.3, 0.02]], np.float32), (P, 1))
    rgb = rng.random((P, 3)).astype(np.float32)
    cam = dict(W=W, H=H, tanfovx=1.0, tanfovy=1.0, viewmatrix=np.eye(4, dtype=np.float32),
               projmatrix=np.eye(4, dtype=np.float32), campos=np.zeros(3, np.float32))
    in_big = np.zeros(P, bool)
    in_big[np.argsort(order)[:n_big]] = True
    return cam, dict(means2D=means2D, depths=depths, radii=radii, conic_opacity=conic, rgb=rgb), in_big


def test_split_big_region_single_depth_global_sort():
    # 10,000 entries of one region at one depth: sort_filter_big finds no
    # varying depth bit and sorts the list in global memory by (depth, compact
    # index), i.e. ascending id, then filters it per tile (filter_global)
    n = 10000
    cam, pre, in_big = _one_big_region_scene(n, np.full(n, 6.5, np.float32), 41)
    assert _big_region_branch(pre["depths"][in_big]) == ("global", n)
    g, ob, _ = _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))
    rg = ob["ranges"].reshape(8, 16, 2)
    counts = (rg[2:4, 6:8, 1] - rg[2:4, 6:8, 0]).astype(np.int64)
    assert counts.min() > 2000 and counts.sum() > n      # entries spread over all four tiles, some over several


def test_split_big_region_crowded_digit_global_sort():
    # 9,000 entries of one region: 8,500 distinct depths in [4.0, 4.01] and 500
    # spread over [0.5, 90]; the 12-bit digit under the highest varying bit
    # lumps the 8,500 together (> 4096), so the list is sorted in global memory
    rng = np.random.default_rng(43)
    d = np.concatenate([rng.uniform(4.0, 4.01, 8500), rng.uniform(0.5, 90.0, 500)]).astype(np.float32)
    d = d[rng.permutation(d.size)]
    assert np.unique(d[:8500]).size > 4096 or np.unique(d).size > 4096
    cam, pre, in_big = _one_big_region_scene(d.size, d, 44)
    branch, mx = _big_region_branch(pre["depths"][in_big])
    assert branch == "global" and mx > 4096, (branch, mx)
    assert np.unique(pre["depths"][in_big]).size > 4096
    _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))


def test_split_big_region_depth_ranges_on_chip():
    # the same region with 12,000 well-spread depths takes the on-chip branch
    # (depth ranges of at most 4096 entries sorted one after another, tile
    # positions carried over) -- the complement of the two tests above
    rng = np.random.default_rng(45)
    d = rng.uniform(0.5, 90.0, 12000).astype(np.float32)
    d[:200] = d[0]                                       # a tie run inside one range
    cam, pre, in_big = _one_big_region_scene(d.size, d, 46)
    assert _big_region_branch(pre["depths"][in_big])[0] == "split"
    _check_binning_and_render(cam, pre, (0.0, 0.0, 0.0))


def test_sub_image_share_matches_full_image():
    # config-3 style: a contiguous tile-row block; its ranges equal the full
    # render's ranges of those tiles shifted by a constant
    scene, cam = synth.small_scene(12000, seed=3, W=512, H=400, extent=1.6)
    pre = _oracle_pre(scene, cam)
    gx, gy = 32, 25
    rs = settings_for(cam)
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    full = gpu_render_forward(rs, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"])
    lo, hi = synth.tile_row_block(gy, 4, 1)
    cl = np.zeros((gy, gx), np.uint8)
    cl[lo:hi] = 1
    sub = gpu_render_forward(rs, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], cl)
    fr, sr = np_(full["ranges"]).astype(np.int64), np_(sub["ranges"]).astype(np.int64)
    t0, t1 = lo * gx, hi * gx
    off = fr[t0, 0]
    assert (sr[t0:t1] == fr[t0:t1] - off).all()
    assert not sr[:t0].any() and not sr[t1:].any()
    fc, sc = np_(full["color"]), np_(sub["color"])
    rows = slice(lo * 16, min(hi * 16, cam["H"]))
    assert_bitexact(sc[:, rows], fc[:, rows], "sub-image colour")
    assert not sc[:, :lo * 16].any() and not sc[:, hi * 16:].any()


def _grad_chain(scene, cam, bg, dLd):
    pre, bn, rf = O.full_forward(cam, scene, bg=np.asarray(bg, np.float32))
    rb = O.render_bwd(cam["W"], cam["H"], np.asarray(bg, np.float32), pre["means2D"], pre["conic_opacity"],
                      pre["rgb"], bn["ranges"], bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd)
    pb = O.preprocess_bwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"], pre["radii"],
                          pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic_opacity"],
                          rb["dL_dcolors"])
    return pre, bn, rf, rb, pb


def test_preprocess_backward_recomputed_cov3D_and_row_layouts():
    """The preprocess backward without the forward's cov3D (recomputed from
    scales and rotations by the forward's own code) equals the one with it,
    bit for bit, also through the C ABI with dL/dmeans3D and dL/dscales at
    4-byte (not 16-byte) aligned addresses and a partial last block
    (P = 3000)."""
    import ctypes as C
    from blitzgs_amd import rasterizer as R
    scene, cam = synth.small_scene(3000, seed=31, W=200, H=150, extent=1.2)
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    P = scene["means3D"].shape[0]
    rng = np.random.default_rng(5)
    dm2 = to_dev(rng.standard_normal((P, 2)).astype(np.float32))
    dco = to_dev(rng.standard_normal((P, 4)).astype(np.float32))
    drgb = to_dev(rng.standard_normal((P, 3)).astype(np.float32))
    t = {k: to_dev(np.asarray(scene[k], np.float32)) for k in ["means3D", "scales", "rotations", "sh"]}
    args = (t["means3D"], t["scales"], t["rotations"], t["sh"], rs, dm2, dco, drgb)
    with_cov = R._preprocess_backward_raw(g["radii"], g["cov3D"], g["clamped"], *args)
    without = R._preprocess_backward_raw(g["radii"], None, g["clamped"], *args)
    for a, b, name in zip(with_cov, without, ["means3D", "scales", "rotations", "sh", "opacity"]):
        assert torch.equal(a, b), name
    assert (np_(g["radii"]) > 0).sum() > 500
    # misaligned dL/dmeans3D and dL/dscales
    lib = _lib.load()
    buf_m, buf_s = torch.empty(3 * P + 1, device="cuda"), torch.empty(3 * P + 1, device="cuda")
    dmean, dscale = buf_m[1:], buf_s[1:]
    drot = torch.empty((P, 4), device="cuda")
    dsh = torch.empty((P, 16, 3), device="cuda")
    dop = torch.empty((P, 1), device="cuda")
    p_ = _lib.ptr
    _lib.check(lib.gs_preprocess_backward(
        P, 3, 16, p_(t["means3D"]), p_(t["scales"]), p_(t["rotations"]), p_(t["sh"]), 1.0,
        p_(rs.viewmatrix.contiguous()), p_(rs.projmatrix.contiguous()), p_(rs.campos.contiguous()), float(rs.tanfovx), float(rs.tanfovy), int(rs.image_height),
        int(rs.image_width), p_(g["radii"]), None, p_(g["clamped"]), p_(dm2), 2, p_(dco), p_(drgb), p_(dmean),
        p_(dscale), p_(drot), p_(dsh), p_(dop), _lib.stream_of()), "preprocess_backward")
    torch.cuda.synchronize()
    assert torch.equal(dmean.view(P, 3), with_cov[0])
    assert torch.equal(dscale.view(P, 3), with_cov[1])
    assert torch.equal(drot, with_cov[2]) and torch.equal(dsh, with_cov[3]) and torch.equal(dop, with_cov[4])


@pytest.mark.parametrize("P,D,K,extent,keep_cov", [(3000, 3, 16, 6.0, False), (4097, 3, 16, 1.2, True),
                                                   (777, 2, 9, 6.0, False), (64, 0, 1, 6.0, False),
                                                   (130, 1, 16, 40.0, False), (779, 2, 16, 1.5, False),
                                                   (197, 0, 16, 6.0, True)])
def test_preprocess_records_equal_array_path(P, D, K, extent, keep_cov):
    """gs_preprocess_forward_rec / gs_preprocess_backward_rec (the backward
    reads the forward's packed records of the visible Gaussians instead of
    means3D, scales, rotations, radii and clamped) give the same outputs as
    gs_preprocess_forward / gs_preprocess_backward, bit for bit: partly visible
    scenes (extent 6 puts Gaussians behind the near plane and outside the
    frustum; 40 leaves few visible), partial last waves and blocks, the staged
    (K = 16) and unstaged dL/dsh layouts, SH degrees 0-3, with and without the
    forward's cov3D.  With dL/dsh cleared beforehand and 16-byte rows (K a
    multiple of 4) the packed kernel runs: degrees 0-3, one and several
    rounds per block (extent 1.2 / 1.5: most Gaussians visible), partial runs.  The record forward leaves clamped unwritten (the records
    hold the flags); some colours are forced below zero so that flags are set."""
    from blitzgs_amd import rasterizer as R
    scene, cam = synth.small_scene(P, seed=40 + D, W=200, H=150, extent=extent)
    scene["sh"][::5, 0, 1] = -4.0
    rs = settings_for(cam, sh_degree=D)
    t = {k: to_dev(np.asarray(scene[k], np.float32)) for k in ["means3D", "scales", "rotations", "opacities"]}
    t["sh"] = to_dev(np.ascontiguousarray(np.asarray(scene["sh"], np.float32)[:, :K]))
    fwd_args = (t["means3D"], t["scales"], t["rotations"], t["sh"], t["opacities"], rs)
    a = R._preprocess_forward_raw(*fwd_args, keep_cov3D=keep_cov)
    b = R._preprocess_forward_raw(*fwd_args, keep_cov3D=keep_cov, records=True, keep_clamped=False)
    names = ["num_rendered", "means2D", "depths", "radii", "cov3D", "conic_opacity", "rgb"]
    for x, y, name in zip(a[1:7], b[1:7], names[1:]):
        assert (x is None and y is None) or torch.equal(x, y), name
    assert b[7] is None
    radii = np_(a[3])
    n_vis = int((radii > 0).sum())
    assert 0 < n_vis < P or extent <= 1.5, n_vis
    assert n_vis < 50 or np_(a[7])[radii > 0].any()          # clamp flags among the visible
    rng = np.random.default_rng(P)
    dm2 = to_dev(rng.standard_normal((P, 2)).astype(np.float32))
    dco = to_dev(rng.standard_normal((P, 4)).astype(np.float32))
    drgb = to_dev(rng.standard_normal((P, 3)).astype(np.float32))
    _, _, _, radii_t, cov3D, _, _, clamped = a
    args = (t["means3D"], t["scales"], t["rotations"], t["sh"], rs, dm2, dco, drgb)
    ref = R._preprocess_backward_raw(radii_t, cov3D, clamped, *args)
    # the record path reads neither the input arrays nor radii / clamped:
    # garbage in them changes nothing
    junk = {k: torch.full_like(v, float("nan")) for k, v in t.items()}
    got = R._preprocess_backward_raw(torch.zeros_like(radii_t), cov3D, torch.ones_like(clamped), junk["means3D"],
                                     junk["scales"], junk["rotations"], t["sh"], rs, dm2, dco, drgb, records=b[8])
    for x, y, name in zip(ref, got, ["means3D", "scales", "rotations", "sh", "opacity"]):
        assert torch.equal(x, y), name
    # outputs cleared beforehand (the autograd pair clears them on a side
    # stream while the render runs): only the visible rows are written
    zeroed = torch.zeros_like(ref[3])
    got_z = R._preprocess_backward_raw(torch.zeros_like(radii_t), cov3D, torch.ones_like(clamped), junk["means3D"],
                                       junk["scales"], junk["rotations"], t["sh"], rs, dm2, dco, drgb, records=b[8],
                                       zeroed=zeroed)
    for x, y, name in zip(ref, got_z, ["means3D", "scales", "rotations", "sh", "opacity"]):
        assert torch.equal(x, y), ("zeroed", name)
    assert got_z[3] is zeroed
    with pytest.raises(RuntimeError, match="record buffer"):
        R._preprocess_backward_raw(radii_t, cov3D, clamped, *args, records=b[8][:-256])


@pytest.mark.parametrize("extra", ["none", "summed", "hook_in_place", "geo"])
def test_preprocess_backward_reads_render_accumulators(monkeypatch, extra):
    """The preprocess backward reads the render backward's accumulators
    instead of the dense dL/dmeans2D, dL/dconic_opacity and dL/drgb when it
    receives exactly the tensors that backward returned; bit-identical
    gradients.  Another contribution to rgb's gradient (summed by autograd),
    a hook that changes the gradient in place, or render_geo's backward: the
    dense arrays are read whenever the received gradients are not the render
    backward's own (here: summed, hook), and the gradients still equal the
    dense path's."""
    from blitzgs_amd import rasterizer as R
    scene, cam = synth.small_scene(3000, seed=16, W=200, H=150, extent=1.5)
    rs = settings_for(cam)
    if extra == "geo":
        from blitzgs_amd.dropin import diff_gaussian_rasterization_r as R_pkg
        rs = R_pkg.GaussianRasterizationSettings(**dict(rs._asdict(), render_geo=True))
    seen = []
    real = R._preprocess_backward_raw

    def spy(*a, **kw):
        seen.append(kw.get("acc") is not None)
        return real(*a, **kw)

    monkeypatch.setattr(R, "_preprocess_backward_raw", spy)

    def grads():
        params = {k: to_dev(np.asarray(scene[k], np.float32)).requires_grad_(True)
                  for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
        ras = R.GaussianRasterizer(rs)
        args = {"avoid_pixel_all2all": False}
        means2D, rgb, conic, radii, depths = ras.preprocess_gaussians(
            params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], args)
        if extra == "hook_in_place":
            rgb.register_hook(lambda g: g.mul_(2.0))
        P = means2D.shape[0]
        amap = to_dev(np.random.default_rng(3).uniform(-1, 1, (P, 5)).astype(np.float32))
        color, *rest = ras.render_gaussians(means2D, torch.zeros((P, 3), device="cuda", requires_grad=True), conic,
                                            rgb, amap, depths, radii, None, None, args)
        loss = (color * to_dev(scene["dL_dimage"])).sum()
        if extra == "summed":
            loss = loss + 0.5 * rgb.sum()
        if extra == "geo":
            loss = loss + rest[4].sum() + rest[5].sum()
        loss.backward()
        return [params[k].grad for k in ["means3D", "scales", "rotations", "sh", "opacities"]]

    a = grads()
    monkeypatch.setattr(R._ZeroedGrads, "take_acc", lambda self, g: None)
    b = grads()
    assert seen == [extra in ("none", "geo"), False], seen
    # two runs: the render backward's float atomics may sum in another order
    for x, y, name in zip(a, b, ["means3D", "scales", "rotations", "sh", "opacities"]):
        assert rel_l2(np_(x), np_(y)) < 1e-6, (extra, name)
    if extra != "none":
        return
    # one render backward, both readings of its outputs: bit-identical
    monkeypatch.undo()
    t = {k: to_dev(np.asarray(scene[k], np.float32)) for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    pre = R._preprocess_forward_raw(t["means3D"], t["scales"], t["rotations"], t["sh"], t["opacities"], rs,
                                    keep_cov3D=False, records=True, keep_clamped=False)
    _, m2d, depths, radii, _, conic, rgb, _, records = pre
    W, H = int(rs.image_width), int(rs.image_height)
    f = R._render_forward_raw(rs.bg, H, W, m2d, depths, radii, conic, rgb, None)
    Rn, geom, binning, img = f[0], f[6], f[7], f[8]
    gm2d, _, gco, gcol, _ = R._render_backward_raw(rs.bg, Rn, H, W, m2d, conic, rgb, None, geom, binning, img,
                                                   to_dev(scene["dL_dimage"]), 2, False, False)
    P, K = m2d.shape[0], t["sh"].shape[1]
    args = (radii, None, None, t["means3D"], t["scales"], t["rotations"], t["sh"], rs, gm2d, gco, gcol)
    zd = torch.zeros((P, K, 3), device="cuda")
    dense = R._preprocess_backward_raw(*args, records=records, zeroed=zd)
    za = torch.zeros((P, K, 3), device="cuda")
    viaacc = R._preprocess_backward_raw(*args, records=records, zeroed=za, acc=(geom, Rn, W, H))
    for x, y, name in zip(dense, viaacc, ["means3D", "scales", "rotations", "sh", "opacity"]):
        assert torch.equal(x, y), ("accumulators", name)


@pytest.mark.parametrize("case", ["wide", "small", "masked", "ragged"])
def test_region_sides_give_identical_results(case):
    """Every output of the split forward -- image, per-tile and per-pixel
    counters, out_observe, ranges, the sorted ids and keys -- is the same for
    region sides 2 (default), 4 and 8, through both forward routes; the
    default side is checked against the oracle elsewhere."""
    from blitzgs_amd import rasterizer as R
    from tests.gpu_helpers import buffer_views
    W, H, cl = 200, 150, None
    if case == "wide":
        scene, cam = synth.small_scene(2500, seed=91, W=W, H=H, extent=1.2, log_mu=-1.2)
    elif case == "small":
        scene, cam = synth.small_scene(3000, seed=12, W=W, H=H, extent=1.2)
    elif case == "masked":
        scene, cam = synth.small_scene(4000, seed=33, W=W, H=H, extent=1.2, log_mu=-1.8)
        cl = torch.as_tensor(np.random.default_rng(5).random(((H + 15) // 16, (W + 15) // 16)) < 0.5, device="cuda")
    else:
        W, H = 333, 177
        scene, cam = synth.small_scene(3500, seed=34, W=W, H=H, extent=1.3, log_mu=-1.6)
    rs = settings_for(cam, bg=(0.2, 0.1, 0.3))
    pre = gpu_preprocess(scene, rs)
    args = (rs.bg, H, W, pre["means2D"], pre["depths"], pre["radii"], pre["conic_opacity"], pre["rgb"], cl)
    outs = {}
    for side in (2, 4, 8):
        for reserved in (False, True):
            if not reserved:
                _lib.RESERVE.reset()
            o = R._render_forward_raw(*args, region_side=side)
            Rn, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, _ = o
            v = buffer_views(Rn, W, H, binning, img, pre["means2D"].shape[0], pre["depths"], geom)
            outs[(side, reserved)] = dict(R=Rn, color=color, n_render=n_render, n_consider=n_consider,
                                         n_contrib=n_contrib, out_observe=out_observe, **v)
    ref = outs[(2, False)]
    for key, o in outs.items():
        assert o["R"] == ref["R"] > 0, key
        for k in ref:
            if k != "R":
                assert torch.equal(o[k], ref[k]), (case, key, k)


def test_autograd_clears_preprocess_grads_beside_the_render(monkeypatch):
    """The render backward clears the preprocess backward's dL/dsh while its
    blend runs, and the preprocess backward writes only the visible rows into
    it; without a render in between the preprocess backward writes every row.
    Gradients equal those of a run without the clearing (float atomics in the
    render backward: within 1e-6), and the clearing happens once: a second render backward (retain_graph) leaves the returned
    gradient alone."""
    from blitzgs_amd import rasterizer as R
    scene, cam = synth.small_scene(3000, seed=14, W=200, H=150, extent=1.5)
    rs = settings_for(cam)
    seen = []
    real = R._preprocess_backward_raw

    def spy(*a, **kw):
        seen.append(kw.get("zeroed") is not None)
        return real(*a, **kw)

    monkeypatch.setattr(R, "_preprocess_backward_raw", spy)

    def grads(render=True):
        params = {k: to_dev(np.asarray(scene[k], np.float32)).requires_grad_(True)
                  for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
        ras = R.GaussianRasterizer(rs)
        args = {"avoid_pixel_all2all": False}
        means2D, rgb, conic, radii, depths = ras.preprocess_gaussians(
            params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], args)
        if render:
            P = means2D.shape[0]
            color, *_ = ras.render_gaussians(means2D, torch.zeros((P, 3), device="cuda", requires_grad=True), conic,
                                             rgb, torch.zeros((P, 5), device="cuda"), depths, radii, None, None, args)
            torch.autograd.backward([color], [to_dev(scene["dL_dimage"])])
        else:
            torch.autograd.backward([means2D, rgb], [torch.ones_like(means2D), torch.ones_like(rgb)])
        return [params[k].grad for k in ["means3D", "scales", "rotations", "sh", "opacities"]]

    a = grads()
    monkeypatch.setattr(R._ZeroedGrads, "claim", lambda self: None)
    b = grads()
    assert seen == [True, False]
    for x, y in zip(a, b):
        assert rel_l2(np_(x), np_(y)) < 1e-6
    monkeypatch.undo()
    c = grads(render=False)
    assert np.isfinite(np_(c[3])).all()
    # the render backward twice: the second does not clear the returned dL/dsh
    params = {k: to_dev(np.asarray(scene[k], np.float32)).requires_grad_(True)
              for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    ras = R.GaussianRasterizer(rs)
    args = {"avoid_pixel_all2all": False}
    means2D, rgb, conic, radii, depths = ras.preprocess_gaussians(
        params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], args)
    P = means2D.shape[0]
    color, *_ = ras.render_gaussians(means2D, torch.zeros((P, 3), device="cuda", requires_grad=True), conic, rgb,
                                     torch.zeros((P, 5), device="cuda"), depths, radii, None, None, args)
    dL = to_dev(scene["dL_dimage"])
    torch.autograd.backward([color], [dL], retain_graph=True)
    g1 = params["sh"].grad.clone()
    torch.autograd.backward([color], [dL])
    assert rel_l2(np_(params["sh"].grad), 2.0 * np_(g1)) < 1e-6


@pytest.mark.parametrize("cfg", ["small", "config0", "wide"])
def test_autograd_forward_backward_vs_oracle(cfg):
    """The autograd pair against the oracle's chain.  "wide": Gaussians with
    more than 24 tile instances each on average, for which the backward walks
    16x8 half tiles with two pixels per lane instead of 8x8 quadrants (the
    200x150 image leaves partial tiles on both edges)."""
    from blitzgs_amd import rasterizer as R
    if cfg == "small":
        scene, cam = synth.small_scene(3000, seed=12, W=200, H=150, extent=1.2)
        bg = (0.3, 0.2, 0.1)
    elif cfg == "wide":
        scene, cam = synth.small_scene(2500, seed=91, W=200, H=150, extent=1.2, log_mu=-1.2)
        bg = (0.1, 0.2, 0.3)
    else:
        scene, cam = synth.config0()
        bg = (0.0, 0.0, 0.0)
    dLd = scene["dL_dimage"]
    pre, bn, rf, rb, pb = _grad_chain(scene, cam, bg, dLd)
    n_inst, n_listed = len(bn["point_list"]), int((pre["radii"] > 0).sum())
    assert (n_inst >= 24 * n_listed) == (cfg == "wide"), (n_inst, n_listed)
    rs = settings_for(cam, bg=bg)
    params = {k: to_dev(scene[k]).requires_grad_(True) for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    ras = R.GaussianRasterizer(rs)
    cuda_args = {"avoid_pixel_all2all": False, "stats_collector": {}}
    means2D, rgb, conic_opacity, radii, depths = ras.preprocess_gaussians(
        params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], cuda_args)
    means2D.retain_grad()
    means2D_abs = torch.zeros((means2D.shape[0], 3), device="cuda", requires_grad=True) + 0
    means2D_abs.retain_grad()
    all_map = torch.zeros((means2D.shape[0], 5), device="cuda")
    color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth = ras.render_gaussians(
        means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, None, None, cuda_args)
    assert_close_abs(np_(color), rf["color"], "color")
    assert_blend_counts(dict(out_observe=np_(out_observe), n_consider=np_(n_consider), n_contrib=np_(n_contrib)), rf)
    assert set(cuda_args["stats_collector"]) >= {"forward_render_time"}
    (color * to_dev(dLd)).sum().backward()
    assert "backward_render_time" in cuda_args["stats_collector"]
    checks = [(means2D.grad, rb["dL_dmeans2D"][:, :2], "dL_dmeans2D"),
              (means2D_abs.grad, rb["dL_dmeans2D_abs"], "dL_dmeans2D_abs"),
              (params["means3D"].grad, pb["dL_dmeans3D"], "dL_dmeans3D"),
              (params["scales"].grad, pb["dL_dscales"], "dL_dscales"),
              (params["rotations"].grad, pb["dL_drotations"], "dL_drotations"),
              (params["sh"].grad, pb["dL_dsh"], "dL_dsh"),
              (params["opacities"].grad, pb["dL_dopacity"], "dL_dopacity")]
    for got, ref, name in checks:
        e = rel_l2(np_(got), ref)
        assert e < 1e-3, (name, e)


def test_render_backward_vs_oracle_with_background():
    scene, cam = synth.small_scene(5000, seed=44, W=300, H=180, extent=1.5, log_mu=-2.2)
    bg = (0.7, 0.1, 0.4)
    dLd = scene["dL_dimage"]
    pre, bn, rf, rb, pb = _grad_chain(scene, cam, bg, dLd)
    rs = settings_for(cam, bg=bg)
    from blitzgs_amd import rasterizer as R
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    out = R._render_forward_raw(rs.bg, cam["H"], cam["W"], dev["means2D"], dev["depths"], dev["radii"],
                                dev["conic_opacity"], dev["rgb"], None)
    Rn, color, *_rest, geom, binning, img, _ = out
    g = R._render_backward_raw(rs.bg, Rn, cam["H"], cam["W"], dev["means2D"], dev["conic_opacity"], dev["rgb"],
                               None, geom, binning, img, to_dev(dLd), m2d_stride=3)
    dm, dma, dco, dcol, _ = g
    assert rel_l2(np_(dm), rb["dL_dmeans2D"]) < 1e-3
    assert not np_(dm)[:, 2].any()
    assert rel_l2(np_(dma), rb["dL_dmeans2D_abs"]) < 1e-3
    assert rel_l2(np_(dco), rb["dL_dconic_opacity"]) < 1e-3
    assert rel_l2(np_(dcol), rb["dL_dcolors"]) < 1e-3


def test_quadrant_cull_keeps_results_exact_on_hard_cases():
    # needle-like and huge Gaussians, opacities around 1/255, means exactly on
    # pixel centres and tile borders: the blend kernels cull Gaussians that
    # cannot reach alpha >= 1/255 in a quadrant; the image, transmittance and
    # contributor counts must still equal the unculled CPU evaluation bit for bit
    rng = np.random.default_rng(123)
    P, W, H = 6000, 160, 128
    means2D = np.stack([rng.uniform(-40, W + 40, P), rng.uniform(-40, H + 40, P)], 1).astype(np.float32)
    means2D[:500] = np.round(means2D[:500])
    means2D[500:800, 0] = 16.0 * rng.integers(0, 10, 300) - 0.5
    ang = rng.uniform(0, np.pi, P)
    s_long = np.exp(rng.uniform(0, 5, P))
    s_short = np.exp(rng.uniform(-1, 1.5, P))
    ca, sa = np.cos(ang), np.sin(ang)
    cxx = ca * ca * s_long ** 2 + sa * sa * s_short ** 2 + 0.3
    cyy = sa * sa * s_long ** 2 + ca * ca * s_short ** 2 + 0.3
    cxy = ca * sa * (s_long ** 2 - s_short ** 2)
    det = cxx * cyy - cxy * cxy
    conic = np.stack([cyy / det, -cxy / det, cxx / det], 1)
    op = rng.uniform(0, 1, P)
    op[:1500] = rng.choice([1 / 255.0, 0.0039, 0.0040, 0.004, 0.99, 1.0], 1500)
    co = np.concatenate([conic, op[:, None]], 1).astype(np.float32)
    radii = np.ceil(3.33 * np.sqrt(np.maximum(cxx, cyy))).astype(np.int32)
    depths = rng.uniform(1, 100, P).astype(np.float32)
    rgb = rng.random((P, 3)).astype(np.float32)
    cam = dict(W=W, H=H, tanfovx=1.0, tanfovy=1.0, viewmatrix=np.eye(4, dtype=np.float32),
               projmatrix=np.eye(4, dtype=np.float32), campos=np.zeros(3, np.float32))
    pre = dict(means2D=means2D, depths=depths, radii=radii, conic_opacity=co, rgb=rgb)
    _check_binning_and_render(cam, pre, (0.1, 0.2, 0.3))
    # and the backward over the same lists
    dLd = rng.standard_normal((3, H, W)).astype(np.float32)
    bn = O.binning(W, H, means2D, depths, radii)
    rf = O.render_fwd(W, H, np.array([0.1, 0.2, 0.3], np.float32), means2D, co, rgb, bn["ranges"], bn["point_list"])
    rb = O.render_bwd(W, H, np.array([0.1, 0.2, 0.3], np.float32), means2D, co, rgb, bn["ranges"], bn["point_list"],
                      rf["final_T"], rf["n_contrib_px"], dLd)
    from blitzgs_amd import rasterizer as R
    rs = settings_for(cam, bg=(0.1, 0.2, 0.3))
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    out = R._render_forward_raw(rs.bg, H, W, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"],
                                dev["rgb"], None)
    Rn, *_rest, geom, binning, img, _ = out
    dm, dma, dco, dcol, _ = R._render_backward_raw(rs.bg, Rn, H, W, dev["means2D"], dev["conic_opacity"],
                                                   dev["rgb"], None, geom, binning, img, to_dev(dLd), m2d_stride=3)
    for g, r, nm in ((dm, rb["dL_dmeans2D"], "dmean2D"), (dma, rb["dL_dmeans2D_abs"], "abs"),
                     (dco, rb["dL_dconic_opacity"], "conic_opacity"), (dcol, rb["dL_dcolors"], "colors")):
        assert rel_l2(np_(g), r) < 1e-3, nm


def test_wave_sum12_lane_layout():
    # the backward's 12-value wave reduction (permlane32/16 swaps, then DPP
    # transpose-adds) against a plain sum, with values that make any mis-routed
    # lane visible
    rng = np.random.default_rng(0)
    x = rng.integers(-1000, 1000, (12, 64)).astype(np.float32)
    x[7] = 1.0
    x[3, 5] = 1e6
    xt = to_dev(x.reshape(-1))
    y = torch.zeros(12, device="cuda")
    _lib.check(_lib.load().gs_diag_math(3, 12 * 64, _lib.ptr(xt), _lib.ptr(y), None), "diag sum12")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np_(y), x.astype(np.float64).sum(1).astype(np.float32))


@pytest.mark.parametrize("op,iters", [(5, 20), (7, 2), (8, 1)])
def test_valu_rate_probe_runs_and_writes_nothing(op, iters):
    # the VALU issue-rate references bench.py times (the FMA chains, the
    # forward and backward blend probes): they run, and their sentinel store
    # is not taken
    y = torch.full((1,), -7.0, device="cuda")
    _lib.check(_lib.load().gs_diag_math(op, iters, None, _lib.ptr(y), None), "diag valu")
    torch.cuda.synchronize()
    assert float(y.item()) == -7.0
    assert _lib.load().gs_diag_math(op, 1, None, None, None) != 0


def _split_forward(scene, cam, bg):
    from blitzgs_amd import rasterizer as R
    rs = settings_for(cam, bg=bg)
    params = {k: to_dev(scene[k]).requires_grad_(True) for k in ["means3D", "scales", "rotations", "sh", "opacities"]}
    ras = R.GaussianRasterizer(rs)
    cuda_args = {"avoid_pixel_all2all": False}
    means2D, rgb, conic_opacity, radii, depths = ras.preprocess_gaussians(
        params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], cuda_args)
    P = means2D.shape[0]
    means2D_abs = torch.zeros((P, 3), device="cuda", requires_grad=True)
    all_map = torch.zeros((P, 5), device="cuda")
    color = ras.render_gaussians(means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, None, None,
                                 cuda_args)[0]
    return params, color


def test_autograd_interleaved_and_repeated_backward():
    """Two cameras' forwards before either backward (each keeps its own
    buffers), then one graph differentiated twice (retain_graph): the second
    backward starts from cleared accumulators and repeats the first."""
    bg = (0.1, 0.2, 0.3)
    sA, cA = synth.small_scene(3000, seed=12, W=200, H=150, extent=1.2)
    sB, cB = synth.small_scene(2500, seed=13, W=160, H=120, extent=1.0)
    pA, colA = _split_forward(sA, cA, bg)
    pB, colB = _split_forward(sB, cB, bg)
    (colB * to_dev(sB["dL_dimage"])).sum().backward()
    lossA = (colA * to_dev(sA["dL_dimage"])).sum()
    lossA.backward(retain_graph=True)
    gA1 = {k: p.grad.detach().clone() for k, p in pA.items()}
    for p in pA.values():
        p.grad = None
    lossA.backward()
    names = {"means3D": "dL_dmeans3D", "scales": "dL_dscales", "rotations": "dL_drotations", "sh": "dL_dsh",
             "opacities": "dL_dopacity"}
    for scene, cam, params in ((sA, cA, pA), (sB, cB, pB)):
        _, _, _, _, pb = _grad_chain(scene, cam, bg, scene["dL_dimage"])
        for k, n in names.items():
            assert rel_l2(np_(params[k].grad), pb[n]) < 1e-3, (k, rel_l2(np_(params[k].grad), pb[n]))
    for k in names:
        assert rel_l2(np_(pA[k].grad), np_(gA1[k])) < 1e-5, k


def _dilate(m):
    """A tile mask grown by one tile in every direction (a wider extended mask)."""
    d = m.copy()
    d[1:] |= m[:-1]
    d[:-1] |= m[1:]
    d[:, 1:] |= m[:, :-1]
    d[:, :-1] |= m[:, 1:]
    return d


@pytest.mark.parametrize("avoid", [False, True])
def test_masked_step_and_extended_mask_vs_oracle(avoid):
    """The masked render through the autograd API, forward and backward
    (render backward under compute_locally, backward.cu:354-355).  With
    avoid_pixel_all2all the forward bins and blends the wider
    extended_compute_locally and the backward differentiates only the
    compute_locally tiles over the forward's lists (_f __init__.py:231)."""
    from tests.gpu_helpers import autograd_step, check_step, oracle_step
    scene, cam = synth.small_scene(8000, seed=91, W=331, H=203, extent=1.5, log_mu=-2.3)
    gx, gy = (331 + 15) // 16, (203 + 15) // 16
    rng = np.random.default_rng(17)
    cl = (rng.random((gy, gx)) < 0.35).astype(np.uint8)
    ext = _dilate(cl)
    assert ext.sum() > cl.sum()
    bg = (0.2, 0.4, 0.1)
    g = autograd_step(scene, cam, bg=bg, cl=cl, ext=ext, avoid=avoid, dL_dimage=scene["dL_dimage"])
    fwd_mask = ext if avoid else cl
    pre, bn, rf, rb, pb = oracle_step(scene, cam, bg=bg, cl_fwd=fwd_mask, cl_bwd=cl, dL_dimage=scene["dL_dimage"])
    check_step(g, pre, bn, rf, rb, pb)
    if avoid:
        # the extended-only tiles are rendered but give no gradient: the
        # same step with dL/dimage zeroed outside compute_locally matches
        pre2, bn2, rf2, rb2, pb2 = oracle_step(scene, cam, bg=bg, cl_fwd=ext, cl_bwd=ext,
                                               dL_dimage=_masked_pixels(scene["dL_dimage"], cl))
        for k in ("dL_dmeans3D", "dL_dsh"):
            assert rel_l2(np_(g[k]), pb2[k]) < 1e-3, k


def _masked_pixels(img, cl):
    m = np.repeat(np.repeat(cl.astype(bool), 16, 0), 16, 1)[:img.shape[1], :img.shape[2]]
    return np.where(m[None], img, 0).astype(np.float32)


def test_masked_step_more_than_16384_local_tiles_vs_oracle():
    """A masked image with more local tiles than the LDS histogram holds: the
    mask numbering kernel and the global-atomics count / scatter path run
    together, forward and backward, plain and extended masks."""
    from tests.gpu_helpers import autograd_step, check_step, oracle_step
    W, H = 2304, 2048                     # 144 x 128 = 18432 tiles
    scene, cam = synth.small_scene(20000, seed=5, W=W, H=H, extent=1.6, log_mu=-3.6, log_sd=0.3)
    gx, gy = 144, 128
    rng = np.random.default_rng(23)
    cl = (rng.random((gy, gx)) < 0.93).astype(np.uint8)
    assert cl.sum() > 16384
    ext = _dilate(cl)
    g = autograd_step(scene, cam, cl=cl, ext=ext, avoid=True, dL_dimage=scene["dL_dimage"])
    pre, bn, rf, rb, pb = oracle_step(scene, cam, cl_fwd=ext, cl_bwd=cl, dL_dimage=scene["dL_dimage"])
    assert bn["R"] > 100_000
    check_step(g, pre, bn, rf, rb, pb)


def test_point_list_written_on_request():
    """The forward keeps only the blend's compact list (its unsorted keys use
    the point list's space as scratch): the blend is right without the
    reference's sorted ids and keys, which gs_render_point_list writes when a
    caller asks."""
    import ctypes as C
    scene, cam = synth.small_scene(5000, seed=8, W=240, H=176, extent=1.5, log_mu=-2.2)
    pre = _oracle_pre(scene, cam)
    W, H = cam["W"], cam["H"]
    lib = _lib.load()
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    P = pre["means2D"].shape[0]
    T = ((W + 15) // 16) * ((H + 15) // 16)
    s = _lib.stream_of()
    geom = torch.empty(lib.gs_render_geom_bytes(P, W, H), device="cuda", dtype=torch.uint8)
    img = torch.empty(lib.gs_render_img_bytes(W, H), device="cuda", dtype=torch.uint8)
    R = C.c_int64(0)
    _lib.check(lib.gs_render_forward_count(P, W, H, _lib.ptr(dev["means2D"]), _lib.ptr(dev["radii"]), None,
                                           _lib.ptr(geom), C.byref(R), 0, s), "count")
    R = int(R.value)
    binning = torch.full((lib.gs_render_binning_bytes(R),), 0xAB, device="cuda", dtype=torch.uint8)
    color = torch.empty((3, H, W), device="cuda")
    i32 = lambda n: torch.empty(n, device="cuda", dtype=torch.int32)
    n_render, n_consider, n_contrib, obs = i32(T), i32(T), i32(T), i32(P)
    bg = to_dev(np.zeros(3, np.float32))
    _lib.check(lib.gs_render_forward(P, R, W, H, _lib.ptr(bg), _lib.ptr(dev["means2D"]), _lib.ptr(dev["depths"]),
                                     _lib.ptr(dev["radii"]), _lib.ptr(dev["conic_opacity"]), _lib.ptr(dev["rgb"]),
                                     None, _lib.ptr(geom), _lib.ptr(binning), _lib.ptr(img), _lib.ptr(color),
                                     _lib.ptr(n_render), _lib.ptr(n_consider), _lib.ptr(n_contrib), _lib.ptr(obs), 0,
                                     None, 0, s),
               "forward")
    torch.cuda.synchronize()
    from tests.gpu_helpers import buffer_views
    ob = O.binning(W, H, pre["means2D"], pre["depths"], pre["radii"])
    orf = O.render_fwd(W, H, np.zeros(3, np.float32), pre["means2D"], pre["conic_opacity"], pre["rgb"], ob["ranges"],
                       ob["point_list"])
    assert_close_abs(np_(color), orf["color"], "color without the sorted id list")
    v = buffer_views(R, W, H, binning, img, P, dev["depths"], geom)
    assert R == ob["R"]
    assert_bitexact(np_(v["point_list"]).view(np.uint32), ob["point_list"], "point_list")
    assert_bitexact(np_(v["keys"]).view(np.uint64), ob["keys"], "point_list_keys")
