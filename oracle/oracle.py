"""ctypes wrapper around the C oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline.  The product
(blitzgs_amd) never imports it.

All functions take and return numpy arrays (float32 / int32 / uint8 / ...).
Camera dictionaries use the keys produced by blitzgs_amd.synth.make_camera:
W, H, tanfovx, tanfovy, viewmatrix (4x4), projmatrix (4x4), campos (3),
plus the preprocess settings scale_modifier and sh_degree.
"""
import ctypes as C
import os

import numpy as np

from . import build as _build

_lib = None


class OCamera(C.Structure):
    _fields_ = [("W", C.c_int), ("H", C.c_int), ("tanfovx", C.c_float), ("tanfovy", C.c_float),
                ("scale_modifier", C.c_float), ("sh_degree", C.c_int),
                ("view", C.c_float * 16), ("proj", C.c_float * 16), ("campos", C.c_float * 3)]


def lib():
    global _lib
    if _lib is None:
        path = _build.build()
        _lib = C.CDLL(path)
        fp = C.c_void_p
        _lib.o_binning_count.restype = C.c_int64
        _lib.o_higher_msb.restype = C.c_uint32
        _lib.o_higher_msb.argtypes = [C.c_uint32]
        _lib.o_num_threads.restype = C.c_int
        for name in ["o_preprocess_fwd", "o_preprocess_bwd", "o_binning", "o_render_fwd",
                     "o_render_bwd", "o_knn_meandist3", "o_ssim_fwd", "o_ssim_bwd",
                     "o_vec_expf", "o_vec_logf", "o_local2j_ids_bool", "o_local2j_ids_bool_rect",
                     "o_render_geo_fwd", "o_render_bwd_geo"]:
            getattr(_lib, name).restype = None
        del fp
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def camera_struct(cam, scale_modifier=1.0, sh_degree=3):
    c = OCamera()
    c.W = int(cam["W"])
    c.H = int(cam["H"])
    c.tanfovx = float(cam["tanfovx"])
    c.tanfovy = float(cam["tanfovy"])
    c.scale_modifier = float(scale_modifier)
    c.sh_degree = int(sh_degree)
    v = _f32(cam["viewmatrix"]).reshape(-1)
    p = _f32(cam["projmatrix"]).reshape(-1)
    cp = _f32(cam["campos"]).reshape(-1)
    for i in range(16):
        c.view[i] = float(v[i])
        c.proj[i] = float(p[i])
    for i in range(3):
        c.campos[i] = float(cp[i])
    return c


def num_threads():
    return lib().o_num_threads()


def vec_expf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().o_vec_expf(C.c_int(x.size), _p(x), _p(y))
    return y


def vec_logf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().o_vec_logf(C.c_int(x.size), _p(x), _p(y))
    return y


def higher_msb(n):
    return int(lib().o_higher_msb(C.c_uint32(n)))


def preprocess_fwd(cam, means3D, scales, rotations, sh, opacities, scale_modifier=1.0, sh_degree=3):
    means3D, scales, rotations, sh, opacities = map(_f32, (means3D, scales, rotations, sh, opacities))
    P = means3D.shape[0]
    K = sh.shape[1] if sh.ndim == 3 else 1
    cs = camera_struct(cam, scale_modifier, sh_degree)
    out = dict(
        means2D=np.empty((P, 2), np.float32), depths=np.empty(P, np.float32),
        radii=np.empty(P, np.int32), cov3D=np.empty((P, 6), np.float32),
        conic_opacity=np.empty((P, 4), np.float32), rgb=np.empty((P, 3), np.float32),
        clamped=np.empty((P, 3), np.uint8))
    lib().o_preprocess_fwd(C.c_int(P), C.c_int(K), C.byref(cs), _p(means3D), _p(scales), _p(rotations),
                           _p(sh), _p(opacities), _p(out["means2D"]), _p(out["depths"]), _p(out["radii"]),
                           _p(out["cov3D"]), _p(out["conic_opacity"]), _p(out["rgb"]), _p(out["clamped"]))
    return out


def preprocess_bwd(cam, means3D, scales, rotations, sh, radii, cov3D, clamped,
                   dL_dmeans2D, dL_dconic_opacity, dL_drgb, scale_modifier=1.0, sh_degree=3):
    means3D, scales, rotations, sh, cov3D = map(_f32, (means3D, scales, rotations, sh, cov3D))
    dL_dmeans2D, dL_dconic_opacity, dL_drgb = map(_f32, (dL_dmeans2D, dL_dconic_opacity, dL_drgb))
    radii = np.ascontiguousarray(radii, dtype=np.int32)
    clamped = np.ascontiguousarray(clamped, dtype=np.uint8)
    P = means3D.shape[0]
    K = sh.shape[1]
    cs = camera_struct(cam, scale_modifier, sh_degree)
    out = dict(dL_dmeans3D=np.empty((P, 3), np.float32), dL_dscales=np.empty((P, 3), np.float32),
               dL_drotations=np.empty((P, 4), np.float32), dL_dsh=np.empty((P, K, 3), np.float32),
               dL_dopacity=np.empty((P, 1), np.float32))
    lib().o_preprocess_bwd(C.c_int(P), C.c_int(K), C.byref(cs), _p(means3D), _p(scales), _p(rotations),
                           _p(sh), _p(radii), _p(cov3D), _p(clamped), _p(dL_dmeans2D),
                           C.c_int(dL_dmeans2D.shape[1]), _p(dL_dconic_opacity), _p(dL_drgb),
                           _p(out["dL_dmeans3D"]), _p(out["dL_dscales"]), _p(out["dL_drotations"]),
                           _p(out["dL_dsh"]), _p(out["dL_dopacity"]))
    return out


def tile_grid(W, H):
    return (W + 15) // 16, (H + 15) // 16


def binning(W, H, means2D, depths, radii, compute_locally=None):
    means2D, depths = _f32(means2D), _f32(depths)
    radii = np.ascontiguousarray(radii, dtype=np.int32)
    gx, gy = tile_grid(W, H)
    if compute_locally is None:
        compute_locally = np.ones(gx * gy, np.uint8)
    cl = np.ascontiguousarray(compute_locally, dtype=np.uint8).reshape(-1)
    P = means2D.shape[0]
    tt = np.empty(P, np.uint32)
    R = lib().o_binning_count(C.c_int(P), C.c_int(W), C.c_int(H), _p(means2D), _p(radii), _p(cl), _p(tt))
    keys = np.empty(R, np.uint64)
    vals = np.empty(R, np.uint32)
    ranges = np.empty((gx * gy, 2), np.uint32)
    lib().o_binning(C.c_int(P), C.c_int(W), C.c_int(H), _p(means2D), _p(depths), _p(radii), _p(cl),
                    _p(tt), C.c_int64(R), _p(keys), _p(vals), _p(ranges))
    return dict(R=int(R), tiles_touched=tt, keys=keys, point_list=vals, ranges=ranges)


def render_fwd(W, H, bg, means2D, conic_opacity, rgb, ranges, point_list, compute_locally=None):
    """Render forward with the per-tile statistics; also the decision margins
    (obs_near per Gaussian, stop_near per pixel) that bound which integer
    outputs a blend with a slightly different exp may change."""
    means2D, conic_opacity, rgb, bg = map(_f32, (means2D, conic_opacity, rgb, bg))
    gx, gy = tile_grid(W, H)
    if compute_locally is None:
        compute_locally = np.ones(gx * gy, np.uint8)
    cl = np.ascontiguousarray(compute_locally, dtype=np.uint8).reshape(-1)
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    P = means2D.shape[0]
    T = gx * gy
    out = dict(color=np.empty((3, H, W), np.float32), final_T=np.empty((H, W), np.float32),
               n_contrib_px=np.empty((H, W), np.uint32), n_contrib2loss_px=np.empty((H, W), np.uint32),
               out_observe=np.zeros(P, np.int32), n_render=np.empty(T, np.int32),
               n_consider=np.empty(T, np.int32), n_contrib=np.empty(T, np.int32),
               obs_near=np.zeros(P, np.int32), stop_near=np.empty((H, W), np.uint8))
    lib().o_render_fwd(C.c_int(P), C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity), _p(rgb),
                       _p(cl), _p(ranges), _p(point_list), _p(out["color"]), _p(out["final_T"]),
                       _p(out["n_contrib_px"]), _p(out["n_contrib2loss_px"]), _p(out["out_observe"]),
                       _p(out["n_render"]), _p(out["n_consider"]), _p(out["n_contrib"]),
                       _p(out["obs_near"]), _p(out["stop_near"]))
    return out


def set_blend_margin_model(exp_delta=0.0, bound_rel=4e-6):
    """Test hook of render_fwd: perturb every evaluated exp by a relative
    +-exp_delta, and set the relative exp error its decision margins assume
    (default: O_EXP_REL = 4e-6).  set_blend_margin_model() restores both."""
    f = lib().o_set_blend_margin_model
    f.restype = None
    f.argtypes = [C.c_float, C.c_float]
    f(float(exp_delta), float(bound_rel))


def render_bwd(W, H, bg, means2D, conic_opacity, rgb, ranges, point_list, final_T, n_contrib_px,
               dL_dpixels, compute_locally=None):
    means2D, conic_opacity, rgb, bg, final_T, dL_dpixels = map(
        _f32, (means2D, conic_opacity, rgb, bg, final_T, dL_dpixels))
    gx, gy = tile_grid(W, H)
    if compute_locally is None:
        compute_locally = np.ones(gx * gy, np.uint8)
    cl = np.ascontiguousarray(compute_locally, dtype=np.uint8).reshape(-1)
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    n_contrib_px = np.ascontiguousarray(n_contrib_px, dtype=np.uint32)
    P = means2D.shape[0]
    out = dict(dL_dmeans2D=np.zeros((P, 3), np.float32), dL_dmeans2D_abs=np.zeros((P, 3), np.float32),
               dL_dconic=np.zeros((P, 4), np.float32), dL_dopacity=np.zeros(P, np.float32),
               dL_dcolors=np.zeros((P, 3), np.float32))
    lib().o_render_bwd(C.c_int(P), C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity), _p(rgb),
                       _p(cl), _p(ranges), _p(point_list), _p(final_T), _p(n_contrib_px), _p(dL_dpixels),
                       _p(out["dL_dmeans2D"]), _p(out["dL_dmeans2D_abs"]), _p(out["dL_dconic"]),
                       _p(out["dL_dopacity"]), _p(out["dL_dcolors"]))
    dc = out["dL_dconic"]
    # rasterize_points.cu:425-433: repack (P,2,2) slots into [c00, c01, c11, opacity]
    out["dL_dconic_opacity"] = np.stack([dc[:, 0], dc[:, 1], dc[:, 3], out["dL_dopacity"]], axis=1)
    return out


class OGeoBwd(C.Structure):
    _fields_ = [("fx", C.c_float), ("fy", C.c_float), ("all_maps", C.c_void_p), ("all_map_pixels", C.c_void_p),
                ("dL_dmaps", C.c_void_p), ("dL_dplane", C.c_void_p), ("dL_dall_map", C.c_void_p)]


def focal(W, H, tanfovx, tanfovy):
    """focal_x, focal_y as the render host computes them in float
    (_r rasterize_points.cu:325-326): W / (2 tan_fovx), H / (2 tan_fovy)."""
    fx = np.float32(W) / (np.float32(2.0) * np.float32(tanfovx))
    fy = np.float32(H) / (np.float32(2.0) * np.float32(tanfovy))
    return np.float32(fx), np.float32(fy)


def render_geo_fwd(W, H, tanfovx, tanfovy, means2D, conic_opacity, all_map, ranges, point_list,
                   compute_locally=None):
    """render_geo's maps: out_all_map (5,H,W) and out_plane_depth (1,H,W)."""
    means2D, conic_opacity, all_map = map(_f32, (means2D, conic_opacity, all_map))
    assert all_map.shape == (means2D.shape[0], 5)
    gx, gy = tile_grid(W, H)
    if compute_locally is None:
        compute_locally = np.ones(gx * gy, np.uint8)
    cl = np.ascontiguousarray(compute_locally, dtype=np.uint8).reshape(-1)
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    fx, fy = focal(W, H, tanfovx, tanfovy)
    out_all_map = np.empty((5, H, W), np.float32)
    out_plane_depth = np.empty((1, H, W), np.float32)
    # cx, cy = float(W * 0.5f), float(H * 0.5f) (rasterize_points.cu:339)
    lib().o_render_geo_fwd(C.c_int(W), C.c_int(H), C.c_float(fx), C.c_float(fy), C.c_float(0.5 * W),
                           C.c_float(0.5 * H), _p(means2D), _p(conic_opacity), _p(all_map), _p(cl), _p(ranges),
                           _p(point_list), _p(out_all_map), _p(out_plane_depth))
    return dict(out_all_map=out_all_map, out_plane_depth=out_plane_depth)


def render_bwd_geo(W, H, tanfovx, tanfovy, bg, means2D, conic_opacity, rgb, all_maps, all_map_pixels, ranges,
                   point_list, final_T, n_contrib_px, dL_dpixels, dL_dmaps, dL_dplane, compute_locally=None):
    """render_bwd with render_geo on: also dL_dall_map (P,5)."""
    means2D, conic_opacity, rgb, bg, final_T, dL_dpixels = map(
        _f32, (means2D, conic_opacity, rgb, bg, final_T, dL_dpixels))
    all_maps, all_map_pixels, dL_dmaps, dL_dplane = map(_f32, (all_maps, all_map_pixels, dL_dmaps, dL_dplane))
    gx, gy = tile_grid(W, H)
    if compute_locally is None:
        compute_locally = np.ones(gx * gy, np.uint8)
    cl = np.ascontiguousarray(compute_locally, dtype=np.uint8).reshape(-1)
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    n_contrib_px = np.ascontiguousarray(n_contrib_px, dtype=np.uint32)
    P = means2D.shape[0]
    fx, fy = focal(W, H, tanfovx, tanfovy)
    out = dict(dL_dmeans2D=np.zeros((P, 3), np.float32), dL_dmeans2D_abs=np.zeros((P, 3), np.float32),
               dL_dconic=np.zeros((P, 4), np.float32), dL_dopacity=np.zeros(P, np.float32),
               dL_dcolors=np.zeros((P, 3), np.float32), dL_dall_map=np.zeros((P, 5), np.float32))
    geo = OGeoBwd(fx, fy, all_maps.ctypes.data, all_map_pixels.ctypes.data, dL_dmaps.ctypes.data,
                  dL_dplane.ctypes.data, out["dL_dall_map"].ctypes.data)
    lib().o_render_bwd_geo(C.c_int(P), C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity), _p(rgb),
                           _p(cl), _p(ranges), _p(point_list), _p(final_T), _p(n_contrib_px), _p(dL_dpixels),
                           _p(out["dL_dmeans2D"]), _p(out["dL_dmeans2D_abs"]), _p(out["dL_dconic"]),
                           _p(out["dL_dopacity"]), _p(out["dL_dcolors"]), C.byref(geo))
    dc = out["dL_dconic"]
    out["dL_dconic_opacity"] = np.stack([dc[:, 0], dc[:, 1], dc[:, 3], out["dL_dopacity"]], axis=1)
    return out


def knn_meandist3(points):
    points = _f32(points)
    P = points.shape[0]
    out = np.empty(P, np.float32)
    lib().o_knn_meandist3(C.c_int(P), _p(points), _p(out))
    return out


def adam_update(param, grad, exp_avg, exp_avg_sq, visible, lr, b1, b2, eps):
    """In-place sparse Adam step on (N, M) float32 arrays (adam.cu:9-38)."""
    for a in (param, grad, exp_avg, exp_avg_sq):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    N = param.shape[0]
    M = param.size // max(N, 1)
    vis = np.ascontiguousarray(visible, dtype=np.uint8)
    lib().o_adam_update(_p(param), _p(grad), _p(exp_avg), _p(exp_avg_sq), _p(vis), C.c_float(lr), C.c_float(b1),
                        C.c_float(b2), C.c_float(eps), C.c_int64(N), C.c_int64(M))


def local2j_ids_bool(H, W, means2D, radii, strategy, avoid=False):
    """(P, world) bool routing matrix, interval mode (rasterize_points.cu:212-289).
    strategy holds world + 1 tile indices."""
    m2d = _f32(means2D).reshape(-1, 2)
    r = np.ascontiguousarray(radii, dtype=np.int32)
    st = np.ascontiguousarray(strategy, dtype=np.int32)
    P, world = m2d.shape[0], st.size - 1
    out = np.empty((P, world), np.uint8)
    lib().o_local2j_ids_bool(P, H, W, world, _p(m2d), _p(r), _p(st), int(bool(avoid)), _p(out))
    return out.astype(bool)


def local2j_ids_bool_rect(H, W, means2D, radii, rectangles, avoid=False):
    """(P, world) bool routing matrix, one tile rectangle (y_l, y_r, x_l, x_r)
    per rank (rasterize_points.cu:291-367)."""
    m2d = _f32(means2D).reshape(-1, 2)
    r = np.ascontiguousarray(radii, dtype=np.int32)
    rc = np.ascontiguousarray(rectangles, dtype=np.int32).reshape(-1, 4)
    P, world = m2d.shape[0], rc.shape[0]
    out = np.empty((P, world), np.uint8)
    lib().o_local2j_ids_bool_rect(P, H, W, world, _p(m2d), _p(r), _p(rc), int(bool(avoid)), _p(out))
    return out.astype(bool)


def ssim_fwd(img1, img2, C1=0.01 ** 2, C2=0.03 ** 2, train=True):
    img1, img2 = _f32(img1), _f32(img2)
    B, Ch, H, W = img1.shape
    m = np.empty_like(img1)
    if train:
        d1, d2, d3 = np.empty_like(img1), np.empty_like(img1), np.empty_like(img1)
        lib().o_ssim_fwd(B, Ch, H, W, C.c_float(C1), C.c_float(C2), _p(img1), _p(img2), _p(m),
                         _p(d1), _p(d2), _p(d3))
        return m, d1, d2, d3
    lib().o_ssim_fwd(B, Ch, H, W, C.c_float(C1), C.c_float(C2), _p(img1), _p(img2), _p(m),
                     None, None, None)
    return m, None, None, None


def ssim_bwd(img1, img2, dL_dmap, d1, d2, d3, C1=0.01 ** 2, C2=0.03 ** 2):
    img1, img2, dL_dmap, d1, d2, d3 = map(_f32, (img1, img2, dL_dmap, d1, d2, d3))
    B, Ch, H, W = img1.shape
    g = np.empty_like(img1)
    lib().o_ssim_bwd(B, Ch, H, W, C.c_float(C1), C.c_float(C2), _p(img1), _p(img2), _p(dL_dmap),
                     _p(d1), _p(d2), _p(d3), _p(g))
    return g


def full_forward(cam, scene, bg=None, compute_locally=None, scale_modifier=1.0, sh_degree=3):
    """Preprocess + binning + render forward, the reference's training forward."""
    pre = preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                         scene["opacities"], scale_modifier, sh_degree)
    W, H = int(cam["W"]), int(cam["H"])
    bn = binning(W, H, pre["means2D"], pre["depths"], pre["radii"], compute_locally)
    if bg is None:
        bg = np.zeros(3, np.float32)
    rf = render_fwd(W, H, bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"],
                    bn["point_list"], compute_locally)
    return pre, bn, rf


# ---------------------------------------------------------------- full-image path

def _opt_f32(a):
    return None if a is None else _f32(a)


def preprocess_fwd_full(cam, means3D, scales, rotations, dc, rest, opacities, colors_precomp=None,
                        cov3D_precomp=None, culling=None, scale_modifier=1.0, sh_degree=3):
    """preprocessCUDA with the full path's arguments (_f forward.cu:165-284)."""
    means3D, scales, rotations, opacities = map(_f32, (means3D, scales, rotations, opacities))
    P = means3D.shape[0]
    dc = _f32(dc).reshape(P, 3) if dc is not None else np.zeros((P, 3), np.float32)
    rest = _f32(rest).reshape(P, -1, 3) if rest is not None else np.zeros((P, 0, 3), np.float32)
    M = rest.shape[1]
    cp, c3 = _opt_f32(colors_precomp), _opt_f32(cov3D_precomp)
    cull = np.zeros(P, np.uint8) if culling is None else np.ascontiguousarray(culling, dtype=np.uint8)
    cs = camera_struct(cam, scale_modifier, sh_degree)
    out = dict(
        means2D=np.empty((P, 2), np.float32), depths=np.empty(P, np.float32),
        radii=np.empty(P, np.int32), cov3D=np.empty((P, 6), np.float32),
        conic_opacity=np.empty((P, 4), np.float32), rgb=np.empty((P, 3), np.float32),
        clamped=np.empty((P, 3), np.uint8), rects=np.empty((P, 2), np.float32),
        tiles_touched=np.empty(P, np.uint32))
    lib().o_preprocess_fwd_full(C.c_int(P), C.c_int(M), C.byref(cs), _p(means3D), _p(scales), _p(rotations),
                                _p(dc), _p(rest), _p(opacities), None if cp is None else _p(cp),
                                None if c3 is None else _p(c3), _p(cull), _p(out["means2D"]), _p(out["depths"]),
                                _p(out["radii"]), _p(out["cov3D"]), _p(out["conic_opacity"]), _p(out["rgb"]),
                                _p(out["clamped"]), _p(out["rects"]), _p(out["tiles_touched"]))
    return out


def preprocess_bwd_full(cam, means3D, scales, rotations, dc, rest, radii, cov3D, clamped, dL_dmeans2D,
                        dL_dconic, dL_dcolors, colors_precomp=None, cov3D_precomp=None, scale_modifier=1.0,
                        sh_degree=3):
    """BACKWARD::preprocess with the full path's arguments (_f backward.cu:759-827).
    dL_dconic: (P,4) float4 slots (.x=c00, .y=c01, .w=c11)."""
    means3D, scales, rotations, cov3D = map(_f32, (means3D, scales, rotations, cov3D))
    P = means3D.shape[0]
    dc = _f32(dc).reshape(P, 3) if dc is not None else np.zeros((P, 3), np.float32)
    rest = _f32(rest).reshape(P, -1, 3) if rest is not None else np.zeros((P, 0, 3), np.float32)
    M = rest.shape[1]
    dL_dmeans2D = _f32(dL_dmeans2D).reshape(P, 3)
    dL_dconic, dL_dcolors = _f32(dL_dconic).reshape(P, 4), _f32(dL_dcolors).reshape(P, 3)
    radii = np.ascontiguousarray(radii, dtype=np.int32)
    clamped = np.ascontiguousarray(clamped, dtype=np.uint8)
    cp, c3 = _opt_f32(colors_precomp), _opt_f32(cov3D_precomp)
    cs = camera_struct(cam, scale_modifier, sh_degree)
    out = dict(dL_dmeans3D=np.empty((P, 3), np.float32), dL_dcov3D=np.empty((P, 6), np.float32),
               dL_ddc=np.empty((P, 1, 3), np.float32), dL_dsh=np.empty((P, M, 3), np.float32),
               dL_dscales=np.empty((P, 3), np.float32), dL_drotations=np.empty((P, 4), np.float32))
    lib().o_preprocess_bwd_full(C.c_int(P), C.c_int(M), C.byref(cs), _p(means3D), _p(scales), _p(rotations),
                                _p(dc), _p(rest) if M > 0 else None, None if cp is None else _p(cp),
                                None if c3 is None else _p(c3), _p(radii), _p(cov3D), _p(clamped),
                                _p(dL_dmeans2D), _p(dL_dconic), _p(dL_dcolors), _p(out["dL_dmeans3D"]),
                                _p(out["dL_dcov3D"]), _p(out["dL_ddc"]), _p(out["dL_dsh"]),
                                _p(out["dL_dscales"]), _p(out["dL_drotations"]))
    return out


def full_tile_keep(xy, co, tx, ty):
    xy, co = _f32(xy), _f32(co)
    return bool(lib().o_full_tile_keep(_p(xy), _p(co), C.c_uint(tx), C.c_uint(ty)))


def binning_full(W, H, means2D, depths, radii, rects, conic_opacity, tiles_touched):
    """Binning of the full path (rasterizer_impl.cu:119-210,440-480): R = sum of
    tiles_touched entries, culled slots padded and sorted last."""
    means2D, depths, rects, conic_opacity = map(_f32, (means2D, depths, rects, conic_opacity))
    radii = np.ascontiguousarray(radii, dtype=np.int32)
    tt = np.ascontiguousarray(tiles_touched, dtype=np.uint32)
    gx, gy = tile_grid(W, H)
    P = means2D.shape[0]
    R = int(tt.astype(np.int64).sum())
    keys = np.empty(R, np.uint64)
    vals = np.empty(R, np.uint32)
    ranges = np.empty((gx * gy, 2), np.uint32)
    nb = C.c_int64(0)
    lib().o_binning_full.restype = C.c_int64
    valid = lib().o_binning_full(C.c_int(P), C.c_int(W), C.c_int(H), _p(means2D), _p(depths), _p(radii),
                                 _p(rects), _p(conic_opacity), _p(tt), C.c_int64(R), _p(keys), _p(vals),
                                 _p(ranges), C.byref(nb))
    return dict(R=R, valid=int(valid), keys=keys, point_list=vals, ranges=ranges, num_buckets=int(nb.value))


def render_fwd_full(W, H, bg, means2D, conic_opacity, colors, ranges, point_list, flag_max_count=True,
                    simp=False):
    """renderCUDA / render_simpCUDA of the full path (forward.cu:291-607)."""
    means2D, conic_opacity, colors, bg = map(_f32, (means2D, conic_opacity, colors, bg))
    gx, gy = tile_grid(W, H)
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    P = means2D.shape[0]
    out = dict(color=np.empty((3, H, W), np.float32), final_T=np.empty((H, W), np.float32),
               n_contrib_px=np.empty((H, W), np.uint32), max_contrib=np.empty(gx * gy, np.uint32),
               accum_max_count=np.zeros(P, np.float32))
    if simp:
        out["accum_weights"] = np.zeros(P, np.float32)
        out["accum_weights_count"] = np.zeros(P, np.int32)
    lib().o_render_fwd_full(C.c_int(P), C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity),
                            _p(colors), _p(ranges), _p(point_list), C.c_int(int(bool(flag_max_count))),
                            _p(out["color"]), _p(out["final_T"]), _p(out["n_contrib_px"]), _p(out["max_contrib"]),
                            _p(out["accum_max_count"]), _p(out["accum_weights"]) if simp else None,
                            _p(out["accum_weights_count"]) if simp else None)
    return out


def inv4_colmajor(m):
    """Inverse of the 4x4 matrix stored column-major in m (16 floats), as the depth render uses it."""
    m = _f32(np.asarray(m).reshape(-1))
    out = np.empty(16, np.float32)
    lib().o_inv4_colmajor(_p(m), _p(out))
    return out


def render_depth_full(W, H, bg, means2D, conic_opacity, colors, ranges, point_list, means3D, scales, rotations,
                      projmatrix, campos):
    """render_depthCUDA of the full path (_f forward.cu:616-835)."""
    means2D, conic_opacity, colors, bg, means3D, scales, rotations = map(
        _f32, (means2D, conic_opacity, colors, bg, means3D, scales, rotations))
    projmatrix, campos = _f32(np.asarray(projmatrix).reshape(-1)), _f32(np.asarray(campos).reshape(-1))
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    out = dict(color=np.empty((3, H, W), np.float32), out_pts=np.empty((3, H, W), np.float32),
               depth=np.empty((1, H, W), np.float32), accum_alpha=np.empty((1, H, W), np.float32),
               gidx=np.empty((1, H, W), np.int32), discriminants=np.empty((1, H, W), np.float32))
    lib().o_render_depth_full(C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity), _p(colors),
                              _p(ranges), _p(point_list), _p(means3D), _p(scales), _p(rotations), _p(projmatrix),
                              _p(campos), _p(out["color"]), _p(out["out_pts"]), _p(out["depth"]),
                              _p(out["accum_alpha"]), _p(out["gidx"]), _p(out["discriminants"]))
    return out


def full_path_depth(cam, scene, bg=None, culling=None, colors_precomp=None, cov3D_precomp=None, scale_modifier=1.0,
                    sh_degree=3):
    """render_depth of the full path (rasterizer_impl.cu:671-847): preprocess,
    binning as the forward, the depth blend."""
    sh = _f32(scene["sh"])
    pre = preprocess_fwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], sh[:, :1], sh[:, 1:],
                              scene["opacities"], colors_precomp, cov3D_precomp, culling, scale_modifier,
                              sh_degree)
    W, H = int(cam["W"]), int(cam["H"])
    bn = binning_full(W, H, pre["means2D"], pre["depths"], pre["radii"], pre["rects"], pre["conic_opacity"],
                      pre["tiles_touched"])
    if bg is None:
        bg = np.zeros(3, np.float32)
    colors = pre["rgb"] if colors_precomp is None else colors_precomp
    rd = render_depth_full(W, H, bg, pre["means2D"], pre["conic_opacity"], colors, bn["ranges"], bn["point_list"],
                           scene["means3D"], scene["scales"], scene["rotations"], cam["projmatrix"], cam["campos"])
    return pre, bn, rd


def render_bwd_full(W, H, bg, means2D, conic_opacity, colors, ranges, point_list, final_T, n_contrib_px,
                    dL_dpixels):
    """Render backward of the full path (per-pixel gradients with the clamp rule of
    PerGaussianRenderCUDA, _f backward.cu:403-588)."""
    means2D, conic_opacity, colors, bg, final_T, dL_dpixels = map(
        _f32, (means2D, conic_opacity, colors, bg, final_T, dL_dpixels))
    ranges = np.ascontiguousarray(ranges, dtype=np.uint32)
    point_list = np.ascontiguousarray(point_list, dtype=np.uint32)
    n_contrib_px = np.ascontiguousarray(n_contrib_px, dtype=np.uint32)
    P = means2D.shape[0]
    out = dict(dL_dmeans2D=np.zeros((P, 3), np.float32), dL_dconic=np.zeros((P, 4), np.float32),
               dL_dopacity=np.zeros(P, np.float32), dL_dcolors=np.zeros((P, 3), np.float32))
    lib().o_render_bwd_full(C.c_int(P), C.c_int(W), C.c_int(H), _p(bg), _p(means2D), _p(conic_opacity),
                            _p(colors), _p(ranges), _p(point_list), _p(final_T), _p(n_contrib_px),
                            _p(dL_dpixels), _p(out["dL_dmeans2D"]), _p(out["dL_dconic"]), _p(out["dL_dopacity"]),
                            _p(out["dL_dcolors"]))
    return out


def full_path_forward(cam, scene, bg=None, culling=None, colors_precomp=None, cov3D_precomp=None,
                      flag_max_count=True, simp=False, scale_modifier=1.0, sh_degree=3):
    """GaussianRasterizer.forward / render_simp of the full path
    (rasterizer_impl.cu:336-486): preprocess, binning, render."""
    sh = _f32(scene["sh"])
    pre = preprocess_fwd_full(cam, scene["means3D"], scene["scales"], scene["rotations"], sh[:, :1], sh[:, 1:],
                              scene["opacities"], colors_precomp, cov3D_precomp, culling, scale_modifier,
                              sh_degree)
    W, H = int(cam["W"]), int(cam["H"])
    bn = binning_full(W, H, pre["means2D"], pre["depths"], pre["radii"], pre["rects"], pre["conic_opacity"],
                      pre["tiles_touched"])
    if bg is None:
        bg = np.zeros(3, np.float32)
    colors = pre["rgb"] if colors_precomp is None else colors_precomp
    rf = render_fwd_full(W, H, bg, pre["means2D"], pre["conic_opacity"], colors, bn["ranges"],
                         bn["point_list"], flag_max_count, simp)
    return pre, bn, rf
