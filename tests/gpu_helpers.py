"""Shared helpers for the GPU parity tests: run the HIP path through the C ABI
(via the Python operator layer) and the CPU oracle on the same inputs."""
import ctypes as C

import numpy as np
import torch

from blitzgs_amd import _lib, rasterizer
from blitzgs_amd.rasterizer import GaussianRasterizationSettings


def settings_for(cam, bg=(0.0, 0.0, 0.0), sh_degree=3, scale_modifier=1.0, device="cuda"):
    t = lambda a: torch.as_tensor(np.asarray(a, np.float32), device=device)
    return GaussianRasterizationSettings(
        image_height=int(cam["H"]), image_width=int(cam["W"]), tanfovx=float(cam["tanfovx"]),
        tanfovy=float(cam["tanfovy"]), bg=t(bg), scale_modifier=float(scale_modifier),
        viewmatrix=t(cam["viewmatrix"]), projmatrix=t(cam["projmatrix"]), sh_degree=int(sh_degree),
        campos=t(cam["campos"]), prefiltered=False, debug=False)


def to_dev(a, device="cuda"):
    return torch.as_tensor(np.ascontiguousarray(a), device=device)


def np_(t):
    return t.detach().cpu().numpy()


def gpu_preprocess(scene, rs):
    r = rasterizer._preprocess_forward_raw(to_dev(scene["means3D"]), to_dev(scene["scales"]),
                                           to_dev(scene["rotations"]), to_dev(scene["sh"]),
                                           to_dev(scene["opacities"]), rs)
    _, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped = r
    return dict(means2D=means2D, depths=depths, radii=radii, cov3D=cov3D, conic_opacity=conic_opacity, rgb=rgb,
                clamped=clamped)


def gpu_render_forward(rs, means2D, depths, radii, conic_opacity, rgb, compute_locally=None):
    H, W = int(rs.image_height), int(rs.image_width)
    out = rasterizer._render_forward_raw(rs.bg, H, W, means2D, depths, radii, conic_opacity, rgb,
                                         None if compute_locally is None else to_dev(compute_locally))
    R, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, _ = out
    views = buffer_views(R, W, H, binning, img, means2D.shape[0], depths, geom)
    return dict(R=R, color=color, n_render=n_render, n_consider=n_consider, n_contrib=n_contrib,
                out_observe=out_observe, geom=geom, binning=binning, img=img, **views)


def buffer_views(R, W, H, binning, img, P=None, depths=None, geom=None):
    """Copy the sorted ids/keys, ranges and per-pixel state out of the opaque
    buffers; with P / depths / geom the sorted ids and keys are first written
    from the forward's compact list (gs_render_point_list)."""
    lib = _lib.load()
    if depths is not None:
        _lib.check(lib.gs_render_point_list(int(P), R, W, H, _lib.ptr(depths.contiguous()), _lib.ptr(geom),
                                            _lib.ptr(binning), _lib.ptr(img), _lib.stream_of()),
                   "gs_render_point_list")
    pl, keys, rg, ft, nc, n2 = (C.c_void_p() for _ in range(6))
    _lib.check(lib.gs_render_buffer_views(R, W, H, _lib.ptr(binning), _lib.ptr(img), C.byref(pl), C.byref(keys),
                                          C.byref(rg), C.byref(ft), C.byref(nc), C.byref(n2)), "buffer_views")
    base_b, base_i = binning.data_ptr(), img.data_ptr()
    T = ((H + 15) // 16) * ((W + 15) // 16)

    def view(buf, base, addr, n, dtype, nbytes):
        off = (addr.value or base) - base
        return buf[off:off + n * nbytes].view(dtype)
    torch.cuda.synchronize()
    return dict(point_list=view(binning, base_b, pl, R, torch.int32, 4),
                keys=view(binning, base_b, keys, R, torch.int64, 8),
                ranges=view(img, base_i, rg, 2 * T, torch.int32, 4).reshape(T, 2),
                final_T=view(img, base_i, ft, H * W, torch.float32, 4).reshape(H, W),
                n_contrib_px=view(img, base_i, nc, H * W, torch.int32, 4).reshape(H, W),
                n_contrib2loss_px=view(img, base_i, n2, H * W, torch.int32, 4).reshape(H, W))


def bits(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float32:
        return a.view(np.uint32)
    return a


def assert_bitexact(got, ref, name):
    g, r = bits(np.asarray(got)), bits(np.asarray(ref))
    assert g.shape == r.shape, (name, g.shape, r.shape)
    bad = np.flatnonzero(g.reshape(-1) != r.reshape(-1))
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{name}: {bad.size} of {g.size} entries differ; first at flat index {i}: "
                             f"got {np.asarray(got).reshape(-1)[i]!r} ref {np.asarray(ref).reshape(-1)[i]!r}")


# The blend evaluates G = exp(power) with the hardware exp2 (a few 1e-7
# relative from the oracle's exact fp32 exp; the alpha >= 1/255 cut-off is
# decided exactly), so its outputs carry the north_star's tolerance: RGB and
# transmittance within 1e-4 max-abs of the oracle.  Its integer outputs (last
# contributor, contributor counts, observations) are equal except where a
# pixel's transmittance lands within ~1e-6 of a decision threshold (the
# T < 1e-4 stop, the T > 0.5 observation): at most 1e-4 of the entries may
# differ (and at least 3 are allowed).
BLEND_ATOL = 1e-4


def assert_close_abs(got, ref, name, atol=BLEND_ATOL):
    g, r = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert g.shape == r.shape, (name, g.shape, r.shape)
    if not g.size:
        return
    nan_g, nan_r = np.isnan(g), np.isnan(r)
    assert (nan_g == nan_r).all(), f"{name}: NaN positions differ"
    d = np.abs(np.where(nan_g, 0.0, g - r))
    i = int(np.argmax(d))
    assert d.flat[i] <= atol, (f"{name}: max-abs difference {d.flat[i]:.3g} > {atol} at flat index {i}: "
                               f"got {g.flat[i]!r} ref {r.flat[i]!r}")


def assert_counts_close(got, ref, name, frac=1e-4, min_allowed=3):
    g = np.asarray(got).astype(np.int64).ravel()
    r = np.asarray(ref).astype(np.int64).ravel()
    assert g.shape == r.shape, (name, g.shape, r.shape)
    bad = np.flatnonzero(g != r)
    allowed = max(min_allowed, int(frac * g.size))
    assert bad.size <= allowed, (f"{name}: {bad.size} of {g.size} entries differ (allowed {allowed}); first at "
                                 f"{bad[:5].tolist()}: got {g[bad[:5]].tolist()} ref {r[bad[:5]].tolist()}")


def _tile_sums(px, W, H):
    """Per-16x16-tile sums of an (H, W) per-pixel array, tile-row-major."""
    gx, gy = (W + 15) // 16, (H + 15) // 16
    a = np.zeros((gy * 16, gx * 16), np.int64)
    a[:H, :W] = np.asarray(px).astype(np.int64).reshape(H, W)
    return a.reshape(gy, 16, gx, 16).sum(axis=(1, 3)).reshape(-1)


def assert_blend_counts(got, rf, label=""):
    """The blend's integer outputs against the oracle's, with every mismatch
    attributed to a decision that the oracle's margins mark as near its
    threshold (oracle.render_fwd's stop_near / obs_near: the T < 1e-4 stop
    within the first-order bound of T's relative error for an exp off by
    4e-6 relative, the T > 0.5 observation likewise):
      * a pixel's last contributor / contributor count may differ only where
        stop_near is set;
      * out_observe[g] may differ from the oracle's by at most obs_near[g]
        (the number of g's blends whose T > 0.5 test was near 0.5);
      * the per-tile sums equal the sums of the device's own per-pixel counts
        when those are given (else they may differ only in tiles holding a
        stop_near pixel).
    got: any of n_contrib_px, n_contrib2loss_px (H, W), out_observe (P),
    n_consider, n_contrib (tiles).  Prints the mismatch counts; returns them."""
    H, W = rf["stop_near"].shape
    near = rf["stop_near"].astype(bool)
    summary = {}
    for key in ("n_contrib_px", "n_contrib2loss_px"):
        if key in got:
            g = np.asarray(got[key]).astype(np.int64).reshape(H, W)
            bad = g != rf[key].astype(np.int64).reshape(H, W)
            unexplained = np.flatnonzero(bad & ~near)
            summary[key] = int(bad.sum())
            assert unexplained.size == 0, (
                f"{key}: {unexplained.size} pixels differ from the oracle away from the T < 1e-4 threshold; first "
                f"at flat pixel {unexplained[:5].tolist()}: got {g.reshape(-1)[unexplained[:5]].tolist()} ref "
                f"{rf[key].reshape(-1)[unexplained[:5]].tolist()}")
    if "out_observe" in got:
        g = np.asarray(got["out_observe"]).astype(np.int64).ravel()
        r = rf["out_observe"].astype(np.int64).ravel()
        d = np.abs(g - r)
        unexplained = np.flatnonzero(d > rf["obs_near"])
        summary["out_observe"] = int((d > 0).sum())
        assert unexplained.size == 0, (
            f"out_observe: {unexplained.size} Gaussians differ by more than their near-0.5 blends; first "
            f"{unexplained[:5].tolist()}: got {g[unexplained[:5]].tolist()} ref {r[unexplained[:5]].tolist()} "
            f"near {rf['obs_near'][unexplained[:5]].tolist()}")
    near_tiles = _tile_sums(near, W, H) > 0
    for tkey, pkey in (("n_consider", "n_contrib_px"), ("n_contrib", "n_contrib2loss_px")):
        if tkey not in got:
            continue
        g = np.asarray(got[tkey]).astype(np.int64).ravel()
        r = rf[tkey].astype(np.int64).ravel()
        summary[tkey] = int((g != r).sum())
        if pkey in got:
            own = _tile_sums(got[pkey], W, H)
            bad = np.flatnonzero(g != own)
            assert bad.size == 0, (f"{tkey}: {bad.size} tiles differ from the sum of the device's own per-pixel "
                                   f"{pkey}; first {bad[:5].tolist()}: {g[bad[:5]].tolist()} vs {own[bad[:5]].tolist()}")
        else:
            unexplained = np.flatnonzero((g != r) & ~near_tiles)
            assert unexplained.size == 0, (f"{tkey}: {unexplained.size} tiles differ away from the T < 1e-4 "
                                           f"threshold; first {unexplained[:5].tolist()}")
    print(f"blend counts{(' ' + label) if label else ''}: differing entries {summary}; near-threshold pixels "
          f"{int(near.sum())} of {near.size}, near-0.5 blends {int(rf['obs_near'].sum())}", flush=True)
    return summary


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


# ------------------------------------------------ full autograd step vs oracle

PARAM_KEYS = ("means3D", "scales", "rotations", "sh", "opacities")
GRAD_NAMES = {"means3D": "dL_dmeans3D", "scales": "dL_dscales", "rotations": "dL_drotations", "sh": "dL_dsh",
              "opacities": "dL_dopacity"}


def autograd_step(scene, cam, bg=(0.0, 0.0, 0.0), cl=None, ext=None, avoid=False, dL_dimage=None, loss_fn=None):
    """One training step through the drop-in autograd API, in the order
    gaussian_renderer uses it (preprocess_gaussians -> retain_grad on means2D ->
    render_gaussians with a means2D_abs leaf -> backward).  cl / ext: the
    compute_locally and extended_compute_locally tile masks (numpy, or None);
    avoid: cuda_args["avoid_pixel_all2all"].  The backward takes dL/dimage
    (dL_dimage) or the gradient of loss_fn(color).  Returns the forward
    outputs, the seven gradients and the render's saved buffers."""
    from blitzgs_amd.rasterizer import GaussianRasterizer
    rs = settings_for(cam, bg=bg)
    params = {k: to_dev(scene[k]).requires_grad_(True) for k in PARAM_KEYS}
    ras = GaussianRasterizer(rs)
    cuda_args = {"avoid_pixel_all2all": bool(avoid), "stats_collector": {}}
    means2D, rgb, conic_opacity, radii, depths = ras.preprocess_gaussians(
        params["means3D"], params["scales"], params["rotations"], params["sh"], params["opacities"], cuda_args)
    means2D.retain_grad()
    P = means2D.shape[0]
    means2D_abs = torch.zeros((P, 3), device="cuda", requires_grad=True) + 0
    means2D_abs.retain_grad()
    all_map = torch.zeros((P, 5), device="cuda")
    dcl = None if cl is None else to_dev(np.asarray(cl, np.uint8)).bool()
    dext = None if ext is None else to_dev(np.asarray(ext, np.uint8)).bool()
    color, n_render, n_consider, n_contrib, out_observe, _, _ = ras.render_gaussians(
        means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, dcl, dext, cuda_args)
    node = color.grad_fn
    R = int(node.num_rendered)
    geom, binning, img = node.saved_tensors[5:8]
    views = buffer_views(R, int(cam["W"]), int(cam["H"]), binning, img, P, depths, geom)
    if loss_fn is None:
        torch.autograd.backward([color], [to_dev(dL_dimage)])
    else:
        loss_fn(color).backward()
    torch.cuda.synchronize()
    out = dict(R=R, color=color, n_render=n_render, n_consider=n_consider, n_contrib=n_contrib,
               out_observe=out_observe, means2D=means2D, rgb=rgb, conic_opacity=conic_opacity, radii=radii,
               depths=depths, dL_dmeans2D=means2D.grad, dL_dmeans2D_abs=means2D_abs.grad, stats=cuda_args,
               **views)
    for k in PARAM_KEYS:
        out[GRAD_NAMES[k]] = params[k].grad
    return out


def oracle_step(scene, cam, bg=(0.0, 0.0, 0.0), cl_fwd=None, cl_bwd=None, dL_dimage=None, dL_dimage_fn=None):
    """The CPU oracle's forward (tile mask cl_fwd) and backward (mask cl_bwd,
    over the forward's lists and per-pixel state).  dL/dimage is given, or
    computed from the oracle's image by dL_dimage_fn."""
    from oracle import oracle as O
    bgv = np.asarray(bg, np.float32)
    pre, bn, rf = O.full_forward(cam, scene, bg=bgv, compute_locally=cl_fwd)
    dLd = dL_dimage if dL_dimage_fn is None else dL_dimage_fn(rf["color"])
    rb = O.render_bwd(cam["W"], cam["H"], bgv, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"],
                      bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd, cl_bwd)
    pb = O.preprocess_bwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"], pre["radii"],
                          pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic_opacity"], rb["dL_dcolors"])
    return pre, bn, rf, rb, pb


def check_step(g, pre, bn, rf, rb, pb, tol=1e-3, binning=True, label=""):
    """The bar: preprocess outputs and binning arrays bit-exact; image and
    transmittance within 1e-4 max-abs, the per-pixel / per-tile / per-Gaussian
    counts equal except at decisions the oracle marks as near their
    thresholds (assert_blend_counts); the seven gradients within tol relative
    L2."""
    for k in ("means2D", "depths", "radii", "conic_opacity", "rgb"):
        assert_bitexact(np_(g[k]), pre[k], k)
    assert g["R"] == bn["R"], (g["R"], bn["R"])
    if binning:
        assert_bitexact(np_(g["point_list"]).view(np.uint32), bn["point_list"], "point_list")
        assert_bitexact(np_(g["keys"]).view(np.uint64), bn["keys"], "point_list_keys")
    assert_bitexact(np_(g["ranges"]).view(np.uint32), bn["ranges"], "ranges")
    assert_bitexact(np_(g["n_render"]), rf["n_render"], "n_render")
    assert_close_abs(np_(g["color"]), rf["color"], "color")
    assert_close_abs(np_(g["final_T"]), rf["final_T"], "final_T")
    assert_blend_counts(dict(n_contrib_px=np_(g["n_contrib_px"]).view(np.uint32),
                             n_contrib2loss_px=np_(g["n_contrib2loss_px"]).view(np.uint32),
                             out_observe=np_(g["out_observe"]), n_consider=np_(g["n_consider"]),
                             n_contrib=np_(g["n_contrib"])), rf, label)
    errs = {"dL_dmeans2D": rel_l2(np_(g["dL_dmeans2D"]), rb["dL_dmeans2D"][:, :2]),
            "dL_dmeans2D_abs": rel_l2(np_(g["dL_dmeans2D_abs"]), rb["dL_dmeans2D_abs"])}
    for k in PARAM_KEYS:
        n = GRAD_NAMES[k]
        errs[n] = rel_l2(np_(g[n]), pb[n])
    bad = {k: v for k, v in errs.items() if not v < tol}
    assert not bad, f"gradients above {tol} relative L2: {bad} (all: {errs})"
    # the gradients are not trivially zero
    assert np.linalg.norm(pb["dL_dsh"]) > 0 and np.linalg.norm(rb["dL_dmeans2D"]) > 0
    return errs
