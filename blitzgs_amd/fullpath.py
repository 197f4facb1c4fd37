"""The full-image rasterize path of diff-gaussian-rasterization_f:
GaussianRasterizer.forward (the eval / render_imp path, differentiable),
render_simp (the importance accumulation of the Gaussian-pruning steps) and
markVisible.

Mirrors BlitzGS submodule/diff-gaussian-rasterization_f:
  diff_gaussian_rasterization_f/__init__.py:319-646
      rasterize_gaussians, rasterize_gaussians_simp, rasterize_gaussians_depth,
      _RasterizeGaussians (forward, render_simp, render_depth, backward)
  diff_gaussian_rasterization_f/__init__.py:660-810   GaussianRasterizer methods
  rasterize_points.cu:370-805   RasterizeGaussiansCUDA, RasterizeGaussiansSimpCUDA,
                                RasterizeGaussiansBackwardCUDA, markVisible
Same arguments, return tuples and gradient order.  The work is done by
libblitzgs_amd.so: gs_preprocess_forward_full, gs_render_full_count /
gs_render_full_forward (tile-culled binning + blend), gs_render_full_depth,
gs_render_full_backward,
gs_preprocess_backward_full, gs_mark_visible.

The reference keeps its intermediate state in four byte buffers
(geom / binning / img / sample).  Here geomBuffer holds the preprocess
outputs followed by the render's geometry workspace and a 256-byte header
(the instance count), binningBuffer and imgBuffer are the render's
workspaces, and sampleBuffer is empty: the backward replays the blend per
pixel from the final transmittance instead of from per-bucket samples.
render_depth (no caller in BlitzGS, no backward) runs the same preprocess and
binning and gs_render_full_depth's blend.
"""
import torch

from . import _lib
from ._lib import check, ptr


def _stream(device):
    return _lib.stream_of(device)


def _given(t):
    """The reference passes empty tensors (torch.Tensor([])) for unused inputs."""
    return t is not None and isinstance(t, torch.Tensor) and t.numel() > 0


def _f32(t, dev):
    return t.to(device=dev, dtype=torch.float32).contiguous()


def _align16(t):
    if t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _a256(n):
    return (n + 255) // 256 * 256


class _Geom:
    """Byte layout of geomBuffer: header (instance count), the preprocess
    outputs, then the render's geometry workspace."""

    def __init__(self, P, W, H):
        self.P = P
        o = 256                                  # header: int64 instance count
        self.off = {}
        for name, nbytes in [("means2D", 8 * P), ("depths", 4 * P), ("cov3D", 24 * P), ("conic", 16 * P),
                             ("rgb", 12 * P), ("clamped", 3 * P), ("rects", 8 * P), ("tiles", 4 * P)]:
            self.off[name] = o
            o = _a256(o + nbytes)
        self.off["render"] = o
        self.total = o + int(_lib.load().gs_render_geom_bytes(P, W, H))

    def views(self, buf):
        P = self.P

        def v(name, dtype, shape, nbytes):
            o = self.off[name]
            return buf[o:o + nbytes].view(dtype).view(shape)
        return dict(
            means2D=v("means2D", torch.float32, (P, 2), 8 * P), depths=v("depths", torch.float32, (P,), 4 * P),
            cov3D=v("cov3D", torch.float32, (P, 6), 24 * P), conic=v("conic", torch.float32, (P, 4), 16 * P),
            rgb=v("rgb", torch.float32, (P, 3), 12 * P),
            clamped=buf[self.off["clamped"]:self.off["clamped"] + 3 * P].view(P, 3),
            rects=v("rects", torch.float32, (P, 2), 8 * P), tiles=v("tiles", torch.int32, (P,), 4 * P))

    def render_ws(self, buf):
        return buf[self.off["render"]:]


def _inputs(rs, means3D, dc, sh, colors_precomp, opacities, scales, rotations, cov3D_precomp):
    if means3D.ndimension() != 2 or means3D.size(1) != 3:
        raise RuntimeError("means3D must have dimensions (num_points, 3)")
    if not means3D.is_cuda:
        raise RuntimeError("means3D must be a HIP device tensor (blitzgs_amd has no CPU path)")
    dev = means3D.device
    P = means3D.size(0)
    cp = _f32(colors_precomp, dev) if _given(colors_precomp) else None
    c3 = _f32(cov3D_precomp, dev) if _given(cov3D_precomp) else None
    d = _f32(dc, dev).reshape(P, 3) if _given(dc) else None
    rest = _f32(sh, dev).reshape(P, -1, 3) if _given(sh) else None
    M = rest.size(1) if rest is not None else 0
    if cp is None and d is None:
        raise RuntimeError("provide either dc (+ sh) or colors_precomp")
    sc = _f32(scales, dev) if _given(scales) else None
    rot = _align16(_f32(rotations, dev)) if _given(rotations) else None
    return dict(dev=dev, P=P, M=M, means3D=_f32(means3D, dev), dc=d, rest=rest, colors_precomp=cp,
                cov3D_precomp=c3, opacities=_f32(opacities, dev), scales=sc, rotations=rot,
                view=_f32(rs.viewmatrix, dev), proj=_f32(rs.projmatrix, dev), campos=_f32(rs.campos, dev),
                bg=_f32(rs.bg, dev))


def _forward(rs, x, culling, flag_max_count, simp, depth=False):
    """Preprocess + binning + blend.  Returns (color, radii, accum_max_count,
    accum_weights, accum_weights_count, geom, binning, img, R); with depth the
    third item is the dict of render_depth's per-pixel outputs."""
    dev, P = x["dev"], x["P"]
    H, W = int(rs.image_height), int(rs.image_width)
    lib = _lib.load()
    s = _stream(dev)
    gl = _Geom(P, W, H)
    geom = torch.empty(gl.total, dtype=torch.uint8, device=dev)
    g = gl.views(geom)
    radii = torch.empty(P, dtype=torch.int32, device=dev)
    color = torch.empty((3, H, W), dtype=torch.float32, device=dev)
    amc = torch.empty(P, dtype=torch.float32, device=dev)
    aw = torch.empty(P, dtype=torch.float32, device=dev) if simp else None
    awc = torch.empty(P, dtype=torch.int32, device=dev) if simp else None
    if culling is None or culling.numel() == 0:
        cull = torch.zeros(P, dtype=torch.uint8, device=dev)
    else:
        cull = culling.to(device=dev).reshape(-1).to(torch.uint8).contiguous()
        if cull.numel() != P:
            raise RuntimeError("culling must have one entry per Gaussian")
    if P > 0:
        check(lib.gs_preprocess_forward_full(
            P, int(rs.sh_degree), x["M"], ptr(x["means3D"]), ptr(x["scales"]), ptr(x["rotations"]), ptr(x["dc"]),
            ptr(x["rest"]), ptr(x["opacities"]), ptr(x["colors_precomp"]), ptr(x["cov3D_precomp"]), ptr(cull),
            float(rs.scale_modifier), ptr(x["view"]), ptr(x["proj"]), ptr(x["campos"]), float(rs.tanfovx),
            float(rs.tanfovy), H, W, ptr(g["means2D"]), ptr(g["depths"]), ptr(radii), ptr(g["cov3D"]),
            ptr(g["conic"]), ptr(g["rgb"]), ptr(g["clamped"]), ptr(g["rects"]), ptr(g["tiles"]), s),
            "gs_preprocess_forward_full")
    rws = gl.render_ws(geom)
    img = torch.empty(int(lib.gs_render_img_bytes(W, H)), dtype=torch.uint8, device=dev)
    colors = x["colors_precomp"] if x["colors_precomp"] is not None else g["rgb"]
    want_amc = flag_max_count or simp
    cap = None if depth else _lib.RESERVE.capacity(dev)
    if cap is not None:
        # one call, no host round trip between the count and the duplication
        binning = torch.empty(int(lib.gs_render_binning_bytes(cap)), dtype=torch.uint8, device=dev)
        Rv = _lib.C.c_int64(0)
        check(lib.gs_render_full_forward_reserved(
            P, cap, W, H, ptr(x["bg"]), ptr(g["means2D"]), ptr(g["depths"]), ptr(radii), ptr(g["rects"]),
            ptr(g["conic"]), ptr(colors), ptr(rws), ptr(binning), ptr(img), ptr(color),
            ptr(amc) if want_amc else None, ptr(aw), ptr(awc), _lib.C.byref(Rv), s), "gs_render_full_forward_reserved")
        _lib.RESERVE.update(dev, int(Rv.value))
        if Rv.value <= cap:
            R = int(Rv.value)
            geom[:8].view(torch.int64).fill_(R)
            if not want_amc:
                amc.zero_()
            _lib.debug_sync(getattr(rs, "debug", False), "rasterize_gaussians")
            return color, radii, amc, aw, awc, geom, binning, img, R
    # the exact path: first forward on the device, more instances than
    # reserved, or the depth render
    R = _lib.C.c_int64(0)
    check(lib.gs_render_full_count(P, W, H, ptr(g["means2D"]), ptr(radii), ptr(g["rects"]), ptr(g["conic"]),
                                   ptr(rws), _lib.C.byref(R), s), "gs_render_full_count")
    R = int(R.value)
    _lib.RESERVE.update(dev, R)
    geom[:8].view(torch.int64).fill_(R)
    binning = torch.empty(int(lib.gs_render_binning_bytes(R)), dtype=torch.uint8, device=dev)
    if depth:
        d = dict(out_pts=torch.empty((3, H, W), dtype=torch.float32, device=dev),
                 depth=torch.empty((1, H, W), dtype=torch.float32, device=dev),
                 accum_alpha=torch.empty((1, H, W), dtype=torch.float32, device=dev),
                 gidx=torch.empty((1, H, W), dtype=torch.int32, device=dev),
                 discriminants=torch.empty((1, H, W), dtype=torch.float32, device=dev))
        check(lib.gs_render_full_depth(P, R, W, H, ptr(x["bg"]), ptr(g["means2D"]), ptr(g["depths"]), ptr(radii),
                                       ptr(g["rects"]), ptr(g["conic"]), ptr(colors), ptr(x["means3D"]),
                                       ptr(x["scales"]), ptr(x["rotations"]), ptr(x["proj"]), ptr(x["campos"]),
                                       ptr(rws), ptr(binning), ptr(img), ptr(color), ptr(d["out_pts"]),
                                       ptr(d["depth"]), ptr(d["accum_alpha"]), ptr(d["gidx"]),
                                       ptr(d["discriminants"]), s), "gs_render_full_depth")
        _lib.debug_sync(getattr(rs, "debug", False), "rasterize_gaussians_depth")
        return color, radii, d, None, None, geom, binning, img, R
    check(lib.gs_render_full_forward(P, R, W, H, ptr(x["bg"]), ptr(g["means2D"]), ptr(g["depths"]), ptr(radii),
                                     ptr(g["rects"]), ptr(g["conic"]), ptr(colors), ptr(rws), ptr(binning), ptr(img),
                                     ptr(color), ptr(amc) if want_amc else None, ptr(aw), ptr(awc),
                                     s), "gs_render_full_forward")
    if not want_amc:
        amc.zero_()
    _lib.debug_sync(getattr(rs, "debug", False), "rasterize_gaussians")
    return color, radii, amc, aw, awc, geom, binning, img, R


def _backward(rs, x, radii, geom, R, binning, img, grad_out_color):
    """Render backward + preprocess backward; the reference's 9-tuple
    (dL_dmeans2D, dL_dcolors, dL_dopacity, dL_dmeans3D, dL_dcov3D, dL_ddc,
    dL_dsh, dL_dscales, dL_drotations)."""
    dev, P, M = x["dev"], x["P"], x["M"]
    H, W = int(grad_out_color.size(1)), int(grad_out_color.size(2))
    lib = _lib.load()
    s = _stream(dev)
    f32 = dict(device=dev, dtype=torch.float32)
    dL_dmeans2D = torch.empty((P, 3), **f32)
    dL_dco = torch.empty((P, 4), **f32)
    dL_dcolors = torch.empty((P, 3), **f32)
    dL_dopacity = torch.empty((P, 1), **f32)
    dL_dmeans3D = torch.empty((P, 3), **f32)
    dL_dcov3D = torch.empty((P, 6), **f32)
    dL_ddc = torch.empty((P, 1, 3), **f32)
    dL_dsh = torch.empty((P, M, 3), **f32)
    dL_dscales = torch.empty((P, 3), **f32)
    dL_drotations = torch.empty((P, 4), **f32)
    if P > 0:
        gl = _Geom(P, W, H)
        g = gl.views(geom)
        dpix = grad_out_color.to(**f32).contiguous()
        check(lib.gs_render_full_backward(P, R, W, H, ptr(x["bg"]), ptr(g["means2D"]), ptr(g["conic"]),
                                          ptr(gl.render_ws(geom)), ptr(binning), ptr(img), ptr(dpix),
                                          ptr(dL_dmeans2D), ptr(dL_dco), ptr(dL_dcolors), s),
              "gs_render_full_backward")
        scales = x["scales"] if x["cov3D_precomp"] is None else None
        rots = x["rotations"] if x["cov3D_precomp"] is None else None
        check(lib.gs_preprocess_backward_full(
            P, int(rs.sh_degree), M, ptr(x["means3D"]), ptr(scales), ptr(rots), ptr(x["dc"]), ptr(x["rest"]),
            ptr(x["colors_precomp"]), ptr(x["cov3D_precomp"]), float(rs.scale_modifier), ptr(x["view"]),
            ptr(x["proj"]), ptr(x["campos"]), float(rs.tanfovx), float(rs.tanfovy), H, W, ptr(radii),
            ptr(g["cov3D"]), ptr(g["clamped"]), ptr(dL_dmeans2D), ptr(dL_dco), ptr(dL_dcolors), ptr(dL_dmeans3D),
            ptr(dL_dcov3D), ptr(dL_ddc), ptr(dL_dsh), ptr(dL_dscales), ptr(dL_drotations), ptr(dL_dopacity), s),
            "gs_preprocess_backward_full")
        _lib.debug_sync(getattr(rs, "debug", False), "rasterize_gaussians_backward")
    return dL_dmeans2D, dL_dcolors, dL_dopacity, dL_dmeans3D, dL_dcov3D, dL_ddc, dL_dsh, dL_dscales, dL_drotations


def _num_buckets(img, R, W, H):
    """sum over tiles of ceil(len / 32) (perTileBucketCount)."""
    gx, gy = (W + 15) // 16, (H + 15) // 16
    rng = img[:8 * gx * gy].view(torch.int32).view(gx * gy, 2).to(torch.int64)
    return int(((rng[:, 1] - rng[:, 0] + 31) // 32).sum().item())


class _RasterizeGaussians(torch.autograd.Function):
    """_f __init__.py:398-646."""

    @staticmethod
    def forward(ctx, means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                flag_max_count, culling, raster_settings):
        x = _inputs(raster_settings, means3D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp)
        color, radii, amc, _, _, geom, binning, img, R = _forward(raster_settings, x, culling, bool(flag_max_count),
                                                                  False)
        ctx.raster_settings = raster_settings
        ctx.x = {k: v for k, v in x.items()}
        ctx.R = R
        ctx.shapes = (tuple(dc.shape) if _given(dc) else None, tuple(sh.shape) if _given(sh) else None)
        ctx.save_for_backward(radii, geom, binning, img)
        ctx.mark_non_differentiable(radii, amc)
        # radii and the max-count output take no gradient: not zero-filled
        ctx.set_materialize_grads(False)
        return color, radii, amc

    @staticmethod
    def backward(ctx, grad_out_color, *_):
        radii, geom, binning, img = ctx.saved_tensors
        if grad_out_color is None:
            rs = ctx.raster_settings
            grad_out_color = torch.zeros((3, int(rs.image_height), int(rs.image_width)), device=radii.device,
                                         dtype=torch.float32)
        (g_m2d, g_col, g_op, g_m3d, g_cov, g_dc, g_sh, g_sc, g_rot) = _backward(
            ctx.raster_settings, ctx.x, radii, geom, ctx.R, binning, img, grad_out_color)
        x = ctx.x
        if ctx.shapes[0] is not None:
            g_dc = g_dc.reshape(ctx.shapes[0])
        if ctx.shapes[1] is not None:
            g_sh = g_sh.reshape(ctx.shapes[1])
        return (g_m3d, g_m2d, g_dc if x["dc"] is not None else None, g_sh if x["rest"] is not None else None,
                g_col if x["colors_precomp"] is not None else None, g_op,
                g_sc if x["scales"] is not None else None, g_rot if x["rotations"] is not None else None,
                g_cov if x["cov3D_precomp"] is not None else None, None, None, None)


    @staticmethod
    def render_simp(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, culling,
                    raster_settings):
        """_f __init__.py:476-511."""
        return rasterize_gaussians_simp(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations,
                                        cov3Ds_precomp, culling, raster_settings)

    @staticmethod
    def render_depth(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp, culling,
                     raster_settings):
        """_f __init__.py:525-577."""
        return rasterize_gaussians_depth(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations,
                                         cov3Ds_precomp, culling, raster_settings)


def rasterize_gaussians(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                        flag_max_count, culling, raster_settings):
    return _RasterizeGaussians.apply(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations,
                                     cov3Ds_precomp, flag_max_count, culling, raster_settings)


@torch.no_grad()
def rasterize_gaussians_simp(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                             culling, raster_settings):
    """_RasterizeGaussians.render_simp (_f __init__.py:476-511): returns
    (color, radii, accum_weights, accum_weights_count, accum_max_count)."""
    x = _inputs(raster_settings, means3D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp)
    color, radii, amc, aw, awc, _, _, _, _ = _forward(raster_settings, x, culling, True, True)
    return color, radii, aw, awc, amc


def _depth_inputs(raster_settings, means3D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp):
    x = _inputs(raster_settings, means3D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp)
    if x["scales"] is None or x["rotations"] is None:
        # the depth kernel reads every blended Gaussian's scale and rotation
        raise RuntimeError("render_depth needs scales and rotations (it intersects the camera ray with each "
                           "Gaussian's ellipsoid)")
    return x


@torch.no_grad()
def rasterize_gaussians_depth(means3D, means2D, dc, sh, colors_precomp, opacities, scales, rotations, cov3Ds_precomp,
                              culling, raster_settings):
    """_RasterizeGaussians.render_depth (_f __init__.py:525-577): returns the
    dict {render, out_pts, rendered_depth, discriminants, gidx, accum_alpha}."""
    x = _depth_inputs(raster_settings, means3D, dc, sh, colors_precomp, opacities, scales, rotations,
                      cov3Ds_precomp)
    color, _, d, _, _, _, _, _, _ = _forward(raster_settings, x, culling, False, False, depth=True)
    return {"render": color, "out_pts": d["out_pts"], "rendered_depth": d["depth"],
            "discriminants": d["discriminants"], "gidx": d["gidx"], "accum_alpha": d["accum_alpha"]}


@torch.no_grad()
def mark_visible(positions, viewmatrix, projmatrix):
    """markVisible (_f rasterize_points.cu:785-805): view-space z > 0.2."""
    if not positions.is_cuda:
        raise RuntimeError("positions must be a HIP device tensor")
    dev = positions.device
    P = positions.size(0)
    present = torch.empty(P, dtype=torch.bool, device=dev)
    m = _f32(positions, dev)
    check(_lib.load().gs_mark_visible(P, ptr(m), ptr(_f32(viewmatrix, dev)), ptr(_f32(projmatrix, dev)),
                                      ptr(present), _stream(dev)), "gs_mark_visible")
    return present


# ------------------------------------------------------------ raw _C entry points

def _settings(bg, scale_modifier, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height, image_width, degree,
              campos, prefiltered, debug):
    from .rasterizer import GaussianRasterizationSettings
    return GaussianRasterizationSettings(image_height=int(image_height), image_width=int(image_width),
                                         tanfovx=float(tan_fovx), tanfovy=float(tan_fovy), bg=bg,
                                         scale_modifier=float(scale_modifier), viewmatrix=viewmatrix,
                                         projmatrix=projmatrix, sh_degree=int(degree), campos=campos,
                                         prefiltered=bool(prefiltered), debug=bool(debug))


def C_rasterize_gaussians(background, means3D, colors, opacity, scales, rotations, scale_modifier, cov3D_precomp,
                          viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height, image_width, dc, sh, degree,
                          campos, prefiltered, flag_max_count, culling, debug):
    """_C.rasterize_gaussians (rasterize_points.cu:370-475): returns
    (num_rendered, num_buckets, color, accum_max_count, radii, geomBuffer,
    binningBuffer, imgBuffer, sampleBuffer)."""
    rs = _settings(background, scale_modifier, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height,
                   image_width, degree, campos, prefiltered, debug)
    x = _inputs(rs, means3D, dc, sh, colors, opacity, scales, rotations, cov3D_precomp)
    color, radii, amc, _, _, geom, binning, img, R = _forward(rs, x, culling, bool(flag_max_count), False)
    g = _Geom(x["P"], int(image_width), int(image_height)).views(geom)
    num_rendered = int(g["tiles"].to(torch.int64).sum().item()) if x["P"] else 0
    nb = _num_buckets(img, R, int(image_width), int(image_height))
    sample = torch.empty(0, dtype=torch.uint8, device=x["dev"])
    return num_rendered, nb, color, amc, radii, geom, binning, img, sample


def C_rasterize_gaussians_backward(background, means3D, radii, colors, scales, rotations, scale_modifier,
                                   cov3D_precomp, viewmatrix, projmatrix, tan_fovx, tan_fovy, dL_dout_color, dc, sh,
                                   degree, campos, geomBuffer, R, binningBuffer, imageBuffer, B, sampleBuffer, debug):
    """_C.rasterize_gaussians_backward (rasterize_points.cu:697-783): returns
    (dL_dmeans2D, dL_dcolors, dL_dopacity, dL_dmeans3D, dL_dcov3D, dL_ddc,
    dL_dsh, dL_dscales, dL_drotations).  R and B (the reference's counts) are
    not needed: the instance count travels in geomBuffer's header."""
    H, W = int(dL_dout_color.size(1)), int(dL_dout_color.size(2))
    rs = _settings(background, scale_modifier, viewmatrix, projmatrix, tan_fovx, tan_fovy, H, W, degree, campos,
                   False, debug)
    x = _inputs(rs, means3D, dc, sh, colors, torch.zeros(means3D.size(0), device=means3D.device), scales,
                rotations, cov3D_precomp)
    R_ours = int(geomBuffer[:8].view(torch.int64).item())
    return _backward(rs, x, radii, geomBuffer, R_ours, binningBuffer, imageBuffer, dL_dout_color)


def C_rasterize_gaussians_depth(background, means3D, colors, opacity, scales, rotations, scale_modifier,
                                cov3D_precomp, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height, image_width,
                                dc, sh, degree, campos, prefiltered, culling, debug):
    """_C.rasterize_gaussians_depth (rasterize_points.cu:588-690): returns
    (num_rendered, color, out_pts, depth, accum_alpha, gidx, discriminants,
    radii, geomBuffer, binningBuffer, imgBuffer)."""
    rs = _settings(background, scale_modifier, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height,
                   image_width, degree, campos, prefiltered, debug)
    x = _depth_inputs(rs, means3D, dc, sh, colors, opacity, scales, rotations, cov3D_precomp)
    color, radii, d, _, _, geom, binning, img, R = _forward(rs, x, culling, False, False, depth=True)
    g = _Geom(x["P"], int(image_width), int(image_height)).views(geom)
    num_rendered = int(g["tiles"].to(torch.int64).sum().item()) if x["P"] else 0
    return (num_rendered, color, d["out_pts"], d["depth"], d["accum_alpha"], d["gidx"], d["discriminants"], radii,
            geom, binning, img)


def C_rasterize_gaussians_simp(background, means3D, colors, opacity, scales, rotations, scale_modifier,
                               cov3D_precomp, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height, image_width,
                               dc, sh, degree, campos, prefiltered, culling, debug):
    """_C.rasterize_gaussians_simp (rasterize_points.cu:477-583): returns
    (num_rendered, color, accum_weights, accum_weights_count, accum_max_count,
    radii, geomBuffer, binningBuffer, imgBuffer)."""
    rs = _settings(background, scale_modifier, viewmatrix, projmatrix, tan_fovx, tan_fovy, image_height,
                   image_width, degree, campos, prefiltered, debug)
    x = _inputs(rs, means3D, dc, sh, colors, opacity, scales, rotations, cov3D_precomp)
    color, radii, amc, aw, awc, geom, binning, img, R = _forward(rs, x, culling, True, True)
    g = _Geom(x["P"], int(image_width), int(image_height)).views(geom)
    num_rendered = int(g["tiles"].to(torch.int64).sum().item()) if x["P"] else 0
    return num_rendered, color, aw, awc, amc, radii, geom, binning, img
