"""The reference extensions' raw operator signatures (their pybind `_C` modules).

diff_gaussian_rasterization_f._C / diff_gaussian_rasterization_r._C expose
(ext.cpp of each package; C++ signatures in rasterize_points.h):
  preprocess_gaussians            _f/rasterize_points.cu:834-923
  preprocess_gaussians_backward   _f/rasterize_points.cu:926-1029
  render_gaussians                _r/rasterize_points.cu:273-361
  render_gaussians_backward       _r/rasterize_points.cu:363-436
  rasterize_gaussians             _f/rasterize_points.cu:370-475
  rasterize_gaussians_simp        _f/rasterize_points.cu:477-583
  rasterize_gaussians_depth       _f/rasterize_points.cu:588-690
  rasterize_gaussians_backward    _f/rasterize_points.cu:697-783
  mark_visible                    _f/rasterize_points.cu:785-805
  get_local2j_ids_bool            _f/rasterize_points.cu:258-289
  get_local2j_ids_bool_adjust_mode6  _f/rasterize_points.cu:337-367
  adamUpdate                      _f/rasterize_points.cu:807-832
Same positional arguments and return tuples; `args` is the reference's
cuda_args dict (its "stats_collector" entry receives forward_render_time /
backward_render_time in ms).  Not provided: the image-tile utilities of the
multi-GPU path (_r ext.cpp:20-34) and _f's own older fusedssim /
fusedssim_backward pair (_f ext.cpp:23-24, conv.cu:390-470; nothing in BlitzGS
calls it -- the training loss uses the fused_ssim package, blitzgs_amd.ssim).
"""
import torch

from . import rasterizer as _r
from .adam import adamUpdate  # noqa: F401  (the reference's _C.adamUpdate)
from .routing import get_local2j_ids_bool, get_local2j_ids_bool_adjust_mode6  # noqa: F401


class _RS:
    """Minimal settings record for the raw calls."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def preprocess_gaussians(means3D, scales, rotations, sh, opacity, scale_modifier, viewmatrix, projmatrix, tan_fovx,
                         tan_fovy, image_height, image_width, degree, campos, prefiltered, debug, args=None):
    rs = _RS(scale_modifier=scale_modifier, viewmatrix=viewmatrix, projmatrix=projmatrix, tanfovx=tan_fovx,
             tanfovy=tan_fovy, image_height=image_height, image_width=image_width, sh_degree=degree, campos=campos,
             debug=debug)
    return _r._preprocess_forward_raw(means3D, scales, rotations, sh, opacity, rs)


def preprocess_gaussians_backward(radii, cov3D, clamped, means3D, scales, rotations, sh, scale_modifier, viewmatrix,
                                  projmatrix, tan_fovx, tan_fovy, image_height, image_width, degree, campos,
                                  dL_dmeans2D, dL_dconic_opacity, dL_dcolors, R, debug, args=None):
    rs = _RS(scale_modifier=scale_modifier, viewmatrix=viewmatrix, projmatrix=projmatrix, tanfovx=tan_fovx,
             tanfovy=tan_fovy, image_height=image_height, image_width=image_width, sh_degree=degree, campos=campos,
             debug=debug)
    return _r._preprocess_backward_raw(radii, cov3D, clamped, means3D, scales, rotations, sh, rs, dL_dmeans2D,
                                       dL_dconic_opacity, dL_dcolors)


def render_gaussians(background, image_height, image_width, means2D, depths, radii, conic_opacity, rgb,
                     compute_locally, viewmatrix, campos, tan_fovx, tan_fovy, all_map, render_geo, debug, args=None):
    timing = _r._want_timing(args)
    H, W = int(image_height), int(image_width)
    # render_geo: the maps in the colour's walk of the lists
    geo = (tan_fovx, tan_fovy, all_map) if render_geo else None
    # render_geo off: the zero maps and plane depth are cleared by the blend
    zmaps = None
    if not render_geo:
        zmaps = torch.empty(((6 * H * W + 3) // 4) * 4, device=means2D.device, dtype=torch.float32)
    res = _r._render_forward_raw(background, H, W, means2D, depths, radii, conic_opacity, rgb, compute_locally, timing,
                                 bool(debug), geo=geo, clear=zmaps)
    R, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, ms = res[:10]
    if timing:
        args["stats_collector"]["forward_render_time"] = ms
    if render_geo:
        out_all_map, out_plane_depth = res[10:]
    else:
        maps = zmaps[:6 * H * W].view(6, H, W)
        out_all_map, out_plane_depth = maps[:5], maps[5:]
    return R, color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth, geom, binning, img


def render_gaussians_backward(background, tan_fovx, tan_fovy, all_map_pixels, all_maps, R, geomBuffer, binningBuffer,
                              imageBuffer, compute_locally, dL_dout_color, dL_dout_all_map, dL_dout_plane_depth,
                              means2D, conic_opacity, rgb, render_geo, debug, args=None):
    H, W = int(dL_dout_color.size(1)), int(dL_dout_color.size(2))
    timing = _r._want_timing(args)
    if render_geo:
        (dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms,
         dL_dall_map) = _r._render_backward_raw(
            background, int(R), H, W, means2D, conic_opacity, rgb, compute_locally, geomBuffer, binningBuffer,
            imageBuffer, dL_dout_color.contiguous(), 3, timing, bool(debug),
            geo=(tan_fovx, tan_fovy, all_map_pixels, all_maps, dL_dout_all_map, dL_dout_plane_depth))
    else:
        dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms = _r._render_backward_raw(
            background, int(R), H, W, means2D, conic_opacity, rgb, compute_locally, geomBuffer, binningBuffer,
            imageBuffer, dL_dout_color.contiguous(), 3, timing, bool(debug))
        dL_dall_map = torch.zeros((means2D.size(0), 5), device=means2D.device, dtype=torch.float32)
    if timing:
        args["stats_collector"]["backward_render_time"] = ms
    return dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, dL_dall_map


from .fullpath import C_rasterize_gaussians as rasterize_gaussians  # noqa: E402,F401
from .fullpath import C_rasterize_gaussians_backward as rasterize_gaussians_backward  # noqa: E402,F401
from .fullpath import C_rasterize_gaussians_simp as rasterize_gaussians_simp  # noqa: E402,F401
from .fullpath import mark_visible  # noqa: E402,F401

from .fullpath import C_rasterize_gaussians_depth as rasterize_gaussians_depth  # noqa: E402,F401
