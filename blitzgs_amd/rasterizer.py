"""Python operator layer of the rasterizer: the reference's split training API.

Mirrors BlitzGS submodule/diff-gaussian-rasterization_f/diff_gaussian_rasterization_f/__init__.py
(and the _r package it dispatches render ops to):
  GaussianRasterizationSettings          _f __init__.py:647-659 (_r adds render_geo)
  GaussianRasterizer.preprocess_gaussians _f __init__.py:677-689
  GaussianRasterizer.render_gaussians     _f __init__.py:812-829
  preprocess_gaussians / _PreprocessGaussians   _f __init__.py:55-173
  render_gaussians / _RenderGaussians           _f __init__.py:177-318, _r __init__.py:178-289
Same argument order, return tuples, dtypes, saved buffers and
non-differentiable outputs; the work is done by libblitzgs_amd.so (HIP,
gfx950) through its C ABI.  Differences that do not change results:
  * the (P,3) padding of dL/dmeans2D before the preprocess backward and the
    [:, :2] slice after the render backward are not materialised: the C ABI
    takes a row stride;
  * dL/dall_map (all zeros when render_geo is off) is returned only when the
    all_map input requires a gradient;
  * the preprocess backward's dL/dsh (zero for the invisible Gaussians; the
    reference allocates it with torch::zeros) is allocated by the preprocess
    forward and cleared by the render backward of a render that read this
    call's means2D, while its VALU-bound blend runs (gs_render_backward's
    clear_dst); the preprocess backward then writes only the visible
    Gaussians' rows.
"""
import ctypes as C
from typing import NamedTuple

import torch
import torch.nn as nn

from . import _lib
from ._lib import check, ptr


class GaussianRasterizationSettings(NamedTuple):
    image_height: int
    image_width: int
    tanfovx: float
    tanfovy: float
    bg: torch.Tensor
    scale_modifier: float
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    sh_degree: int
    campos: torch.Tensor
    prefiltered: bool
    debug: bool


def _dev_f32(t, device):
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    return t.to(device=device, dtype=torch.float32).contiguous()


def _aligned(t, nbytes=16):
    t = t.contiguous()
    if t.numel() and t.data_ptr() % nbytes != 0:
        t = t.clone()
    return t


def _require_device(t, name):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a HIP device tensor (blitzgs_amd has no CPU path)")


def _stream(device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _want_timing(cuda_args):
    return isinstance(cuda_args, dict) and isinstance(cuda_args.get("stats_collector"), dict)


# --------------------------------------------------------------- preprocess

def preprocess_gaussians(means3D, scales, rotations, sh, opacities, raster_settings, cuda_args):
    return _PreprocessGaussians.apply(means3D, scales, rotations, sh, opacities, raster_settings, cuda_args)


def _preprocess_forward_raw(means3D, scales, rotations, sh, opacities, rs, keep_cov3D=True, records=False,
                            keep_clamped=True):
    """Direct call of the C ABI; returns the reference's 8-tuple
    (num_rendered, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped).
    keep_cov3D False: cov3D is None (not written; the backward recomputes it
    from scales and rotations).  records True: a 9th element, the backward's
    record buffer (gs_preprocess_forward_rec), follows; with records,
    keep_clamped False leaves clamped None (the records hold the flags)."""
    if means3D.ndimension() != 2 or means3D.size(1) != 3:
        raise RuntimeError("means3D must have dimensions (num_points, 3)")
    _require_device(means3D, "means3D")
    dev = means3D.device
    P = means3D.size(0)
    if sh.size(0) != 0 and (sh.ndimension() != 3 or sh.size(2) != 3 or sh.size(1) < 1):
        raise RuntimeError("sh must have dimensions (num_points, num_sh_coeffs, 3) with num_sh_coeffs >= 1")
    f32 = dict(device=dev, dtype=torch.float32)
    means2D = torch.empty((P, 2), **f32)
    depths = torch.empty((P,), **f32)
    radii = torch.empty((P,), device=dev, dtype=torch.int32)
    cov3D = torch.empty((P, 6), **f32) if keep_cov3D else None
    conic_opacity = torch.empty((P, 4), **f32)
    rgb = torch.empty((P, 3), **f32)
    clamped = torch.empty((P, 3), device=dev, dtype=torch.bool) if keep_clamped or not records else None
    if P != 0:
        if sh.size(0) == 0:
            raise RuntimeError("sh must be provided (precomputed colours are not supported by the split path)")
        means3D = _dev_f32(means3D, dev)
        scales = _dev_f32(scales, dev)
        rotations = _aligned(_dev_f32(rotations, dev))
        sh = _aligned(_dev_f32(sh, dev))
        opacities = _dev_f32(opacities, dev)
        view = _dev_f32(rs.viewmatrix, dev)
        proj = _dev_f32(rs.projmatrix, dev)
        campos = _dev_f32(rs.campos, dev)
        lib = _lib.load()
        args = (P, int(rs.sh_degree), sh.size(1), ptr(means3D), ptr(scales), ptr(rotations), ptr(sh), ptr(opacities),
                float(rs.scale_modifier), ptr(view), ptr(proj), ptr(campos), float(rs.tanfovx), float(rs.tanfovy),
                int(rs.image_height), int(rs.image_width), ptr(means2D), ptr(depths), ptr(radii),
                ptr(cov3D) if cov3D is not None else None, ptr(conic_opacity), ptr(rgb),
                ptr(clamped) if clamped is not None else None)
        if records:
            # torch's caching allocator hands out 512-byte aligned blocks
            rec = torch.empty(lib.gs_preprocess_record_bytes(P), device=dev, dtype=torch.uint8)
            rc = lib.gs_preprocess_forward_rec(*args, ptr(rec), _stream(dev))
            check(rc, "gs_preprocess_forward_rec")
        else:
            rc = lib.gs_preprocess_forward(*args, _stream(dev))
            check(rc, "gs_preprocess_forward")
        _lib.debug_sync(getattr(rs, "debug", False), "gs_preprocess_forward")
    out = (0, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped)
    if records:
        return out + (rec if P != 0 else torch.empty(0, device=dev, dtype=torch.uint8),)
    return out


def _preprocess_backward_raw(radii, cov3D, clamped, means3D, scales, rotations, sh, rs, dL_dmeans2D,
                             dL_dconic_opacity, dL_drgb, records=None, zeroed=None, acc=None):
    """records: the forward's record buffer (_preprocess_forward_raw with
    records=True); then radii, clamped, scales and rotations are not read.
    zeroed (with records): a (P,K,3) dL/dsh output tensor that already holds
    zeros on the current stream; only the visible Gaussians' rows are written
    into it.  acc (with zeroed; (geom, R, W, H) of a split render whose
    backward returned exactly dL_dmeans2D, dL_dconic_opacity and dL_drgb):
    its accumulators are read instead of those dense arrays (the same
    values)."""
    dev = means3D.device
    P = means3D.size(0)
    K = sh.size(1) if sh.ndimension() == 3 else 1
    f32 = dict(device=dev, dtype=torch.float32)
    dL_dmeans3D = torch.empty((P, 3), **f32)
    dL_dscales = torch.empty((P, 3), **f32)
    dL_drotations = torch.empty((P, 4), **f32)
    if zeroed is not None:
        if records is None or tuple(zeroed.shape) != (P, K, 3):
            raise RuntimeError(f"a zeroed dL/dsh needs the record path and shape ({P}, {K}, 3)")
        dL_dsh = zeroed
    else:
        dL_dsh = torch.empty((P, K, 3), **f32)
    dL_dopacity = torch.empty((P, 1), **f32)
    if P != 0:
        means3D = _dev_f32(means3D, dev)
        scales = _dev_f32(scales, dev)
        rotations = _aligned(_dev_f32(rotations, dev))
        sh = _aligned(_dev_f32(sh, dev))
        dL_dmeans2D = _dev_f32(dL_dmeans2D, dev)
        dL_dconic_opacity = _aligned(_dev_f32(dL_dconic_opacity, dev))
        dL_drgb = _dev_f32(dL_drgb, dev)
        view = _dev_f32(rs.viewmatrix, dev)
        proj = _dev_f32(rs.projmatrix, dev)
        campos = _dev_f32(rs.campos, dev)
        lib = _lib.load()
        cov = ptr(cov3D.contiguous()) if cov3D is not None else None
        if records is not None and zeroed is not None and acc is not None and K % 4 == 0:
            if records.numel() != lib.gs_preprocess_record_bytes(P):
                raise RuntimeError("records must be the preprocess forward's record buffer for these Gaussians")
            geom, R, W, H = acc
            pa, pc = C.c_void_p(), C.c_void_p()
            check(lib.gs_render_accumulators(ptr(geom), P, W, H, R, C.byref(pa), C.byref(pc)),
                  "gs_render_accumulators")
            rc = lib.gs_preprocess_backward_rec_acc(
                P, int(rs.sh_degree), K, ptr(records), ptr(sh), float(rs.scale_modifier), ptr(view), ptr(proj),
                ptr(campos), float(rs.tanfovx), float(rs.tanfovy), int(rs.image_height), int(rs.image_width), cov,
                pa, pc, ptr(dL_dmeans3D), ptr(dL_dscales), ptr(dL_drotations), ptr(dL_dsh), ptr(dL_dopacity),
                _stream(dev))
            check(rc, "gs_preprocess_backward_rec_acc")
        elif records is not None:
            if records.numel() != lib.gs_preprocess_record_bytes(P):
                raise RuntimeError("records must be the preprocess forward's record buffer for these Gaussians")
            rc = lib.gs_preprocess_backward_rec(
                P, int(rs.sh_degree), K, ptr(records), ptr(sh), float(rs.scale_modifier), ptr(view), ptr(proj),
                ptr(campos), float(rs.tanfovx), float(rs.tanfovy), int(rs.image_height), int(rs.image_width), cov,
                ptr(dL_dmeans2D), dL_dmeans2D.size(1), ptr(dL_dconic_opacity), ptr(dL_drgb), ptr(dL_dmeans3D),
                ptr(dL_dscales), ptr(dL_drotations), ptr(dL_dsh), ptr(dL_dopacity), 1 if zeroed is not None else 0,
                _stream(dev))
            check(rc, "gs_preprocess_backward_rec")
        else:
            rc = lib.gs_preprocess_backward(
                P, int(rs.sh_degree), K, ptr(means3D), ptr(scales), ptr(rotations), ptr(sh),
                float(rs.scale_modifier), ptr(view), ptr(proj), ptr(campos), float(rs.tanfovx), float(rs.tanfovy),
                int(rs.image_height), int(rs.image_width), ptr(radii.contiguous()), cov, ptr(clamped.contiguous()),
                ptr(dL_dmeans2D), dL_dmeans2D.size(1), ptr(dL_dconic_opacity), ptr(dL_drgb), ptr(dL_dmeans3D),
                ptr(dL_dscales), ptr(dL_drotations), ptr(dL_dsh), ptr(dL_dopacity), _stream(dev))
            check(rc, "gs_preprocess_backward")
        _lib.debug_sync(getattr(rs, "debug", False), "gs_preprocess_backward")
    return dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh, dL_dopacity


class _ZeroedGrads:
    """The preprocess backward's dL/dsh, allocated by its forward.  The first
    render backward of a render that read that call's means2D claims it and
    clears it while it runs (claim(), then cleared() with an event after the
    call); take() hands it to the preprocess backward, which waits for that
    event, or gives None when no render backward cleared it (the preprocess
    backward then writes every row itself).  Once taken it cannot be claimed
    again, so a later render backward never clears a returned gradient."""

    def __init__(self, P, K, dev):
        self.dev = dev
        self.dL_dsh = torch.empty((P, K, 3), device=dev, dtype=torch.float32)
        self.event = None
        self.claimed = False

    def claim(self):
        if self.claimed or self.dL_dsh is None:
            return None
        self.claimed = True
        return self.dL_dsh

    def cleared(self):
        self.event = torch.cuda.Event()
        self.event.record(torch.cuda.current_stream(self.dev))

    def take(self):
        t, self.dL_dsh = self.dL_dsh, None
        if t is None or self.event is None:
            return None
        torch.cuda.current_stream(self.dev).wait_event(self.event)
        return t

    # The same render backward also offers its accumulators: the preprocess
    # backward reads them instead of the dense gradients when the gradients it
    # receives are exactly the tensors that backward returned (no other
    # contribution summed in, nothing changed in place; holding them here also
    # keeps autograd from summing into them in place).
    acc = None

    def offer(self, geom, R, W, H, grads):
        self.acc = (geom, int(R), int(W), int(H), grads, tuple(g._version for g in grads))

    def take_acc(self, grads):
        a, self.acc = self.acc, None
        if a is None:
            return None
        geom, R, W, H, mine, versions = a
        for g, m, v in zip(grads, mine, versions):
            if g is None or g.data_ptr() != m.data_ptr() or g.shape != m.shape or g.stride() != m.stride() or \
                    g.dtype != m.dtype or m._version != v:
                return None
        return geom, R, W, H


class _PreprocessGaussians(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means3D, scales, rotations, sh, opacities, raster_settings, cuda_args):
        # cov3D is internal to the pair: the backward recomputes it from the
        # records, the visible Gaussians' inputs packed by the forward
        num_rendered, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped, records = _preprocess_forward_raw(
            means3D, scales, rotations, sh, opacities, raster_settings, keep_cov3D=False, records=True,
            keep_clamped=False)
        # the backward's outputs, cleared on a side stream while the render runs
        ctx.zeroed = None
        P = means2D.size(0)
        if P != 0 and ctx.needs_input_grad[3] and sh.size(1) * 12 % 16 == 0:
            ctx.zeroed = _ZeroedGrads(P, sh.size(1), means2D.device)
            means2D._gs_zeroed = ctx.zeroed
        # radii and depths take no gradient; unused outputs are not zero-filled
        ctx.set_materialize_grads(False)
        ctx.raster_settings = raster_settings
        ctx.cuda_args = cuda_args
        ctx.num_rendered = num_rendered
        ctx.save_for_backward(means3D, scales, rotations, sh, means2D, depths, radii, cov3D, conic_opacity, rgb,
                              clamped, records)
        ctx.mark_non_differentiable(radii, depths)
        return means2D, rgb, conic_opacity, radii, depths

    @staticmethod
    def backward(ctx, grad_means2D, grad_rgb, grad_conic_opacity, grad_radii, grad_depths):
        rs = ctx.raster_settings
        (means3D, scales, rotations, sh, means2D, depths, radii, cov3D, conic_opacity, rgb, clamped,
         records) = ctx.saved_tensors
        if grad_means2D is None:
            grad_means2D = torch.zeros_like(means2D)
        if grad_rgb is None:
            grad_rgb = torch.zeros_like(rgb)
        if grad_conic_opacity is None:
            grad_conic_opacity = torch.zeros_like(conic_opacity)
        zeroed = ctx.zeroed.take() if ctx.zeroed is not None else None
        acc = None
        if zeroed is not None:
            acc = ctx.zeroed.take_acc((grad_means2D, grad_rgb, grad_conic_opacity))
            if acc is not None and (acc[2], acc[3]) != (int(rs.image_width), int(rs.image_height)):
                acc = None
        dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh, dL_dopacity = _preprocess_backward_raw(
            radii, cov3D, clamped, means3D, scales, rotations, sh, rs, grad_means2D, grad_conic_opacity, grad_rgb,
            records=records, zeroed=zeroed, acc=acc)
        return dL_dmeans3D, dL_dscales, dL_drotations, dL_dsh, dL_dopacity, None, None


# ------------------------------------------------------------------- render

def render_gaussians(means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, compute_locally,
                     extended_compute_locally, raster_settings, cuda_args):
    return _RenderGaussians.apply(means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii,
                                  compute_locally, extended_compute_locally, raster_settings, cuda_args)


def _tile_mask(cl, H, W, device):
    """compute_locally as the library's uint8 tile mask; None (every tile is
    local) is passed on as a null mask."""
    gy, gx = (H + 15) // 16, (W + 15) // 16
    if cl is None:
        return None
    cl = cl.to(device=device)
    if cl.numel() != gy * gx:
        raise RuntimeError(f"compute_locally must have {gy}x{gx} tile entries, got {tuple(cl.shape)}")
    return cl.reshape(-1).to(torch.uint8).contiguous()


def _render_forward_raw(bg, H, W, means2D, depths, radii, conic_opacity, rgb, compute_locally, timing=False,
                        debug=False, geo=None, region_side=None, clear=None):
    """Returns (num_rendered, color, n_render, n_consider, n_contrib, out_observe,
    geomBuffer, binningBuffer, imgBuffer, render_ms).  The binning buffer may be
    sized for more than num_rendered instances (_lib.InstanceReserve); render_ms
    covers the whole render forward, the instance count included.
    geo = (tanfovx, tanfovy, all_maps (P,5)): render_geo in the same walk of the
    lists; then out_all_map (5,H,W) and out_plane_depth (1,H,W) follow.
    region_side: the binning's region side (0, 2, 4, 8; None: chosen from the
    device's last forward, _lib.InstanceReserve.region_side).
    clear (without geo): a float32 device tensor, 16-byte aligned and a
    multiple of 16 bytes, that the blend fills with zeros while it runs."""
    _require_device(means2D, "means2D")
    dev = means2D.device
    P = means2D.size(0)
    lib = _lib.load()
    T = ((H + 15) // 16) * ((W + 15) // 16)
    i32 = dict(device=dev, dtype=torch.int32)
    cl = _tile_mask(compute_locally, H, W, dev)
    means2D = _aligned(_dev_f32(means2D, dev), 8)
    depths = _dev_f32(depths, dev)
    radii = radii.to(device=dev, dtype=torch.int32).contiguous()
    conic_opacity = _aligned(_dev_f32(conic_opacity, dev))
    rgb = _dev_f32(rgb, dev)
    bg = _dev_f32(bg, dev)
    stream = _stream(dev)
    geom = torch.empty(lib.gs_render_geom_bytes(P, W, H), device=dev, dtype=torch.uint8)
    img = torch.empty(lib.gs_render_img_bytes(W, H), device=dev, dtype=torch.uint8)
    color = torch.empty((3, H, W), device=dev, dtype=torch.float32)
    n_render = torch.empty((T,), **i32)
    n_consider = torch.empty((T,), **i32)
    n_contrib = torch.empty((T,), **i32)
    out_observe = torch.empty((P,), **i32)
    outs = (ptr(color), ptr(n_render), ptr(n_consider), ptr(n_contrib), ptr(out_observe))
    maps = None
    if geo is not None:
        tanfovx, tanfovy, all_maps = geo
        if all_maps is None or tuple(all_maps.shape) != (P, 5):
            raise RuntimeError(f"render_geo needs all_map of shape ({P}, 5)")
        all_maps = _dev_f32(all_maps, dev)
        maps = torch.empty((6, H, W), device=dev, dtype=torch.float32)
        geo_args = (float(tanfovx), float(tanfovy), ptr(all_maps), ptr(maps[:5]), ptr(maps[5:]))
    elif clear is not None:
        if clear.device != dev or clear.dtype != torch.float32 or not clear.is_contiguous():
            raise RuntimeError("clear must be a contiguous float32 tensor on the render's device")
    clear_args = (ptr(clear), C.c_int64(clear.numel() * 4)) if clear is not None and maps is None else (None, 0)
    if timing:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    R = None
    cap = _lib.RESERVE.capacity(dev)
    rside = _lib.RESERVE.region_side(dev) if region_side is None else int(region_side)
    if cap is not None:
        # one call, no host round trip between the count and the duplication
        binning = torch.empty(lib.gs_render_binning_bytes(cap), device=dev, dtype=torch.uint8)
        Rv = C.c_int64(0)
        args = (P, cap, W, H, ptr(bg), ptr(means2D), ptr(depths), ptr(radii), ptr(conic_opacity), ptr(rgb), ptr(cl),
                ptr(geom), ptr(binning), ptr(img), *outs, C.byref(Rv))
        if maps is None:
            check(lib.gs_render_forward_reserved(*args, rside, *clear_args, stream), "gs_render_forward_reserved")
        else:
            check(lib.gs_render_forward_reserved_geo(*args, *geo_args, rside, stream),
                  "gs_render_forward_reserved_geo")
        _lib.RESERVE.update(dev, int(Rv.value), P)
        R = int(Rv.value) if Rv.value <= cap else None
    if R is None:
        # first forward on the device, or more instances than reserved: count,
        # then size the binning buffer exactly
        Rv = C.c_int64(0)
        check(lib.gs_render_forward_count(P, W, H, ptr(means2D), ptr(radii), ptr(cl), ptr(geom), C.byref(Rv),
                                          rside, stream), "gs_render_forward_count")
        R = int(Rv.value)
        _lib.RESERVE.update(dev, R, P)
        binning = torch.empty(lib.gs_render_binning_bytes(R), device=dev, dtype=torch.uint8)
        args = (P, R, W, H, ptr(bg), ptr(means2D), ptr(depths), ptr(radii), ptr(conic_opacity), ptr(rgb), ptr(cl),
                ptr(geom), ptr(binning), ptr(img), *outs)
        if maps is None:
            check(lib.gs_render_forward(*args, rside, *clear_args, stream), "gs_render_forward")
        else:
            check(lib.gs_render_forward_geo(*args, *geo_args, rside, stream), "gs_render_forward_geo")
    _lib.debug_sync(debug, "gs_render_forward")
    ms = None
    if timing:
        ev1.record()
        ev1.synchronize()
        ms = ev0.elapsed_time(ev1)
    if maps is not None:
        return R, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, ms, maps[:5], maps[5:]
    return R, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, ms


def _render_geo_forward_raw(P, H, W, tanfovx, tanfovy, all_maps, compute_locally, R, geom, binning, img,
                            debug=False):
    """render_geo's maps for a completed split forward of P Gaussians (R,
    geom / binning / img as it returned them), by a second walk of its lists:
    out_all_map (5,H,W), out_plane_depth (1,H,W).  (The operators render the
    maps in the forward's own walk: _render_forward_raw(geo=...).)"""
    dev = geom.device
    lib = _lib.load()
    cl = _tile_mask(compute_locally, H, W, dev)
    if all_maps is None or tuple(all_maps.shape) != (P, 5):
        raise RuntimeError(f"render_geo needs all_map of shape ({P}, 5)")
    all_maps = _dev_f32(all_maps, dev)
    maps = torch.empty((6, H, W), device=dev, dtype=torch.float32)
    check(lib.gs_render_geo_forward(P, R, W, H, float(tanfovx), float(tanfovy), ptr(all_maps), ptr(cl), ptr(geom),
                                    ptr(binning), ptr(img), ptr(maps[:5]), ptr(maps[5:]), _stream(dev)),
          "gs_render_geo_forward")
    _lib.debug_sync(debug, "gs_render_geo_forward")
    return maps[:5], maps[5:]


def _render_backward_raw(bg, R, H, W, means2D, conic_opacity, rgb, compute_locally, geom, binning, img, dL_dpixels,
                         m2d_stride=2, timing=False, debug=False, geo=None, clear=None):
    """geo (render_geo): (tanfovx, tanfovy, all_map_pixels, all_maps,
    dL_dout_all_map, dL_dout_plane_depth); dL/dall_map (P,5) is then returned
    after the timing, else None.  clear: a float32 tensor (16-byte multiple)
    that the call fills with zeros while its blend runs."""
    dev = means2D.device
    P = means2D.size(0)
    lib = _lib.load()
    f32 = dict(device=dev, dtype=torch.float32)
    cl = _tile_mask(compute_locally, H, W, dev)
    dL_dmeans2D = torch.empty((P, m2d_stride), **f32)
    dL_dmeans2D_abs = torch.empty((P, 3), **f32)
    dL_dconic_opacity = torch.empty((P, 4), **f32)
    dL_dcolors = torch.empty((P, 3), **f32)
    means2D = _aligned(_dev_f32(means2D, dev), 8)
    conic_opacity = _aligned(_dev_f32(conic_opacity, dev))
    rgb = _dev_f32(rgb, dev)
    bg = _dev_f32(bg, dev)
    dL_dpixels = _dev_f32(dL_dpixels, dev)
    if timing:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
    dL_dall_map = None
    clr = (ptr(clear), clear.numel() * 4) if clear is not None else (None, 0)
    if geo is None:
        check(lib.gs_render_backward(P, R, W, H, ptr(bg), ptr(means2D), ptr(conic_opacity), ptr(rgb), ptr(cl),
                                     ptr(geom), ptr(binning), ptr(img), ptr(dL_dpixels), ptr(dL_dmeans2D),
                                     m2d_stride, ptr(dL_dmeans2D_abs), ptr(dL_dconic_opacity), ptr(dL_dcolors),
                                     *clr, _stream(dev)), "gs_render_backward")
    else:
        tanfovx, tanfovy, map_px, all_maps, dmaps, dplane = geo
        if all_maps is None or tuple(all_maps.shape) != (P, 5):
            raise RuntimeError(f"render_geo needs all_map of shape ({P}, 5)")
        for name, t, n in (("all_map_pixels", map_px, 5), ("dL_dout_all_map", dmaps, 5),
                           ("dL_dout_plane_depth", dplane, 1)):
            if t is not None and t.numel() != n * H * W:
                raise RuntimeError(f"{name} must hold {n}x{H}x{W} values, got {tuple(t.shape)}")
        map_px, all_maps = _dev_f32(map_px, dev), _dev_f32(all_maps, dev)
        dmaps = _dev_f32(dmaps, dev) if dmaps is not None else torch.zeros((5, H, W), **f32)
        dplane = _dev_f32(dplane, dev) if dplane is not None else torch.zeros((1, H, W), **f32)
        dL_dall_map = torch.empty((P, 5), **f32)
        check(lib.gs_render_backward_geo(P, R, W, H, ptr(bg), float(tanfovx), float(tanfovy), ptr(map_px),
                                         ptr(all_maps), ptr(means2D), ptr(conic_opacity), ptr(rgb), ptr(cl),
                                         ptr(geom), ptr(binning), ptr(img), ptr(dL_dpixels), ptr(dmaps),
                                         ptr(dplane), ptr(dL_dmeans2D), m2d_stride, ptr(dL_dmeans2D_abs),
                                         ptr(dL_dconic_opacity), ptr(dL_dcolors), ptr(dL_dall_map), *clr,
                                         _stream(dev)),
              "gs_render_backward_geo")
    _lib.debug_sync(debug, "gs_render_backward")
    ms = None
    if timing:
        ev1.record()
        ev1.synchronize()
        ms = ev0.elapsed_time(ev1)
    if geo is not None:
        return dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms, dL_dall_map
    return dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms


class _RenderGaussians(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means2D, means2D_abs, conic_opacity, rgb, all_maps, depths, radii, compute_locally,
                extended_compute_locally, raster_settings, cuda_args):
        rs = raster_settings
        render_geo = bool(getattr(rs, "render_geo", False))
        if render_geo and (all_maps is None or tuple(all_maps.shape) != (means2D.size(0), 5)):
            raise RuntimeError("render_geo needs all_map of shape (P, 5)")
        # absent output gradients stay None (no zero-filled tensors)
        ctx.set_materialize_grads(False)
        use_ext = isinstance(cuda_args, dict) and bool(cuda_args.get("avoid_pixel_all2all", False))
        cl = extended_compute_locally if use_ext else compute_locally
        H, W = int(rs.image_height), int(rs.image_width)
        timing = _want_timing(cuda_args)
        dev = means2D.device
        # render_geo: the five geometry maps and the plane depth in the colour's
        # walk of the lists (_r forward.cu:381-384,407-412)
        geo = (rs.tanfovx, rs.tanfovy, all_maps) if render_geo else None
        # render_geo off: the maps and the plane depth are zeros, cleared by
        # the blend while it runs (no fill of their own); the buffer is
        # rounded up to whole 16-byte words
        zmaps = None
        if not render_geo:
            n = 6 * H * W
            zmaps = torch.empty(((n + 3) // 4) * 4, device=means2D.device, dtype=torch.float32)
        res = _render_forward_raw(rs.bg, H, W, means2D, depths, radii, conic_opacity, rgb, cl, timing,
                                  bool(rs.debug), geo=geo, clear=zmaps)
        # the preprocess backward's dL/dsh, which this render's backward clears
        zg = getattr(means2D, "_gs_zeroed", None)
        ctx.zeroed = zg if isinstance(zg, _ZeroedGrads) else None
        R, color, n_render, n_consider, n_contrib, out_observe, geom, binning, img, ms = res[:10]
        if timing:
            cuda_args["stats_collector"]["forward_render_time"] = ms
        if render_geo:
            out_all_map, out_plane_depth = res[10:]
        else:
            maps = zmaps[:6 * H * W].view(6, H, W)
            out_all_map, out_plane_depth = maps[:5], maps[5:]
        ctx.raster_settings = rs
        ctx.cuda_args = cuda_args
        ctx.num_rendered = R
        ctx.save_for_backward(means2D, conic_opacity, rgb, all_maps, out_all_map, geom, binning, img,
                              compute_locally, extended_compute_locally)
        ctx.mark_non_differentiable(n_render, n_consider, n_contrib)
        return color, n_render, n_consider, n_contrib, out_observe, out_all_map, out_plane_depth

    @staticmethod
    def backward(ctx, grad_color, grad_n_render, grad_n_consider, grad_n_contrib, grad_out_observe,
                 grad_out_all_map, grad_out_plane_depth):
        rs = ctx.raster_settings
        (means2D, conic_opacity, rgb, all_maps, all_map_pixels, geom, binning, img, compute_locally,
         extended_compute_locally) = ctx.saved_tensors
        H, W = int(rs.image_height), int(rs.image_width)
        if grad_color is None:
            grad_color = torch.zeros((3, H, W), device=means2D.device, dtype=torch.float32)
        timing = _want_timing(ctx.cuda_args)
        dL_dall_map = None
        # the preprocess backward's dL/dsh, cleared by this call while it runs
        zg = getattr(ctx, "zeroed", None)
        clear = zg.claim() if zg is not None else None
        if getattr(rs, "render_geo", False):
            (dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms,
             dL_dall_map) = _render_backward_raw(
                rs.bg, ctx.num_rendered, H, W, means2D, conic_opacity, rgb, compute_locally, geom, binning, img,
                grad_color.contiguous(), 2, timing, bool(rs.debug),
                geo=(rs.tanfovx, rs.tanfovy, all_map_pixels, all_maps, grad_out_all_map, grad_out_plane_depth),
                clear=clear)
        else:
            dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, ms = _render_backward_raw(
                rs.bg, ctx.num_rendered, H, W, means2D, conic_opacity, rgb, compute_locally, geom, binning, img,
                grad_color.contiguous(), 2, timing, bool(rs.debug), clear=clear)
            if ctx.needs_input_grad[4]:
                dL_dall_map = torch.zeros_like(all_maps)
        if clear is not None:
            zg.cleared()
            # the same call's accumulators, for the preprocess backward
            zg.offer(geom, ctx.num_rendered, W, H, (dL_dmeans2D, dL_dcolors, dL_dconic_opacity))
        if timing:
            ctx.cuda_args["stats_collector"]["backward_render_time"] = ms
        if not ctx.needs_input_grad[4]:
            dL_dall_map = None
        return (dL_dmeans2D, dL_dmeans2D_abs, dL_dconic_opacity, dL_dcolors, dL_dall_map,
                None, None, None, None, None, None)


class GaussianRasterizer(nn.Module):
    """The rasterizer module (_f __init__.py:661-829): the split training path
    (preprocess_gaussians, render_gaussians) and the full-image path (forward,
    render_simp, markVisible; blitzgs_amd.fullpath)."""

    def __init__(self, raster_settings):
        super().__init__()
        self.raster_settings = raster_settings

    def preprocess_gaussians(self, means3D, scales, rotations, shs, opacities, cuda_args=None):
        return preprocess_gaussians(means3D, scales, rotations, shs, opacities, self.raster_settings, cuda_args)

    def render_gaussians(self, means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, compute_locally,
                         extended_compute_locally, cuda_args=None):
        return render_gaussians(means2D, means2D_abs, conic_opacity, rgb, all_map, depths, radii, compute_locally,
                                extended_compute_locally, self.raster_settings, cuda_args)

    def markVisible(self, positions):
        """_f __init__.py:665-674."""
        from .fullpath import mark_visible
        rs = self.raster_settings
        return mark_visible(positions, rs.viewmatrix, rs.projmatrix)

    @staticmethod
    def _check_inputs(shs, colors_precomp, scales, rotations, cov3D_precomp):
        # the reference's argument rules (_f __init__.py:695-700)
        if (shs is None and colors_precomp is None) or (shs is not None and colors_precomp is not None):
            raise Exception('Please provide excatly one of either SHs or precomputed colors!')
        if ((scales is None or rotations is None) and cov3D_precomp is None) or \
                ((scales is not None or rotations is not None) and cov3D_precomp is not None):
            raise Exception('Please provide exactly one of either scale/rotation pair or precomputed 3D covariance!')

    def forward(self, means3D, means2D, opacities, culling, dc=None, shs=None, colors_precomp=None, scales=None,
                rotations=None, cov3D_precomp=None, flag_max_count=False):
        """The full-image path (_f __init__.py:691-730): (color, radii, accum_max_count)."""
        from .fullpath import rasterize_gaussians
        self._check_inputs(shs, colors_precomp, scales, rotations, cov3D_precomp)
        return rasterize_gaussians(means3D, means2D, dc, shs, colors_precomp, opacities, scales, rotations,
                                   cov3D_precomp, flag_max_count, culling, self.raster_settings)

    def render_simp(self, means3D, means2D, opacities, culling, dc=None, shs=None, colors_precomp=None, scales=None,
                    rotations=None, cov3D_precomp=None):
        """_f __init__.py:733-770: (color, radii, accum_weights, accum_weights_count, accum_max_count)."""
        from .fullpath import rasterize_gaussians_simp
        self._check_inputs(shs, colors_precomp, scales, rotations, cov3D_precomp)
        return rasterize_gaussians_simp(means3D, means2D, dc, shs, colors_precomp, opacities, scales, rotations,
                                        cov3D_precomp, culling, self.raster_settings)

    def render_depth(self, means3D, means2D, opacities, culling, dc=None, shs=None, colors_precomp=None, scales=None,
                     rotations=None, cov3D_precomp=None):
        """_f __init__.py:773-810: dict of render, out_pts, rendered_depth,
        discriminants, gidx, accum_alpha (no gradients)."""
        from .fullpath import rasterize_gaussians_depth
        self._check_inputs(shs, colors_precomp, scales, rotations, cov3D_precomp)
        return rasterize_gaussians_depth(means3D, means2D, dc, shs, colors_precomp, opacities, scales, rotations,
                                         cov3D_precomp, culling, self.raster_settings)
