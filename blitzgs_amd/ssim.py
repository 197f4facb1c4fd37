"""fused_ssim: fused 11x11 Gaussian-window SSIM with analytic backward.

Mirrors BlitzGS submodule/fused-ssim (fused_ssim/__init__.py:8-41 and the
fused_ssim_cuda extension, ssim.cu:367-441): same argument order, the
"same"/"valid" padding modes, img1-only gradient, .mean() of the map.
"""
import ctypes as C

import torch

from . import _lib

allowed_padding = ["same", "valid"]


def _stream(dev):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check_img(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a HIP device tensor (blitzgs_amd has no CPU path)")
    if t.ndimension() != 4:
        raise RuntimeError(f"{name} must have dimensions (B, C, H, W)")


def fusedssim(C1, C2, img1, img2, train=True):
    """fused_ssim_cuda.fusedssim: returns (ssim_map, dm_dmu1, dm_dsigma1_sq, dm_dsigma12)."""
    _check_img(img1, "img1")
    _check_img(img2, "img2")
    img1 = img1.to(torch.float32).contiguous()
    img2 = img2.to(torch.float32).contiguous()
    if img1.shape != img2.shape:
        raise RuntimeError("img1 and img2 must have the same shape")
    B, Ch, H, W = img1.shape
    ssim_map = torch.empty_like(img1)
    if train:
        d1, d2, d3 = torch.empty_like(img1), torch.empty_like(img1), torch.empty_like(img1)
    else:
        d1 = d2 = d3 = torch.empty(0, device=img1.device)
    lib = _lib.load()
    p = (lambda t: _lib.ptr(t)) if train else (lambda t: None)
    _lib.check(lib.gs_ssim_forward(B, Ch, H, W, float(C1), float(C2), _lib.ptr(img1), _lib.ptr(img2),
                                   _lib.ptr(ssim_map), p(d1), p(d2), p(d3), _stream(img1.device)),
               "gs_ssim_forward")
    return ssim_map, d1, d2, d3


def fusedssim_backward(C1, C2, img1, img2, dL_dmap, dm_dmu1, dm_dsigma1_sq, dm_dsigma12):
    """fused_ssim_cuda.fusedssim_backward: returns dL/dimg1."""
    img1 = img1.to(torch.float32).contiguous()
    img2 = img2.to(torch.float32).contiguous()
    dL_dmap = dL_dmap.to(torch.float32).contiguous()
    B, Ch, H, W = img1.shape
    g = torch.empty_like(img1)
    lib = _lib.load()
    _lib.check(lib.gs_ssim_backward(B, Ch, H, W, float(C1), float(C2), _lib.ptr(img1), _lib.ptr(img2),
                                    _lib.ptr(dL_dmap), _lib.ptr(dm_dmu1.contiguous()),
                                    _lib.ptr(dm_dsigma1_sq.contiguous()), _lib.ptr(dm_dsigma12.contiguous()),
                                    _lib.ptr(g), _stream(img1.device)),
               "gs_ssim_backward")
    return g


# the loss window's half width: "valid" drops this many pixels on every side
_BORDER = 5
_SSIM_C1 = 0.01 ** 2
_SSIM_C2 = 0.03 ** 2


def _interior(t):
    return t[..., _BORDER:t.shape[-2] - _BORDER, _BORDER:t.shape[-1] - _BORDER]


class FusedSSIMMap(torch.autograd.Function):
    """Autograd node of the SSIM map (fused_ssim/__init__.py:8-35): the
    gradient flows to img1 only; "valid" returns the map without its 5-pixel
    border, whose gradient is zero."""

    @staticmethod
    def forward(ctx, C1, C2, img1, img2, padding="same", train=True):
        full_map, *partials = fusedssim(C1, C2, img1, img2, train)
        ctx.consts = (C1, C2)
        ctx.valid = padding == "valid"
        ctx.save_for_backward(img1.detach(), img2, *partials)
        return _interior(full_map) if ctx.valid else full_map

    @staticmethod
    def backward(ctx, grad_map):
        img1, img2, dm_dmu1, dm_dsigma1_sq, dm_dsigma12 = ctx.saved_tensors
        if ctx.valid:
            grad_map = torch.nn.functional.pad(grad_map, (_BORDER,) * 4)
        dL_dimg1 = fusedssim_backward(*ctx.consts, img1, img2, grad_map, dm_dmu1, dm_dsigma1_sq, dm_dsigma12)
        return None, None, dL_dimg1, None, None, None


def fused_ssim(img1, img2, padding="same", train=True):
    """Mean SSIM of img1 against img2 (fused_ssim/__init__.py:37-41)."""
    if padding not in allowed_padding:
        raise AssertionError(f"padding must be one of {allowed_padding}, got {padding!r}")
    return FusedSSIMMap.apply(_SSIM_C1, _SSIM_C2, img1, img2, padding, train).mean()
