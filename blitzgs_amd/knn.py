"""distCUDA2: mean squared distance to the three nearest neighbours.

Mirrors BlitzGS submodule/simple-knn (ext.cpp:16 distCUDA2, spatial.cu:15-26):
takes a (P, 3) float32 device tensor, returns (P,) float32.  Used once at scene
initialisation (scene/gaussian_model.py:317) to seed the Gaussian scales.
"""
import ctypes as C

import torch

from . import _lib


def distCUDA2(points):
    if not isinstance(points, torch.Tensor) or not points.is_cuda:
        raise RuntimeError("distCUDA2: points must be a HIP device tensor (blitzgs_amd has no CPU path)")
    if points.ndimension() != 2 or points.size(1) != 3:
        raise RuntimeError("points must have dimensions (num_points, 3)")
    pts = points.to(torch.float32).contiguous()
    P = pts.size(0)
    out = torch.empty((P,), device=pts.device, dtype=torch.float32)
    if P == 0:
        return out
    lib = _lib.load()
    ws = torch.empty(lib.gs_knn_workspace_bytes(P), device=pts.device, dtype=torch.uint8)
    _lib.check(lib.gs_knn_meandist3(P, _lib.ptr(pts), _lib.ptr(out), _lib.ptr(ws),
                                    C.c_void_p(torch.cuda.current_stream(pts.device).cuda_stream)),
               "gs_knn_meandist3")
    return out
