"""SparseGaussianAdam: Adam restricted to the Gaussians seen this step.

Mirrors BlitzGS submodule/diff-gaussian-rasterization_f
(diff_gaussian_rasterization_f/__init__.py:832-863): a torch.optim.Adam
subclass with the same state layout ('step', 'exp_avg', 'exp_avg_sq'), one
tensor per parameter group, betas fixed at (0.9, 0.999) and the bias
correction folded into the learning rate, lr * sqrt(1 - 0.999^t) / (1 - 0.9^t),
computed with the same torch float32 scalar arithmetic.  The per-element update
(cuda_rasterizer/adam.cu:9-38) runs in the HIP library; all groups of a step go
to the device in one launch (gs_adam_update_groups).
"""
import ctypes as C

import torch

from . import _lib


def _dev_f32(t, name):
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise RuntimeError(f"{name} must be a contiguous float32 HIP device tensor")
    return t


class SparseGaussianAdam(torch.optim.Adam):
    def __init__(self, params, lr, eps):
        super().__init__(params=params, lr=lr, eps=eps)

    @torch.no_grad()
    def step(self, visibility, N):
        groups = []
        keep = []
        for group in self.param_groups:
            lr = group["lr"]
            eps = group["eps"]
            assert len(group["params"]) == 1, "more than one tensor in group"
            param = group["params"][0]
            if param.grad is None or torch.prod(torch.tensor(param.grad.shape)) == 0:
                continue
            # lazy state initialisation, as torch.optim.Adam lays it out
            state = self.state[param]
            if len(state) == 0:
                state["step"] = torch.tensor(0.0, dtype=torch.float32)
                state["exp_avg"] = torch.zeros_like(param, memory_format=torch.preserve_format)
                state["exp_avg_sq"] = torch.zeros_like(param, memory_format=torch.preserve_format)
            exp_avg = state["exp_avg"]
            exp_avg_sq = state["exp_avg_sq"]
            # compensate lr for sparse adam, (1-b2**step)**0.5/(1-b1**step)
            state["step"] += 1
            step = state["step"]
            M = param.numel() // N
            lr_t = float(lr * (1 - 0.999 ** step) ** 0.5 / (1 - 0.9 ** step))
            grad = param.grad.contiguous()
            for t, nm in ((param, "param"), (grad, "grad"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
                _dev_f32(t, nm)
            keep.append(grad)
            groups.append(_lib.AdamGroup(grad=_lib.ptr(grad).value, param=_lib.ptr(param).value,
                                         exp_avg=_lib.ptr(exp_avg).value, exp_avg_sq=_lib.ptr(exp_avg_sq).value,
                                         M=int(M), lr=lr_t, eps=float(eps)))
        if not groups:
            return
        vis = visibility.reshape(-1)
        if vis.dtype != torch.bool:
            vis = vis != 0
        vis = vis.contiguous()
        if vis.numel() != N or not vis.is_cuda:
            raise RuntimeError(f"visibility must be a HIP device tensor of {N} entries")
        lib = _lib.load()
        stream = C.c_void_p(torch.cuda.current_stream(vis.device).cuda_stream)
        for i0 in range(0, len(groups), 8):
            chunk = groups[i0:i0 + 8]
            arr = (_lib.AdamGroup * len(chunk))(*chunk)
            _lib.check(lib.gs_adam_update_groups(len(chunk), arr, int(N), _lib.ptr(vis), 0.9, 0.999, stream),
                       "gs_adam_update_groups")
        del keep


def adamUpdate(param, param_grad, exp_avg, exp_avg_sq, visible, lr, b1, b2, eps, N, M):
    """The reference's _C.adamUpdate (rasterize_points.cu:807-832), in place."""
    for t, nm in ((param, "param"), (param_grad, "param_grad"), (exp_avg, "exp_avg"),
                  (exp_avg_sq, "exp_avg_sq")):
        _dev_f32(t, nm)
    vis = visible.reshape(-1)
    vis = vis.contiguous() if vis.dtype == torch.bool else (vis != 0).contiguous()
    lib = _lib.load()
    stream = C.c_void_p(torch.cuda.current_stream(param.device).cuda_stream)
    _lib.check(lib.gs_adam_update(_lib.ptr(param), _lib.ptr(param_grad), _lib.ptr(exp_avg), _lib.ptr(exp_avg_sq),
                                  _lib.ptr(vis), float(lr), float(b1), float(b2), float(eps), int(N), int(M),
                                  stream),
               "gs_adam_update")
