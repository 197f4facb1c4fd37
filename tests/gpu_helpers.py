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
    views = buffer_views(R, W, H, binning, img)
    return dict(R=R, color=color, n_render=n_render, n_consider=n_consider, n_contrib=n_contrib,
                out_observe=out_observe, geom=geom, binning=binning, img=img, **views)


def buffer_views(R, W, H, binning, img):
    """Copy the sorted ids/keys, ranges and per-pixel state out of the opaque buffers."""
    lib = _lib.load()
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


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
