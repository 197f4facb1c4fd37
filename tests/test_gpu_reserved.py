"""The reserved forward (gs_render_forward_reserved, gs_render_full_forward_reserved):
one library call that queues the count, duplication, sorts and blend against a
binning buffer sized before R is known.  Checked against the exact two-call
forward on the same inputs -- bit-exact, since both run the same kernels on the
same counts -- for capacities equal to R, above it and below it (then the call
reports R and the caller redoes the forward at the exact size), for a scene
with no instances, and through the operator layer, whose first forward on a
device is exact and whose later ones are reserved."""
import ctypes as C

import numpy as np
import pytest
import torch

from blitzgs_amd import _lib, synth
from oracle import oracle as O
from tests.gpu_helpers import assert_close_abs, buffer_views, np_, settings_for, to_dev

pytestmark = pytest.mark.gpu


def _inputs(n=6000, seed=21, W=272, H=208):
    scene, cam = synth.small_scene(n, seed=seed, W=W, H=H, extent=1.5, log_mu=-2.2)
    pre = O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                           scene["opacities"])
    dev = {k: to_dev(pre[k]) for k in ["means2D", "depths", "radii", "conic_opacity", "rgb"]}
    return scene, cam, pre, dev


def _forward(dev, W, H, capacity=None, cl=None, clear_floats=0):
    """capacity None: the exact two-call forward; else the reserved call.
    clear_floats: a NaN-filled buffer of that many floats (a multiple of 4)
    for the blend to clear, returned as "clear"."""
    lib = _lib.load()
    P = dev["means2D"].shape[0]
    T = ((W + 15) // 16) * ((H + 15) // 16)
    s = _lib.stream_of()
    geom = torch.empty(lib.gs_render_geom_bytes(P, W, H), device="cuda", dtype=torch.uint8)
    img = torch.empty(lib.gs_render_img_bytes(W, H), device="cuda", dtype=torch.uint8)
    color = torch.empty((3, H, W), device="cuda")
    i32 = lambda n: torch.empty(n, device="cuda", dtype=torch.int32)
    n_render, n_consider, n_contrib, obs = i32(T), i32(T), i32(T), i32(P)
    bg = to_dev(np.array([0.1, 0.2, 0.3], np.float32))
    clp = None if cl is None else _lib.ptr(cl)
    args = (_lib.ptr(bg), _lib.ptr(dev["means2D"]), _lib.ptr(dev["depths"]), _lib.ptr(dev["radii"]),
            _lib.ptr(dev["conic_opacity"]), _lib.ptr(dev["rgb"]), clp, _lib.ptr(geom))
    outs = (_lib.ptr(color), _lib.ptr(n_render), _lib.ptr(n_consider), _lib.ptr(n_contrib), _lib.ptr(obs))
    clear = torch.full((clear_floats,), float("nan"), device="cuda") if clear_floats else None
    clr = (_lib.ptr(clear), C.c_int64(4 * clear_floats))
    R = C.c_int64(-1)
    if capacity is None:
        _lib.check(lib.gs_render_forward_count(P, W, H, _lib.ptr(dev["means2D"]), _lib.ptr(dev["radii"]), clp,
                                               _lib.ptr(geom), C.byref(R), 0, s), "count")
        binning = torch.empty(lib.gs_render_binning_bytes(R.value), device="cuda", dtype=torch.uint8)
        _lib.check(lib.gs_render_forward(P, R.value, W, H, *args, _lib.ptr(binning), _lib.ptr(img), *outs, 0, *clr,
                                         s), "forward")
    else:
        binning = torch.empty(lib.gs_render_binning_bytes(capacity), device="cuda", dtype=torch.uint8)
        _lib.check(lib.gs_render_forward_reserved(P, capacity, W, H, *args, _lib.ptr(binning), _lib.ptr(img),
                                                  *outs, C.byref(R), 0, *clr, s), "forward_reserved")
    torch.cuda.synchronize()
    return dict(R=int(R.value), color=color, n_render=n_render, n_consider=n_consider, n_contrib=n_contrib,
                obs=obs, geom=geom, binning=binning, img=img, clear=clear)


def _same(a, b, W, H, P, depths):
    assert a["R"] == b["R"]
    for k in ["color", "n_render", "n_consider", "n_contrib", "obs"]:
        assert torch.equal(a[k].view(torch.int32), b[k].view(torch.int32)), k
    va = buffer_views(a["R"], W, H, a["binning"], a["img"], P, depths, a["geom"])
    vb = buffer_views(b["R"], W, H, b["binning"], b["img"], P, depths, b["geom"])
    for k in ["point_list", "keys", "ranges", "final_T", "n_contrib_px"]:
        assert torch.equal(va[k], vb[k]), k


@pytest.mark.parametrize("masked", [False, True])
def test_reserved_forward_matches_two_calls(masked):
    scene, cam, pre, dev = _inputs()
    W, H = cam["W"], cam["H"]
    P = pre["means2D"].shape[0]
    cl = None
    if masked:
        gy, gx = (H + 15) // 16, (W + 15) // 16
        m = np.zeros((gy, gx), np.uint8)
        m[3:9] = 1
        cl = to_dev(m.reshape(-1))
    ref = _forward(dev, W, H, None, cl)
    R = ref["R"]
    assert R > 1000
    for cap in (R, R + 1, 2 * R + 777):
        _same(_forward(dev, W, H, cap, cl), ref, W, H, P, dev["depths"])
    # fewer instances reserved than there are: R comes back, and the exact
    # forward on the same workspaces' inputs is then still right
    small = _forward(dev, W, H, R - 1, cl)
    assert small["R"] == R
    small = _forward(dev, W, H, 1, cl)
    assert small["R"] == R
    _same(_forward(dev, W, H, None, cl), ref, W, H, P, dev["depths"])
    # a caller buffer cleared by the blend (the zero maps of render_geo off),
    # on both routes, fitting or not, larger than one block's share; results
    # unchanged
    nclr = 4 * ((6 * W * H + 3) // 4)
    for cap in (None, R, 1):
        out = _forward(dev, W, H, cap, cl, clear_floats=nclr)
        assert out["R"] == R and not out["clear"].isnan().any() and not out["clear"].any(), cap
        if cap != 1:
            _same(out, ref, W, H, P, dev["depths"])
    # and against the oracle
    ob = O.binning(W, H, pre["means2D"], pre["depths"], pre["radii"], None if cl is None else np_(cl).reshape(
        (H + 15) // 16, (W + 15) // 16))
    assert ob["R"] == R


def test_reserved_forward_without_instances():
    scene, cam, pre, dev = _inputs(n=500, seed=5)
    W, H = cam["W"], cam["H"]
    dev["radii"] = torch.zeros_like(dev["radii"])
    out = _forward(dev, W, H, 4096, clear_floats=4 * 1000)
    assert out["R"] == 0
    assert not out["clear"].isnan().any() and not out["clear"].any()
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    assert_close_abs(np_(out["color"]), np.broadcast_to(bg[:, None, None], (3, H, W)), "background", 0.0)
    assert not out["obs"].any() and not out["n_render"].any()


@pytest.mark.parametrize("reserved", [False, True])
def test_binning_stage_timing_modes(reserved):
    # mode 2 times the binning as one stage and nothing else; mode 1 also every
    # kernel; the stage is closed once per forward, on both forward routes
    scene, cam, pre, dev = _inputs(n=4000, seed=9)
    W, H = cam["W"], cam["H"]
    cap = 1 << 20 if reserved else None
    ref = _forward(dev, W, H)
    for mode_kernels in (False, True):
        _lib.timing_reset()
        _lib.timing_enable(True, stages_only=not mode_kernels)
        try:
            out = _forward(dev, W, H, cap)
        finally:
            _lib.timing_enable(False)
        kt = _lib.timing_read()
        assert kt["binning (wall)"][1] == 1 and kt["binning (wall)"][0] > 0.0
        if mode_kernels:
            assert {"count_regions_kernel", "scan_regions_kernel", "scatter_regions_kernel",
                    "render_fwd_kernel"} <= set(kt)
        else:
            assert set(kt) == {"binning (wall)"}
        assert out["R"] == ref["R"] and torch.equal(out["color"].view(torch.int32), ref["color"].view(torch.int32))
    _lib.timing_reset()


def test_operator_layer_reserves_after_first_forward():
    """The first forward on the device sizes the binning buffer exactly; the
    next ones reserve (from the largest recent count) and give the same
    image; a larger scene after a small one overflows the reserve and is
    redone at the exact size."""
    from blitzgs_amd import rasterizer
    _lib.RESERVE.reset()
    scene, cam, pre, dev = _inputs()
    W, H = cam["W"], cam["H"]
    rs = settings_for(cam)
    args = (rs.bg, H, W, dev["means2D"], dev["depths"], dev["radii"], dev["conic_opacity"], dev["rgb"], None)
    first = rasterizer._render_forward_raw(*args)
    d = torch.device("cuda", torch.cuda.current_device())
    assert _lib.RESERVE.capacity(d) is not None and _lib.RESERVE.capacity(d) > first[0]
    second = rasterizer._render_forward_raw(*args)
    assert first[0] == second[0]
    assert second[7].numel() > first[7].numel()          # sized for the reserve, not for R
    for i in range(1, 6):
        assert torch.equal(first[i].view(torch.int32), second[i].view(torch.int32))
    # a much larger scene: more instances than reserved
    _lib.RESERVE.reset()
    _lib.RESERVE.update(d, 10)
    third = rasterizer._render_forward_raw(*args)
    assert third[0] == first[0]
    assert torch.equal(first[1], third[1])


def test_full_path_reserved_forward_matches_exact():
    from blitzgs_amd.rasterizer import GaussianRasterizer
    scene, cam = synth.small_scene(3000, seed=23, W=160, H=120, log_mu=-1.9)
    rs = settings_for(cam, bg=(0.2, 0.2, 0.2))
    t = lambda a: to_dev(np.ascontiguousarray(a))
    sh = scene["sh"]
    ras = GaussianRasterizer(rs)
    culling = torch.zeros(sh.shape[0], dtype=torch.bool, device="cuda")
    _lib.RESERVE.reset()
    outs = []
    with torch.no_grad():
        for _ in range(2):    # exact, then reserved
            color, radii, amc = ras(means3D=t(scene["means3D"]), means2D=torch.zeros_like(t(scene["means3D"])),
                                    opacities=t(scene["opacities"]), culling=culling, dc=t(sh[:, :1]),
                                    shs=t(sh[:, 1:]), scales=t(scene["scales"]), rotations=t(scene["rotations"]),
                                    flag_max_count=True)
            torch.cuda.synchronize()
            outs.append((color.clone(), radii.clone(), amc.clone()))
    d = torch.device("cuda", torch.cuda.current_device())
    assert _lib.RESERVE.capacity(d) is not None
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
