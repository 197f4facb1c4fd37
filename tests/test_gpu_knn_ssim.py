"""distCUDA2 and fused_ssim on the GPU vs the CPU oracle (bit-exact), and
their drop-in module entry points."""
import numpy as np
import pytest
import torch

from blitzgs_amd import synth, _lib
from oracle import oracle as O
from tests.gpu_helpers import assert_bitexact, np_, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _dev(gpu):
    _lib.load()
    yield


@pytest.mark.parametrize("n,kind", [(1, "u"), (2, "u"), (3, "u"), (4, "u"), (5000, "u"), (20000, "dup"),
                                    (20000, "flat"), (300000, "city")])
def test_knn_bitexact(n, kind):
    from blitzgs_amd.knn import distCUDA2
    rng = np.random.default_rng(n)
    if kind == "u":
        pts = rng.uniform(-2, 2, (n, 3)).astype(np.float32)
    elif kind == "dup":
        pts = rng.uniform(0, 10, (n, 3)).astype(np.float32)
        pts[1000:3000] = pts[7]
    elif kind == "flat":
        pts = np.concatenate([rng.uniform(-5, 5, (n, 2)), np.full((n, 1), 3.0)], 1).astype(np.float32)
    else:
        pts = synth.config4_points(n)
    got = np_(distCUDA2(to_dev(pts)))
    with np.errstate(over="ignore"):
        ref = O.knn_meandist3(pts)
    assert_bitexact(got, ref, f"distCUDA2 {kind} n={n}")


def test_knn_dropin_module():
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(__file__)), "blitzgs_amd", "dropin"))
    from simple_knn._C import distCUDA2
    pts = np.random.default_rng(0).uniform(0, 1, (1000, 3)).astype(np.float32)
    assert_bitexact(np_(distCUDA2(to_dev(pts))), O.knn_meandist3(pts), "dropin distCUDA2")


@pytest.mark.parametrize("shape", [(1, 3, 37, 53), (2, 2, 64, 64), (1, 1, 5, 7), (2, 3, 130, 97)])
def test_ssim_forward_backward_bitexact(shape):
    from blitzgs_amd.ssim import fusedssim, fusedssim_backward
    rng = np.random.default_rng(sum(shape))
    x = rng.random(shape).astype(np.float32)
    y = np.clip(x + rng.normal(0, 0.2, shape), 0, 1).astype(np.float32)
    C1, C2 = 0.01 ** 2, 0.03 ** 2
    m, d1, d2, d3 = fusedssim(C1, C2, to_dev(x), to_dev(y), True)
    om, o1, o2, o3 = O.ssim_fwd(x, y)
    for g, r, nm in ((m, om, "ssim_map"), (d1, o1, "dm_dmu1"), (d2, o2, "dm_dsigma1_sq"), (d3, o3, "dm_dsigma12")):
        assert_bitexact(np_(g), r, nm)
    dL = rng.standard_normal(shape).astype(np.float32)
    g = fusedssim_backward(C1, C2, to_dev(x), to_dev(y), to_dev(dL), d1, d2, d3)
    assert_bitexact(np_(g), O.ssim_bwd(x, y, dL, o1, o2, o3), "dL_dimg1")
    m2, *_ = fusedssim(C1, C2, to_dev(x), to_dev(y), False)
    assert_bitexact(np_(m2), om, "ssim_map (train=False)")


def test_fused_ssim_autograd_same_and_valid():
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(__file__)), "blitzgs_amd", "dropin"))
    from fused_ssim import fused_ssim
    rng = np.random.default_rng(3)
    x = rng.random((2, 3, 120, 96)).astype(np.float32)
    y = rng.random((2, 3, 120, 96)).astype(np.float32)
    om, o1, o2, o3 = O.ssim_fwd(x, y)
    for padding in ["same", "valid"]:
        xt = to_dev(x).requires_grad_(True)
        v = fused_ssim(xt, to_dev(y), padding)
        v.backward()
        ref_map = om if padding == "same" else om[:, :, 5:-5, 5:-5]
        assert abs(float(v) - float(ref_map.astype(np.float64).mean())) < 1e-6
        dL = np.zeros_like(x)
        if padding == "same":
            dL[:] = 1.0 / x.size
        else:
            dL[:, :, 5:-5, 5:-5] = 1.0 / ref_map.size
        ref_g = O.ssim_bwd(x, y, dL.astype(np.float32), o1, o2, o3)
        np.testing.assert_allclose(np_(xt.grad), ref_g, rtol=1e-5, atol=1e-10)
