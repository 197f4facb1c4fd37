"""Pin the oracle's distCUDA2 against O(n^2) brute force, and its fused-ssim
against a float64 closed form (the PyTorch conv SSIM of BlitzGS
utils/loss_utils.py:51-80 restated in numpy) and finite differences."""
import math

import numpy as np
import pytest

from blitzgs_amd import synth
from oracle import oracle as O


def brute_knn(pts):
    pts = np.asarray(pts, np.float32)
    P = len(pts)
    out = np.empty(P, np.float32)
    big = np.float32(np.finfo(np.float32).max)
    for i in range(P):
        d = pts - pts[i]                       # other - self, float32
        dist = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
        dist[i] = np.inf
        b = np.sort(dist)[:3].astype(np.float32)
        b = np.concatenate([b, np.full(3, big, np.float32)])[:3]
        b[~np.isfinite(b)] = big
        with np.errstate(over="ignore"):
            out[i] = np.float32(np.float32(b[0] + b[1]) + b[2]) / np.float32(3.0)
    return out


@pytest.mark.parametrize("kind", ["uniform", "clustered", "duplicates", "flat", "line"])
def test_knn_matches_brute_force(kind):
    rng = np.random.default_rng(sum(map(ord, kind)))
    n = 2500
    if kind == "uniform":
        pts = rng.uniform(-3, 3, (n, 3))
    elif kind == "clustered":
        pts = np.concatenate([rng.normal(0, 0.01, (n // 2, 3)), rng.uniform(-50, 50, (n - n // 2, 3))])
    elif kind == "duplicates":
        pts = rng.uniform(0, 1, (n, 3))
        pts[100:400] = pts[50]
    elif kind == "flat":
        pts = np.concatenate([rng.uniform(-5, 5, (n, 2)), np.zeros((n, 1))], 1)
    else:
        pts = np.stack([np.linspace(0, 1, n), np.zeros(n), np.zeros(n)], 1)
    pts = pts.astype(np.float32)
    np.testing.assert_array_equal(O.knn_meandist3(pts).view(np.uint32), brute_knn(pts).view(np.uint32))


def test_knn_small_counts():
    # fewer than four points: the missing neighbours stay FLT_MAX, as in the reference
    for P in [1, 2, 3, 4]:
        pts = np.arange(3 * P, dtype=np.float32).reshape(P, 3)
        np.testing.assert_array_equal(O.knn_meandist3(pts).view(np.uint32), brute_knn(pts).view(np.uint32))
    assert np.isinf(O.knn_meandist3(np.zeros((1, 3), np.float32)))[0]


def test_knn_config4_distribution_sample():
    pts = synth.config4_points(40000)
    sub = pts[:3000]
    ref = brute_knn(sub)
    np.testing.assert_array_equal(O.knn_meandist3(sub).view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------- SSIM

def _gauss64(ws=11, sigma=1.5):
    g = np.array([math.exp(-((x - ws // 2) ** 2) / (2 * sigma * sigma)) for x in range(ws)])
    return g / g.sum()


def _blur64(img, g):
    # zero-padded "same" separable convolution, float64
    B, C, H, W = img.shape
    p = np.pad(img, ((0, 0), (0, 0), (5, 5), (5, 5)))
    h = sum(g[t] * p[:, :, :, t:t + W] for t in range(11))
    return sum(g[t] * h[:, :, t:t + H, :] for t in range(11))


def ssim_map64(x, y, C1=0.01 ** 2, C2=0.03 ** 2):
    g = _gauss64()
    x = x.astype(np.float64)
    y = y.astype(np.float64)
    mu1, mu2 = _blur64(x, g), _blur64(y, g)
    s11 = _blur64(x * x, g) - mu1 * mu1
    s22 = _blur64(y * y, g) - mu2 * mu2
    s12 = _blur64(x * y, g) - mu1 * mu2
    return ((2 * mu1 * mu2 + C1) * (2 * s12 + C2)) / ((mu1 ** 2 + mu2 ** 2 + C1) * (s11 + s22 + C2))


def test_ssim_window_within_one_ulp_of_formula():
    w = np.empty(11, np.float32)
    import ctypes as C
    O.lib().o_ssim_window(w.ctypes.data_as(C.c_void_p))
    g = _gauss64().astype(np.float32)
    assert np.abs(w.view(np.int32) - g.view(np.int32)).max() <= 1
    assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


def test_ssim_forward_matches_float64_closed_form():
    rng = np.random.default_rng(0)
    x = rng.random((2, 3, 37, 53)).astype(np.float32)
    y = np.clip(x + rng.normal(0, 0.1, x.shape), 0, 1).astype(np.float32)
    m, d1, d2, d3 = O.ssim_fwd(x, y)
    ref = ssim_map64(x, y)
    assert np.abs(m - ref).max() < 2e-5
    # identical images: SSIM == 1
    m1, *_ = O.ssim_fwd(x, x)
    assert np.abs(m1 - 1).max() < 1e-5


def test_ssim_backward_matches_finite_differences():
    rng = np.random.default_rng(1)
    x = rng.random((1, 2, 19, 23)).astype(np.float32)
    y = rng.random((1, 2, 19, 23)).astype(np.float32)
    m, d1, d2, d3 = O.ssim_fwd(x, y)
    dLd = np.full(x.shape, 1.0 / x.size, np.float32)           # loss = mean(map)
    g = O.ssim_bwd(x, y, dLd, d1, d2, d3)
    h = 1e-6
    x64 = x.astype(np.float64)
    idx = [(0, 0, 0, 0), (0, 1, 9, 11), (0, 0, 18, 22), (0, 1, 3, 17), (0, 0, 10, 0)]
    for i in idx:
        xp = x64.copy(); xp[i] += h
        xm = x64.copy(); xm[i] -= h
        fd = (ssim_map64(xp, y).mean() - ssim_map64(xm, y).mean()) / (2 * h)
        np.testing.assert_allclose(g[i], fd, rtol=2e-3, atol=2e-7)
