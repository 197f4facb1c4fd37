"""Pin the oracle's scalar math: o_expf / o_logf against libm in double
precision, the saturating casts through the binning rules, getHigherMsb."""
import math

import numpy as np

from oracle import oracle as O


def _ulp_err(got, ref):
    ref32 = ref.astype(np.float32)
    spacing = np.abs(np.spacing(ref32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref) / spacing


def test_expf_accuracy_render_range():
    # the render evaluates exp on power in [-87, 0]; sweep it densely
    x = np.linspace(-87.0, 0.0, 2_000_001).astype(np.float32)
    got = O.vec_expf(x)
    ref = np.exp(x.astype(np.float64))
    assert _ulp_err(got, ref).max() <= 2.0


def test_expf_accuracy_general_and_special():
    rng = np.random.default_rng(0)
    x = rng.uniform(-80, 88, 1_000_000).astype(np.float32)
    got = O.vec_expf(x)
    assert _ulp_err(got, np.exp(x.astype(np.float64))).max() <= 2.0
    sp = np.array([0.0, -0.0, -87.5, -200.0, 100.0, np.nan, -np.inf], np.float32)
    g = O.vec_expf(sp)
    assert g[0] == 1.0 and g[1] == 1.0
    assert g[2] == 0.0 and g[3] == 0.0 and g[6] == 0.0
    assert np.isinf(g[4]) and np.isnan(g[5])


def test_logf_accuracy():
    rng = np.random.default_rng(1)
    # the preprocess evaluates log(opacity * 255) for opacity in (1/255, 1]
    x = np.concatenate([rng.uniform(1.0, 256.0, 1_000_000),
                        np.exp(rng.uniform(-80, 80, 1_000_000))]).astype(np.float32)
    got = O.vec_logf(x)
    ref = np.log(x.astype(np.float64))
    err = np.abs(got.astype(np.float64) - ref)
    # absolute error relative to the ulp of the result, or 1 ulp of 1 near log=0
    scale = np.maximum(np.abs(np.spacing(ref.astype(np.float32))).astype(np.float64), 2.0 ** -24)
    assert (err / scale).max() <= 3.0
    sp = O.vec_logf(np.array([1.0, 0.0, -1.0, np.inf, np.nan, 0.5], np.float32))
    assert sp[0] == 0.0 and np.isneginf(sp[1]) and np.isnan(sp[2]) and np.isposinf(sp[3]) and np.isnan(sp[4])
    assert abs(sp[5] - math.log(0.5)) < 1e-7


def _higher_msb_py(n):
    # line-by-line restatement of getHigherMsb (_r rasterizer_impl.cu:39-54) with 32-bit shifts
    msb = 16
    step = msb
    while step > 1:
        step //= 2
        if (n >> msb) if msb < 32 else 0:
            msb += step
        else:
            msb -= step
    if (n >> msb) if msb < 32 else 0:
        msb += 1
    return msb


def test_higher_msb_covers_tile_ids():
    # the sort only looks at bits [0, 32+msb): every tile id < T must fit, so
    # sorting the full 64-bit key (as the oracle and the HIP path do) is the
    # same permutation
    for n in list(range(1, 70000)) + [2 ** k for k in range(17, 31)] + [2 ** k + 1 for k in range(17, 31)]:
        b = _higher_msb_py(n)
        assert (n - 1) < (1 << b), n
    for n in [1, 2, 3, 255, 256, 257, 6700, 8160, 43776, 65536, 1 << 20]:
        assert O.higher_msb(n) == _higher_msb_py(n)
    assert O.higher_msb(256) == 9 and O.higher_msb(6700) == 13 and O.higher_msb(43776) == 16
