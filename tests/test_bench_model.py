"""bench.py's algorithmic byte model for the split path's binning counts the
region-list entries (region_entries): checked against a direct enumeration of
every (Gaussian, 2x2-tile region) pair on random rects, with and without a
tile mask of whole tile rows, including culled, NaN and off-image Gaussians."""
import importlib.util
import os

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _enumerate(m, r, W, H, rows=None, side=2):
    """Pairs (Gaussian, region) by brute force: the tile rect of each Gaussian
    (the binning rule: trunc((mean -/+ radius (+15)) / 16) clamped to the grid),
    clipped to the local rows, and every side x side region of the box it meets."""
    gx, gy = (W + 15) // 16, (H + 15) // 16
    by0, by1 = (0, gy) if rows is None else rows
    n = 0
    for (x, y), rad in zip(m, r):
        if rad <= 0 or not np.isfinite(x) or not np.isfinite(y):
            continue
        t = lambda v, hi: min(max(int(np.trunc(v / 16.0)), 0), hi)
        x0, x1 = t(x - rad, gx), t(x + rad + 15.0, gx)
        y0, y1 = max(t(y - rad, gy), by0), min(t(y + rad + 15.0, gy), by1)
        regions = {(tx // side, (ty - by0) // side) for tx in range(x0, x1) for ty in range(y0, y1)}
        n += len(regions)
    return n


@pytest.mark.parametrize("rows,side", [(None, 0), ((3, 9), 0), (None, 4), ((3, 9), 8)])
def test_region_entries_match_enumeration(bench, rows, side):
    rng = np.random.default_rng(5)
    W, H = 300, 230
    P = 3000
    m = np.stack([rng.uniform(-40, W + 40, P), rng.uniform(-40, H + 40, P)], 1).astype(np.float32)
    r = rng.integers(-2, 60, P).astype(np.int32)
    m[7] = [np.nan, 10.0]
    r[8] = 0
    cl = None
    if rows is not None:
        gx, gy = (W + 15) // 16, (H + 15) // 16
        mask = np.zeros((gy, gx), bool)
        mask[rows[0]:rows[1]] = True
        cl = torch.from_numpy(mask.reshape(-1))
    got = bench.region_entries(torch.from_numpy(m), torch.from_numpy(r), W, H, cl, side=side)
    assert got == _enumerate(m, r, W, H, rows, max(side, 2))
    assert got > 1000
