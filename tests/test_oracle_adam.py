"""Pin the oracle's sparse Adam step (adam.cu:9-38): against torch.optim.Adam in
float64 for rows visible at every step (the learning-rate compensation of
SparseGaussianAdam makes the two identical up to the eps term), against the
one-step closed form, and rows of invisible Gaussians must stay untouched."""
import numpy as np
import torch

from oracle import oracle as O

B1, B2 = 0.9, 0.999


def lr_t(lr, step):
    s = torch.tensor(float(step), dtype=torch.float32)
    return float(lr * (1 - 0.999 ** s) ** 0.5 / (1 - 0.9 ** s))


def test_first_step_closed_form():
    rng = np.random.default_rng(0)
    N, M = 50, 3
    g = rng.normal(0, 1, (N, M)).astype(np.float32)
    p = rng.normal(0, 1, (N, M)).astype(np.float32)
    p0 = p.copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    O.adam_update(p, g, m, v, np.ones(N, np.uint8), 1e-3, B1, B2, 1e-15)
    g64 = g.astype(np.float64)
    # (1 - b1) and (1 - b2) are formed in fp32 from the fp32 betas, as in the kernel
    c1 = float(np.float32(1.0) - np.float32(B1))
    c2 = float(np.float32(1.0) - np.float32(B2))
    np.testing.assert_allclose(m, c1 * g64, rtol=1e-6)
    np.testing.assert_allclose(v, c2 * g64 * g64, rtol=1e-6)
    # step = -lr (1-b1) g / (sqrt(1-b2) |g|) = -lr (1-b1) / sqrt(1-b2) * sign(g)
    # p + step is rounded to fp32: allow half an ulp of |p| <= 4
    np.testing.assert_allclose(p.astype(np.float64) - p0, -1e-3 * c1 / np.sqrt(c2) * np.sign(g64), rtol=1e-5,
                               atol=2.5e-7)


def test_matches_torch_adam_when_always_visible_and_skips_invisible():
    rng = np.random.default_rng(1)
    N, M = 64, 5
    vis = (rng.random(N) < 0.6).astype(np.uint8)
    p = rng.normal(0, 1, (N, M)).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    p_start = p.copy()
    ref = torch.tensor(p_start, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([ref], lr=1e-2, betas=(B1, B2), eps=1e-15)
    for step in range(1, 6):
        g = rng.normal(0, 1, (N, M)).astype(np.float32)
        O.adam_update(p, g, m, v, vis, lr_t(1e-2, step), B1, B2, 1e-15)
        ref.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
    r = ref.detach().numpy()
    sel = vis.astype(bool)
    np.testing.assert_allclose(p[sel], r[sel], rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(p[~sel], p_start[~sel])
    assert not m[~sel].any() and not v[~sel].any()
