"""Sparse Adam on the GPU (adam.cu:9-67, SparseGaussianAdam in
diff_gaussian_rasterization_f/__init__.py:832-863) against the CPU oracle, bit
for bit: the reference's single-tensor entry point, the fused multi-group step
of SparseGaussianAdam over several steps, aligned and unaligned tensors."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

B1, B2 = 0.9, 0.999


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("M", [1, 3, 4, 45])
def test_adam_update_bitexact(gpu, M):
    from blitzgs_amd.adam import adamUpdate
    rng = np.random.default_rng(M)
    N = 10007
    p = rng.normal(0, 1, (N, M)).astype(np.float32)
    g = rng.normal(0, 1, (N, M)).astype(np.float32)
    m = rng.normal(0, 0.1, (N, M)).astype(np.float32)
    v = rng.random((N, M)).astype(np.float32) * 0.01
    vis = rng.random(N) < 0.3
    dev = {k: torch.tensor(a, device="cuda") for k, a in dict(p=p, g=g, m=m, v=v).items()}
    adamUpdate(dev["p"], dev["g"], dev["m"], dev["v"], torch.tensor(vis, device="cuda"), 3e-3, B1, B2, 1e-15, N, M)
    O.adam_update(p, g, m, v, vis.astype(np.uint8), 3e-3, B1, B2, 1e-15)
    for k, ref in dict(p=p, m=m, v=v).items():
        np.testing.assert_array_equal(_np(dev[k]).view(np.uint32), ref.view(np.uint32), err_msg=k)


def test_adam_update_unaligned_views(gpu):
    # tensors starting one float into their storage take the scalar path
    from blitzgs_amd.adam import adamUpdate
    rng = np.random.default_rng(7)
    N, M = 999, 3
    arrs = [rng.normal(0, 1, N * M + 1).astype(np.float32) for _ in range(4)]
    arrs[3] = np.abs(arrs[3])
    vis = rng.random(N) < 0.5
    dev = [torch.tensor(a, device="cuda")[1:].view(N, M) for a in arrs]
    assert all(t.data_ptr() % 16 != 0 for t in dev)
    adamUpdate(dev[0], dev[1], dev[2], dev[3], torch.tensor(vis, device="cuda"), 1e-2, B1, B2, 1e-8, N, M)
    ref = [a[1:].reshape(N, M).copy() for a in arrs]
    O.adam_update(ref[0], ref[1], ref[2], ref[3], vis.astype(np.uint8), 1e-2, B1, B2, 1e-8)
    for i in (0, 2, 3):
        np.testing.assert_array_equal(_np(dev[i]).view(np.uint32), ref[i].view(np.uint32))


def test_sparse_gaussian_adam_steps_bitexact(gpu):
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(__file__)), "blitzgs_amd", "dropin"))
    from diff_gaussian_rasterization_f import SparseGaussianAdam
    rng = np.random.default_rng(3)
    N = 4096
    shapes = {"xyz": (N, 3), "f_dc": (N, 1, 3), "f_rest": (N, 15, 3), "opacity": (N, 1), "scaling": (N, 3),
              "rotation": (N, 4)}
    lrs = {"xyz": 1.6e-4, "f_dc": 2.5e-3, "f_rest": 1.25e-4, "opacity": 2.5e-2, "scaling": 5e-3, "rotation": 1e-3}
    init = {k: rng.normal(0, 1, s).astype(np.float32) for k, s in shapes.items()}
    params = {k: torch.tensor(a, device="cuda", requires_grad=True) for k, a in init.items()}
    opt = SparseGaussianAdam([{"params": [params[k]], "lr": lrs[k], "name": k} for k in shapes], lr=0.0, eps=1e-15)
    ref = {k: (a.reshape(N, -1).copy(), np.zeros((N, a.size // N), np.float32),
               np.zeros((N, a.size // N), np.float32)) for k, a in init.items()}
    for step in range(1, 4):
        vis = rng.random(N) < 0.4
        for k in shapes:
            g = rng.normal(0, 1, shapes[k]).astype(np.float32)
            params[k].grad = torch.tensor(g, device="cuda")
            s = torch.tensor(float(step), dtype=torch.float32)
            lr_t = float(lrs[k] * (1 - 0.999 ** s) ** 0.5 / (1 - 0.9 ** s))
            p, m, v = ref[k]
            O.adam_update(p, g.reshape(N, -1), m, v, vis.astype(np.uint8), lr_t, B1, B2, 1e-15)
        opt.step(torch.tensor(vis, device="cuda"), N)
        for k in shapes:
            got = _np(params[k]).reshape(N, -1)
            np.testing.assert_array_equal(got.view(np.uint32), ref[k][0].view(np.uint32), err_msg=f"{k} step {step}")
            st = opt.state[params[k]]
            assert float(st["step"]) == step
            np.testing.assert_array_equal(_np(st["exp_avg"]).reshape(N, -1).view(np.uint32),
                                          ref[k][1].view(np.uint32))
