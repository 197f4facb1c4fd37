"""Pin the oracle's backward (render bwd + preprocess bwd) with central finite
differences of the float64 twin.  The per-tile Gaussian lists come from the
fp32 oracle's binning and are held fixed; finite-difference entries whose +h
and -h evaluations blend a different set of (pixel, Gaussian) pairs (a
threshold crossing) are excluded and counted."""
import numpy as np
import pytest

from blitzgs_amd import synth
from oracle import oracle as O
from oracle import ref64


def _scene(seed, P=14, W=32, H=32, bg=(0.3, 0.1, 0.2)):
    scene, cam = synth.small_scene(P, seed=seed, W=W, H=H, extent=0.6, log_mu=-2.3, log_sd=0.3)
    scene["opacities"] = np.clip(scene["opacities"], 0.05, 0.85)   # o*G < 0.99: no clamp
    return scene, cam, np.asarray(bg, np.float32)


def _loss64(cam, sc, bg, ranges, plist, dLd):
    pr = ref64.project(cam, sc["means3D"], sc["scales"], sc["rotations"], sc["opacities"], sc["sh"])
    img, _, sig = ref64.render(cam["W"], cam["H"], bg, pr["means2D"], pr["conic"], pr["opacity"], pr["rgb"],
                               ranges, plist, signature=True)
    return float((img * dLd).sum()), sig


def _analytic(cam, scene, bg, dLd):
    pre, bn, rf = O.full_forward(cam, scene, bg=bg)
    rb = O.render_bwd(cam["W"], cam["H"], bg, pre["means2D"], pre["conic_opacity"], pre["rgb"], bn["ranges"],
                      bn["point_list"], rf["final_T"], rf["n_contrib_px"], dLd)
    pb = O.preprocess_bwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"], pre["radii"],
                          pre["cov3D"], pre["clamped"], rb["dL_dmeans2D"], rb["dL_dconic_opacity"],
                          rb["dL_dcolors"])
    return pre, bn, rb, pb


@pytest.mark.parametrize("seed", [1, 2])
def test_full_chain_gradients_match_finite_differences(seed):
    scene, cam, bg = _scene(seed)
    dLd = np.random.default_rng(seed).standard_normal((3, cam["H"], cam["W"]))
    pre, bn, rb, pb = _analytic(cam, scene, bg, dLd.astype(np.float32))
    assert (pre["radii"] > 0).all()
    groups = {"means3D": ("dL_dmeans3D", 1e-5), "scales": ("dL_dscales", 1e-6),
              "rotations": ("dL_drotations", 1e-5), "sh": ("dL_dsh", 1e-4), "opacities": ("dL_dopacity", 1e-5)}
    base = {k: np.asarray(v, np.float64) for k, v in scene.items() if k in groups}
    skipped = 0
    for name, (gname, h) in groups.items():
        ana = pb[gname].reshape(-1).astype(np.float64)
        fd = np.zeros_like(ana)
        keep = np.ones_like(ana, bool)
        flat = base[name].reshape(-1)
        for i in range(flat.size):
            sc = dict(base)
            p = flat.copy(); p[i] += h
            sc[name] = p.reshape(base[name].shape)
            lp, sp = _loss64(cam, sc, bg, bn["ranges"], bn["point_list"], dLd)
            p[i] -= 2 * h
            sc[name] = p.reshape(base[name].shape)
            lm, sm = _loss64(cam, sc, bg, bn["ranges"], bn["point_list"], dLd)
            fd[i] = (lp - lm) / (2 * h)
            if sp != sm:
                keep[i] = False
        skipped += (~keep).sum()
        err = np.linalg.norm(ana[keep] - fd[keep]) / max(np.linalg.norm(fd[keep]), 1e-12)
        assert err < 1e-3, (name, err)
    assert skipped < 10


def test_render_bwd_mean2d_is_ndc_scaled_and_abs_bounds():
    # dL/dmeans2D returned by the render backward is dL/d(ndc) = dL/dpx * W/2 (H/2)
    scene, cam, bg = _scene(7)
    dLd = np.random.default_rng(3).standard_normal((3, cam["H"], cam["W"]))
    pre, bn, rb, pb = _analytic(cam, scene, bg, dLd.astype(np.float32))
    pr = ref64.project(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["opacities"], scene["sh"])
    h = 1e-4
    for g in range(4):
        for ax, S in ((0, cam["W"]), (1, cam["H"])):
            m2 = pr["means2D"].copy()
            m2[g, ax] += h
            ip, _ = ref64.render(cam["W"], cam["H"], bg, m2, pr["conic"], pr["opacity"], pr["rgb"], bn["ranges"],
                                 bn["point_list"])
            m2[g, ax] -= 2 * h
            im, _ = ref64.render(cam["W"], cam["H"], bg, m2, pr["conic"], pr["opacity"], pr["rgb"], bn["ranges"],
                                 bn["point_list"])
            dpx = float(((ip - im) * dLd).sum()) / (2 * h)
            np.testing.assert_allclose(rb["dL_dmeans2D"][g, ax], dpx * 0.5 * S, rtol=2e-3, atol=1e-4)
    assert (rb["dL_dmeans2D_abs"][:, :2] >= np.abs(rb["dL_dmeans2D"][:, :2]) - 1e-5).all()
    assert not rb["dL_dmeans2D"][:, 2].any() and not rb["dL_dmeans2D_abs"][:, 2].any()
    # opacity gradient is copied through the preprocess backward for every Gaussian
    np.testing.assert_array_equal(pb["dL_dopacity"][:, 0], rb["dL_dconic_opacity"][:, 3])
