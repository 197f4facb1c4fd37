"""The oracle's decision margins (oracle.render_fwd's stop_near / obs_near),
which the GPU tests use to attribute every differing integer output of the
blend (last contributor, contributor count, out_observe, per-tile sums) to a
decision near its threshold.

Pinned here by emulation: the oracle's own blend is rerun with every exp
perturbed by a relative +-delta (sign hashed per Gaussian and pixel; the
alpha >= 1/255 cut stays exact, as the device's guard window keeps it), and
every change in its integer outputs must be attributed by the margins of the
unperturbed run computed for an exp error of 2 * delta.  With margins for a
much smaller error the same changes must NOT all be attributed (the check
has teeth), and with no perturbation nothing changes."""
import numpy as np
import pytest

from blitzgs_amd import synth
from oracle import oracle as O
from tests.gpu_helpers import assert_blend_counts


def _scene():
    scene, cam = synth.config0()
    pre = O.preprocess_fwd(cam, scene["means3D"], scene["scales"], scene["rotations"], scene["sh"],
                           scene["opacities"])
    W, H = int(cam["W"]), int(cam["H"])
    bn = O.binning(W, H, pre["means2D"], pre["depths"], pre["radii"])
    return W, H, pre, bn


def _render(W, H, pre, bn, delta, bound_rel):
    O.set_blend_margin_model(delta, bound_rel)
    try:
        return O.render_fwd(W, H, np.zeros(3, np.float32), pre["means2D"], pre["conic_opacity"], pre["rgb"],
                            bn["ranges"], bn["point_list"])
    finally:
        O.set_blend_margin_model()


def _counts(rf):
    return {k: rf[k] for k in ("n_contrib_px", "n_contrib2loss_px", "out_observe", "n_consider", "n_contrib")}


@pytest.mark.parametrize("delta", [1e-4, 1e-3])
def test_margins_attribute_every_change_of_a_perturbed_blend(delta):
    W, H, pre, bn = _scene()
    ref = _render(W, H, pre, bn, 0.0, 2 * delta)
    got = _render(W, H, pre, bn, delta, 2 * delta)
    s = assert_blend_counts(_counts(got), ref, f"exp perturbed by {delta:g}")
    # the perturbation really moved decisions (else the check above is empty)
    assert s["n_contrib_px"] > 0 and s["out_observe"] > 0, s


def test_margins_too_small_do_not_attribute():
    W, H, pre, bn = _scene()
    delta = 3e-4
    ref = _render(W, H, pre, bn, 0.0, delta / 100)
    got = _render(W, H, pre, bn, delta, delta / 100)
    with pytest.raises(AssertionError):
        assert_blend_counts(_counts(got), ref)


def test_margins_unperturbed_and_default_model():
    W, H, pre, bn = _scene()
    ref = O.render_fwd(W, H, np.zeros(3, np.float32), pre["means2D"], pre["conic_opacity"], pre["rgb"],
                       bn["ranges"], bn["point_list"])
    s = assert_blend_counts(_counts(ref), ref)
    assert all(v == 0 for v in s.values()), s
    # the default model (exp within 4e-6 relative) marks only a sliver of the decisions
    assert ref["stop_near"].mean() < 1e-3
    assert ref["obs_near"].sum() < 1e-3 * ref["out_observe"].sum()
