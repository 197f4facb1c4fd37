"""The drop-in packages import under the reference's module names and route
the split ops as the reference does (_f __init__.py:17-46): render ops only
from the _r package (missing -> AttributeError), other ops from _f first.
No compute call (runs without a GPU)."""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "blitzgs_amd", "dropin")


@pytest.fixture()
def dropin(monkeypatch):
    monkeypatch.syspath_prepend(DROPIN)
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)
    f = importlib.import_module("diff_gaussian_rasterization_f")
    r = importlib.import_module("diff_gaussian_rasterization_r")
    yield f, r
    for m in ("diff_gaussian_rasterization_f", "diff_gaussian_rasterization_r"):
        sys.modules.pop(m, None)


def test_split_op_dispatch(dropin, monkeypatch):
    f, r = dropin
    for op in ("render_gaussians", "render_gaussians_backward"):
        assert f._get_split_op_backend(op) is r._C
        assert callable(getattr(f._get_split_op_backend(op), op))
    for op in ("preprocess_gaussians", "preprocess_gaussians_backward", "get_local2j_ids_bool",
               "get_local2j_ids_bool_adjust_mode6", "mark_visible", "adamUpdate", "rasterize_gaussians"):
        assert f._get_split_op_backend(op) is f._C
    with pytest.raises(AttributeError):
        f._get_split_op_backend("no_such_op")
    # without the _r package the render ops are an error, not a fallback
    monkeypatch.setattr(f, "_SPLIT_C", None)
    with pytest.raises(AttributeError, match="render_gaussians"):
        f._get_split_op_backend("render_gaussians")
    assert f._get_split_op_backend("preprocess_gaussians") is f._C


def test_dropin_names(dropin):
    f, r = dropin
    for name in ("GaussianRasterizationSettings", "GaussianRasterizer", "SparseGaussianAdam", "_C"):
        assert hasattr(f, name), name
    assert "render_geo" in r.GaussianRasterizationSettings._fields
    assert "render_geo" not in f.GaussianRasterizationSettings._fields
    sys_path = list(sys.path)
    try:
        sys.path.insert(0, DROPIN)
        for m in ("simple_knn._C", "fused_ssim", "fused_ssim_cuda"):
            sys.modules.pop(m, None)
            mod = importlib.import_module(m)
            assert mod is not None
        assert callable(importlib.import_module("simple_knn._C").distCUDA2)
        assert callable(importlib.import_module("fused_ssim").fused_ssim)
        fsc = importlib.import_module("fused_ssim_cuda")
        assert callable(fsc.fusedssim) and callable(fsc.fusedssim_backward)
    finally:
        sys.path[:] = sys_path
