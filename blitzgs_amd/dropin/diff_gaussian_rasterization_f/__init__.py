"""Drop-in for BlitzGS's diff_gaussian_rasterization_f
(submodule/diff-gaussian-rasterization_f/diff_gaussian_rasterization_f/__init__.py):
the split training API, the full-image path (GaussianRasterizer.forward /
render_simp / markVisible) and SparseGaussianAdam, backed by the gfx950 HIP
library.  Render ops dispatch to the same library the _r drop-in uses (the
reference routes them to _r, __init__.py:24-46)."""
from blitzgs_amd import compat_ops as _C
from blitzgs_amd.adam import SparseGaussianAdam
from blitzgs_amd.fullpath import (_RasterizeGaussians, rasterize_gaussians, rasterize_gaussians_depth,
                                  rasterize_gaussians_simp)
from blitzgs_amd.rasterizer import (GaussianRasterizationSettings, GaussianRasterizer, _PreprocessGaussians,
                                    _RenderGaussians, preprocess_gaussians, render_gaussians)

_SPLIT_C = _C


def _get_split_op_backend(op_name):
    if hasattr(_C, op_name):
        return _C
    raise AttributeError(f"No backend provides split op '{op_name}'")


__all__ = ["GaussianRasterizationSettings", "GaussianRasterizer", "preprocess_gaussians", "render_gaussians",
           "rasterize_gaussians", "rasterize_gaussians_simp", "rasterize_gaussians_depth", "_get_split_op_backend",
           "_C", "SparseGaussianAdam"]
