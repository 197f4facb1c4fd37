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

try:
    import diff_gaussian_rasterization_r as _split_package
    _SPLIT_C = _split_package._C
except ImportError:
    _SPLIT_C = None

# render ops must come from the _r package (a missing one is an error, not a
# fallback); every other op comes from this package first
_SPLIT_ONLY = ("render_gaussians", "render_gaussians_backward")


def _get_split_op_backend(op_name):
    """The module that provides split op `op_name` (_f __init__.py:24-46)."""
    if op_name in _SPLIT_ONLY:
        if _SPLIT_C is None or not hasattr(_SPLIT_C, op_name):
            raise AttributeError(f"Missing split backend op '{op_name}': the diff_gaussian_rasterization_r "
                                 "drop-in must be importable for the render ops")
        return _SPLIT_C
    for backend in (_C, _SPLIT_C):
        if backend is not None and hasattr(backend, op_name):
            return backend
    raise AttributeError(f"No backend provides split op '{op_name}'")


__all__ = ["GaussianRasterizationSettings", "GaussianRasterizer", "preprocess_gaussians", "render_gaussians",
           "rasterize_gaussians", "rasterize_gaussians_simp", "rasterize_gaussians_depth", "_get_split_op_backend",
           "_C", "SparseGaussianAdam"]
