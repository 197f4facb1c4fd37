"""Drop-in for BlitzGS's diff_gaussian_rasterization_r
(submodule/diff-gaussian-rasterization_r/diff_gaussian_rasterization_r/__init__.py):
same operators; its settings record carries render_geo."""
from typing import NamedTuple

import torch

from blitzgs_amd import compat_ops as _C
from blitzgs_amd.rasterizer import (GaussianRasterizer, _PreprocessGaussians, _RenderGaussians,
                                    preprocess_gaussians, render_gaussians)


class GaussianRasterizationSettings(NamedTuple):
    image_height: int
    image_width: int
    tanfovx: float
    tanfovy: float
    bg: torch.Tensor
    scale_modifier: float
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    sh_degree: int
    campos: torch.Tensor
    prefiltered: bool
    render_geo: bool
    debug: bool


__all__ = ["GaussianRasterizationSettings", "GaussianRasterizer", "preprocess_gaussians", "render_gaussians", "_C"]
