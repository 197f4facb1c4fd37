"""blitzgs_amd -- MI355X-native (gfx950 HIP) differentiable Gaussian rasterizer.

The compute path lives in the C-ABI library libblitzgs_amd.so (HIP kernels in
blitzgs_amd/csrc, declared in include/blitzgs_amd.h).  The Python modules here
mirror the reference's operator API:

  blitzgs_amd.rasterizer : GaussianRasterizationSettings / GaussianRasterizer
                           (preprocess_gaussians, render_gaussians) as in
                           diff_gaussian_rasterization_f/_r
  blitzgs_amd.knn        : distCUDA2 (simple_knn)
  blitzgs_amd.ssim       : fused_ssim
  blitzgs_amd.adam       : SparseGaussianAdam (the rasterizer package's sparse Adam step)
  blitzgs_amd.routing    : Gaussian -> rank routing and the screen-space pack / unpack
  blitzgs_amd.fullpath   : the full-image rasterize path (GaussianRasterizer.forward,
                           render_simp, markVisible)
  blitzgs_amd.plyio      : trained-scene PLY save / load (records <-> tensors on the GPU)
  blitzgs_amd.checkpoint : the training checkpoint tuple, file naming and resume
                           at another world size
Drop-in packages with the reference's module names live in blitzgs_amd/dropin.
"""
__version__ = "0.1.0"
