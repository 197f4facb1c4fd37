"""Drop-in for the fused_ssim_cuda extension module (submodule/fused-ssim/ext.cpp:4-7)."""
from blitzgs_amd.ssim import fusedssim, fusedssim_backward

__all__ = ["fusedssim", "fusedssim_backward"]
