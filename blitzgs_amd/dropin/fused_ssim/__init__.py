"""Drop-in for fused-ssim (submodule/fused-ssim/fused_ssim/__init__.py)."""
from blitzgs_amd.ssim import FusedSSIMMap, allowed_padding, fused_ssim

__all__ = ["fused_ssim", "FusedSSIMMap", "allowed_padding"]
