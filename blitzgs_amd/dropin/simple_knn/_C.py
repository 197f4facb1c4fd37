from blitzgs_amd.knn import distCUDA2

__all__ = ["distCUDA2"]
