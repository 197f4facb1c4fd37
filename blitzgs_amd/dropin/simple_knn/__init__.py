"""Drop-in for BlitzGS's simple_knn (submodule/simple-knn): `from simple_knn._C import distCUDA2`."""
