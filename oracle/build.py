"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/*.c with gcc into oracle/_build/liboracle_gs.so.  The flags
matter for bit-exactness: -ffp-contract=off keeps gcc from fusing a*b+c, so
the only fused multiply-adds are the fmaf() calls written in the source, which
the HIP kernels issue at the same places; -mfma makes those fmaf() calls
single instructions instead of libm calls.

The reference's own CUDA sources need nvcc, CUB and glm and cannot be built in
this image, so there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle_gs.so")
SOURCES = ["o_preprocess.c", "o_render.c", "o_knn_ssim.c", "o_adam.c", "o_route.c"]
HEADERS = ["o_math.h", "gs_oracle.h"]
CFLAGS = ["-O2", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-mfma", "-fno-math-errno", "-Wall", "-Wno-unused-function"]


def needs_build():
    if not os.path.exists(LIB):
        return True
    t = os.path.getmtime(LIB)
    return any(os.path.getmtime(os.path.join(HERE, f)) > t for f in SOURCES + HEADERS)


def build(force=False, verbose=False):
    if not force and not needs_build():
        return LIB
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["gcc"] + CFLAGS + [os.path.join(HERE, s) for s in SOURCES] + ["-o", LIB + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv, verbose=True))
