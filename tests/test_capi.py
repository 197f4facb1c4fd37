"""CPU-side checks of the C ABI: the library builds for gfx950, loads, and
exports every entry point include/blitzgs_amd.h declares; workspace size
queries are consistent.  No compute call is made (no GPU here)."""
import ctypes as C
import os
import re

import pytest

from blitzgs_amd import _lib, build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "blitzgs_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gs_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if build.needs_build():
        build.build(force=True)
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    # the Python binding covers every declared entry point
    assert set(names) <= set(_lib.exported_symbols())


def test_workspace_queries(lib):
    g = lib.gs_render_geom_bytes(6_000_000, 1600, 1066)
    assert g % 256 == 0 and g > 4 * 100 * 67
    assert lib.gs_render_img_bytes(1600, 1066) >= 1600 * 1066 * 12 + 100 * 67 * 8
    assert lib.gs_render_binning_bytes(0) >= 256
    assert lib.gs_render_binning_bytes(1000) >= 1000 * 20
    assert lib.gs_version() >= 100


def test_argument_errors_without_device(lib):
    # argument validation happens before any HIP call
    rc = lib.gs_preprocess_forward(10, 4, 16, *([None] * 5), C.c_float(1.0), None, None, None, C.c_float(1.0),
                                   C.c_float(1.0), 10, 10, *([None] * 7), None)
    assert rc != 0 and b"sh_degree" in lib.gs_last_error()
    rc = lib.gs_preprocess_forward(10, 3, 9, *([None] * 5), C.c_float(1.0), None, None, None, C.c_float(1.0),
                                   C.c_float(1.0), 10, 10, *([None] * 7), None)
    assert rc != 0 and b"coefficients" in lib.gs_last_error()
    rc = lib.gs_diag_math(7, 1, None, None, None)
    assert rc != 0 and b"op" in lib.gs_last_error()
