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


def _declarations():
    """{name: (return type, [parameter types])} of every entry point in the header."""
    src = open(os.path.join(ROOT, "include", "blitzgs_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"#[^\n]*", "", src)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w ]*?[\s\*]+)(gs_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        types = []
        if params and params != "void":
            for prm in params.split(","):
                prm = " ".join(prm.split())
                # drop the parameter name: the last identifier
                types.append(re.sub(r"\s*\b\w+$", "", prm).strip() if not prm.endswith("*") else prm)
        out[name] = (ret, types)
    return out


def _ctype_class(decl):
    """The ctypes class a C parameter type must be bound with."""
    if "*" in decl or decl == "gs_stream_t":
        return "pointer"
    base = decl.replace("const ", "").strip()
    return {"int": C.c_int, "int32_t": C.c_int32, "int64_t": C.c_int64, "float": C.c_float,
            "size_t": C.c_size_t}[base]


def test_binding_signatures_match_the_header():
    """Every argtypes entry of the ctypes binding has the arity and the kind
    (pointer / int / int64 / float) of the header's declaration, so a call
    with a missing or extra argument cannot pass silently."""
    decls = _declarations()
    assert len(decls) >= 30
    for name, (res, args) in _lib._SIGS.items():
        assert name in decls, name
        ret, params = decls[name]
        assert len(args) == len(params), (name, len(args), len(params))
        for i, (a, p) in enumerate(zip(args, params)):
            want = _ctype_class(p)
            if want == "pointer":
                assert a is C.c_void_p or a is C.c_char_p or hasattr(a, "_type_") and issubclass(a, C._Pointer), \
                    (name, i, p, a)
            else:
                assert a is want, (name, i, p, a)


def test_workspace_queries(lib):
    g = lib.gs_render_geom_bytes(6_000_000, 1600, 1066)
    assert g % 256 == 0 and g > 4 * 100 * 67
    assert lib.gs_render_img_bytes(1600, 1066) >= 1600 * 1066 * 12 + 100 * 67 * 8
    assert lib.gs_render_binning_bytes(0) >= 256
    # compact list (4 B), point list (4 B) and keys (8 B) per instance
    assert lib.gs_render_binning_bytes(1000) >= 1000 * 16
    assert lib.gs_version() >= 100


def test_argument_errors_without_device(lib):
    # argument validation happens before any HIP call
    rc = lib.gs_preprocess_forward(10, 4, 16, *([None] * 5), C.c_float(1.0), None, None, None, C.c_float(1.0),
                                   C.c_float(1.0), 10, 10, *([None] * 7), None)
    assert rc != 0 and b"sh_degree" in lib.gs_last_error()
    rc = lib.gs_preprocess_forward(10, 3, 9, *([None] * 5), C.c_float(1.0), None, None, None, C.c_float(1.0),
                                   C.c_float(1.0), 10, 10, *([None] * 7), None)
    assert rc != 0 and b"coefficients" in lib.gs_last_error()
    rc = lib.gs_diag_math(10, 1, None, None, None)
    assert rc != 0 and b"op" in lib.gs_last_error()
    # timing modes: 0 off, 1 every kernel and the stages, 2 the stages only
    rc = lib.gs_timing_enable(3)
    assert rc != 0 and b"timing mode" in lib.gs_last_error()
    for mode in (2, 1, 0):
        assert lib.gs_timing_enable(mode) == 0


def test_routing_argument_errors_without_device(lib):
    # all of these fail in argument checks, before any HIP call
    rc = lib.gs_local2j_ids_bool(7, 10, 64, 64, 2, None, None, None, 0, None, None)
    assert rc != 0 and b"mode" in lib.gs_last_error()
    rc = lib.gs_local2j_ids_bool(0, 10, 64, 64, 0, None, None, None, 0, None, None)
    assert rc != 0 and b"world_size" in lib.gs_last_error()
    rc = lib.gs_local2j_count(0, 10, 64, 64, 65, C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), 0, None,
                              C.c_void_p(16), C.c_void_p(16), None)
    assert rc != 0 and b"exceeds 64" in lib.gs_last_error()
    assert lib.gs_local2j_workspace_bytes(6_000_000, 4) >= 4 * 4
    assert lib.gs_local2j_workspace_bytes(-1, 4) == 0
    f = (_lib.RowField * 1)(_lib.RowField(src=16, dst=16, src_stride=40, dst_stride=40, width=40, src_type=0,
                                          dst_type=0))
    rc = lib.gs_move_rows(10, None, 10, None, 10, 1, f, 0, None)
    assert rc != 0 and b"columns" in lib.gs_last_error()
    f = (_lib.RowField * 1)(_lib.RowField(src=16, dst=16, src_stride=1, dst_stride=1, width=1, src_type=0,
                                          dst_type=1))
    rc = lib.gs_move_rows(10, None, 10, None, 10, 1, f, 1, None)
    assert rc != 0 and b"accumulate" in lib.gs_last_error()
    rc = lib.gs_move_rows(10, None, 10, None, 10, 9, f, 0, None)
    assert rc != 0 and b"n_fields" in lib.gs_last_error()
    rc = lib.gs_move_rows(11, None, 10, None, 11, 1, f, 0, None)
    assert rc != 0 and b"source rows" in lib.gs_last_error()


def test_render_geo_argument_errors_without_device(lib):
    # render_geo entry points: argument checks come before any HIP call
    nz = C.c_void_p(256)
    rc = lib.gs_render_geo_forward(10, 5, 64, 64, C.c_float(0.5), C.c_float(0.5), None, None, nz, nz, nz, nz, nz,
                                   None)
    assert rc != 0 and b"all_map" in lib.gs_last_error()
    rc = lib.gs_render_geo_forward(10, 5, 64, 64, C.c_float(0.0), C.c_float(0.5), nz, None, nz, nz, nz, nz, nz, None)
    assert rc != 0 and b"tan_fov" in lib.gs_last_error()
    rc = lib.gs_render_geo_forward(10, 5, 64, 64, C.c_float(0.5), C.c_float(0.5), nz, None, None, nz, nz, nz, nz,
                                   None)
    assert rc != 0 and b"workspaces" in lib.gs_last_error()
    # backward: every map input is required, and dL_dall_map
    args = [10, 5, 64, 64, nz, C.c_float(0.5), C.c_float(0.5), nz, nz, nz, nz, nz, None, nz, nz, nz, nz, nz, nz,
            nz, 3, nz, nz, nz, nz, None, 0, None]
    bad = list(args)
    bad[24] = None      # dL_dall_map
    assert lib.gs_render_backward_geo(*bad) != 0 and b"dL_dall_map" in lib.gs_last_error()
    bad = list(args)
    bad[17] = None      # dL_dout_all_map
    assert lib.gs_render_backward_geo(*bad) != 0 and b"dL_dout_all_map" in lib.gs_last_error()


def test_render_geo_shape_checks_without_device(lib):
    import torch
    from blitzgs_amd import rasterizer
    geom = torch.empty(16, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match=r"all_map of shape \(10, 5\)"):
        rasterizer._render_geo_forward_raw(10, 32, 32, 0.5, 0.5, torch.zeros(10, 4), None, 0, geom, geom, geom)
    with pytest.raises(RuntimeError, match=r"all_map of shape \(10, 5\)"):
        rasterizer._render_geo_forward_raw(10, 32, 32, 0.5, 0.5, None, None, 0, geom, geom, geom)


def test_region_side_checked_without_device(lib):
    """The split render's region side must be 0, 2, 4 or 8; checked before any HIP call."""
    nz = C.c_void_p(256)
    R = C.c_int64(0)
    rc = lib.gs_render_forward_count(10, 64, 64, nz, nz, None, nz, C.byref(R), 3, None)
    assert rc != 0 and b"region_side" in lib.gs_last_error()


def test_forward_clear_buffer_checked_without_device(lib):
    """The split forward's clear buffer (a caller buffer the blend zeroes):
    16-byte aligned and a whole number of 16-byte words, or none; checked
    before any HIP call, on both forward routes."""
    nz = C.c_void_p(256)
    R = C.c_int64(0)
    base = [10, 5, 64, 64] + [nz] * 5 + [nz, None] + [nz] * 3 + [nz] * 5
    for dst, nbytes in ((C.c_void_p(264), 32), (nz, 20), (None, 16), (nz, -16)):
        rc = lib.gs_render_forward(*base, 0, dst, C.c_int64(nbytes), None)
        assert rc != 0 and b"clear_dst" in lib.gs_last_error(), (dst, nbytes)
        rc = lib.gs_render_forward_reserved(*base, C.byref(R), 0, dst, C.c_int64(nbytes), None)
        assert rc != 0 and b"clear_dst" in lib.gs_last_error(), (dst, nbytes)


def test_region_side_choice_follows_instances_per_gaussian():
    """InstanceReserve.region_side: 4x4-tile regions after a forward with many
    tile instances per Gaussian, the default otherwise (and without history)."""
    from blitzgs_amd._lib import InstanceReserve
    r = InstanceReserve()
    assert r.region_side("cuda:0") == 0
    r.update("cuda:0", 27_000_000, 1_000_000)     # config 1's shape: 27 per Gaussian
    assert r.region_side("cuda:0") == 4
    r.update("cuda:0", 8_000_000, 6_000_000)      # config 2's shape: 1.3 per Gaussian
    assert r.region_side("cuda:0") == 0
    r.update("cuda:0", 5)                          # no P: the choice is kept
    assert r.region_side("cuda:0") == 0
    r.reset()
    assert r.region_side("cuda:0") == 0
