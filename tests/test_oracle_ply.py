"""CPU checks of the PLY layer: the numpy restatement of the reference's
save_ply / load_ply (oracle/o_ply.py) pinned by known-answer files written
byte by byte here, and the product's host logic (header, attribute names,
argument errors raised before any GPU work).

The reference holds no PLY fixture and plyfile is not installed, so the pins
are hand-assembled files: the header text and the record values are literal,
with f_rest values chosen so that a transposed or mis-sorted SH layout
produces different numbers."""
import struct

import numpy as np
import pytest

from oracle import o_ply

# P = 2, SH degree 1 (K = 3): rest[p, k, c] = 100 p + 10 k + c + 1
XYZ = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
DC = np.array([[[0.5, 0.25, -0.5]], [[1.5, -1.25, 2.0]]], np.float32)
REST = np.array([[[1, 2, 3], [11, 12, 13], [21, 22, 23]],
                 [[101, 102, 103], [111, 112, 113], [121, 122, 123]]], np.float32)
OPAC = np.array([[-1.0], [0.75]], np.float32)
SCALE = np.array([[-3, -4, -5], [-6, -7, -8]], np.float32)
ROT = np.array([[1, 0, 0, 0], [0.5, 0.5, 0.5, 0.5]], np.float32)

HEADER_SH1 = (b"ply\nformat binary_little_endian 1.0\nelement vertex 2\n"
              b"property float x\nproperty float y\nproperty float z\n"
              b"property float nx\nproperty float ny\nproperty float nz\n"
              b"property float f_dc_0\nproperty float f_dc_1\nproperty float f_dc_2\n"
              b"property float f_rest_0\nproperty float f_rest_1\nproperty float f_rest_2\n"
              b"property float f_rest_3\nproperty float f_rest_4\nproperty float f_rest_5\n"
              b"property float f_rest_6\nproperty float f_rest_7\nproperty float f_rest_8\n"
              b"property float opacity\n"
              b"property float scale_0\nproperty float scale_1\nproperty float scale_2\n"
              b"property float rot_0\nproperty float rot_1\nproperty float rot_2\nproperty float rot_3\n"
              b"end_header\n")
RECORDS_SH1 = [
    [1, 2, 3, 0, 0, 0, 0.5, 0.25, -0.5, 1, 11, 21, 2, 12, 22, 3, 13, 23, -1.0, -3, -4, -5, 1, 0, 0, 0],
    [4, 5, 6, 0, 0, 0, 1.5, -1.25, 2.0, 101, 111, 121, 102, 112, 122, 103, 113, 123, 0.75, -6, -7, -8,
     0.5, 0.5, 0.5, 0.5],
]


def known_file_bytes():
    return HEADER_SH1 + b"".join(struct.pack("<26f", *r) for r in RECORDS_SH1)


def test_save_matches_known_answer_bytes(tmp_path):
    p = tmp_path / "a.ply"
    names = o_ply.save_ply(str(p), XYZ, DC, REST, OPAC, SCALE, ROT)
    assert len(names) == 26
    assert p.read_bytes() == known_file_bytes()


def test_load_known_answer_file(tmp_path):
    p = tmp_path / "k.ply"
    p.write_bytes(known_file_bytes())
    g = o_ply.load_ply(str(p), 1)
    np.testing.assert_array_equal(g["xyz"], XYZ)
    np.testing.assert_array_equal(g["features_dc"], DC)
    np.testing.assert_array_equal(g["features_rest"], REST)
    np.testing.assert_array_equal(g["opacity"], OPAC)
    np.testing.assert_array_equal(g["scaling"], SCALE)
    np.testing.assert_array_equal(g["rotation"], ROT)
    assert g["lod_level"] is None
    for k in ("xyz", "features_dc", "features_rest", "opacity", "scaling", "rotation"):
        assert g[k].dtype == np.float32 and g[k].flags.c_contiguous


def test_load_sh_degree_mismatch_raises(tmp_path):
    p = tmp_path / "k.ply"
    p.write_bytes(known_file_bytes())
    with pytest.raises(ValueError):
        o_ply.load_ply(str(p), 3)   # 9 f_rest values cannot be reshaped to (3, 15)


def test_ascii_shuffled_with_extras(tmp_path):
    """ascii body, comments, property order shuffled, an extra uchar property,
    a second element after the vertices; SH degree 0 (no f_rest)."""
    txt = ("ply\nformat ascii 1.0\ncomment made by hand\n"
           "element vertex 2\n"
           "property float opacity\nproperty float rot_1\nproperty float rot_0\nproperty float rot_3\n"
           "property float rot_2\nproperty uchar red\nproperty float scale_1\nproperty float scale_0\n"
           "property float scale_2\nproperty float f_dc_2\nproperty float f_dc_0\nproperty float f_dc_1\n"
           "property float z\nproperty float x\nproperty float y\n"
           "element face 1\nproperty list uchar int vertex_indices\n"
           "end_header\n"
           "0.5 0.1 0.9 0.3 0.2 255 -2 -1 -3 7 5 6 3 1 2\n"
           "-0.5 1 2 4 3 0 -5 -4 -6 10 8 9 30 10 20\n"
           "3 0 1 1\n")
    p = tmp_path / "a.ply"
    p.write_bytes(txt.encode())
    g = o_ply.load_ply(str(p), 0)
    np.testing.assert_array_equal(g["xyz"], np.array([[1, 2, 3], [10, 20, 30]], np.float32))
    np.testing.assert_array_equal(g["features_dc"], np.array([[[5, 6, 7]], [[8, 9, 10]]], np.float32))
    assert g["features_rest"].shape == (2, 0, 3)
    np.testing.assert_array_equal(g["opacity"], np.array([[0.5], [-0.5]], np.float32))
    np.testing.assert_array_equal(g["scaling"], np.array([[-1, -2, -3], [-4, -5, -6]], np.float32))
    np.testing.assert_array_equal(g["rotation"], np.array([[0.9, 0.1, 0.2, 0.3], [2, 1, 3, 4]], np.float32))


def test_big_endian_doubles_round_to_float32(tmp_path):
    """binary_big_endian with double properties: values are rounded to float32
    (a double that is not a float32 checks the rounding)."""
    names = ["x", "y", "z", "f_dc_0", "f_dc_1", "f_dc_2", "opacity", "scale_0", "rot_0", "lod_level"]
    hdr = ("ply\nformat binary_big_endian 1.0\nelement vertex 1\n"
           + "".join(f"property double {n}\n" for n in names) + "end_header\n").encode()
    vals = [0.1, 1e-40, -2.5, 1.0 + 2.0 ** -30, 3.0, 4.0, 0.3, -1.0, 1.0, 2.0]
    p = tmp_path / "b.ply"
    p.write_bytes(hdr + struct.pack(">10d", *vals))
    g = o_ply.load_ply(str(p), 0)
    np.testing.assert_array_equal(g["xyz"], np.array([[np.float32(0.1), np.float32(1e-40), -2.5]], np.float32))
    assert g["features_dc"][0, 0, 0] == np.float32(1.0)      # 1 + 2^-30 rounds to 1 in float32
    assert g["lod_level"].dtype == np.int8 and g["lod_level"][0] == 2
    assert g["scaling"].shape == (1, 1) and g["rotation"].shape == (1, 1)


def test_f_rest_sorted_numerically(tmp_path):
    """SH degree 3: 45 f_rest properties written in reverse order; the loader
    sorts them by their integer (f_rest_10 after f_rest_9), so the tensor is
    the same as for the natural order."""
    rng = np.random.default_rng(0)
    P = 5
    rest = rng.standard_normal((P, 15, 3)).astype(np.float32)
    flat = np.ascontiguousarray(rest.transpose(0, 2, 1)).reshape(P, 45)
    names = ["x", "y", "z", "f_dc_0", "f_dc_1", "f_dc_2", "opacity"] + [f"f_rest_{i}" for i in range(44, -1, -1)]
    cols = np.concatenate([np.zeros((P, 7), np.float32), flat[:, ::-1]], axis=1)
    p = tmp_path / "s.ply"
    p.write_bytes(o_ply.header_bytes(names, P) + cols.astype("<f4").tobytes())
    g = o_ply.load_ply(str(p), 3)
    np.testing.assert_array_equal(g["features_rest"], rest)
    # spot values: file property f_rest_{c*15+k} holds rest[:, k, c]
    assert g["features_rest"][2, 4, 1] == flat[2, 1 * 15 + 4]


def test_round_trip_sh3_with_lod(tmp_path):
    rng = np.random.default_rng(1)
    P = 300
    xyz = rng.standard_normal((P, 3)).astype(np.float32)
    dc = rng.standard_normal((P, 1, 3)).astype(np.float32)
    rest = rng.standard_normal((P, 15, 3)).astype(np.float32)
    op = rng.standard_normal((P, 1)).astype(np.float32)
    sc = rng.standard_normal((P, 3)).astype(np.float32)
    rot = rng.standard_normal((P, 4)).astype(np.float32)
    lod = rng.integers(-3, 20, P).astype(np.int8)
    p = tmp_path / "r.ply"
    names = o_ply.save_ply(str(p), xyz, dc, rest, op, sc, rot, lod)
    assert names[-1] == "lod_level" and len(names) == 63
    assert p.stat().st_size == len(o_ply.header_bytes(names, P)) + P * 63 * 4
    g = o_ply.load_ply(str(p), 3)
    for k, v in (("xyz", xyz), ("features_dc", dc), ("features_rest", rest), ("opacity", op), ("scaling", sc),
                 ("rotation", rot), ("lod_level", lod)):
        np.testing.assert_array_equal(g[k], v)


# ------------------------------------------------------------------ product host logic (no GPU)

def test_product_header_and_names_match():
    from blitzgs_amd import plyio
    names = plyio.construct_list_of_attributes(DC, REST, SCALE, ROT)
    assert names == o_ply.attribute_names(DC.shape[1:], REST.shape[1:], 3, 4)
    assert plyio.ply_header(names, 2) == HEADER_SH1


def test_product_header_parser(tmp_path):
    from blitzgs_amd import plyio
    p = tmp_path / "k.ply"
    p.write_bytes(known_file_bytes())
    h = plyio.read_ply_header(str(p))
    assert h.format == "binary_little_endian" and h.body_offset == len(HEADER_SH1)
    assert h.elements[0][0] == "vertex" and h.elements[0][1] == 2
    assert [n for n, _ in h.elements[0][2]] == plyio.construct_list_of_attributes(DC, REST, SCALE, ROT)
    assert all(t == "f4" for _, t in h.elements[0][2])
    bad = tmp_path / "bad.ply"
    bad.write_bytes(b"plx\n")
    with pytest.raises(ValueError):
        plyio.read_ply_header(str(bad))
    bad.write_bytes(b"ply\nformat binary_little_endian 1.0\nelement vertex 1\nproperty float x\n")
    with pytest.raises(ValueError):
        plyio.read_ply_header(str(bad))
    bad.write_bytes(b"ply\nformat binary_middle_endian 1.0\nelement vertex 1\nproperty float x\nend_header\n")
    with pytest.raises(ValueError):
        plyio.read_ply_header(str(bad))


def test_product_load_errors_before_gpu(tmp_path):
    from blitzgs_amd import plyio
    p = tmp_path / "k.ply"
    p.write_bytes(known_file_bytes())
    with pytest.raises(ValueError, match="reshape"):
        plyio.load_ply(str(p), 3)
    names = ["x", "y", "opacity", "f_dc_0", "f_dc_1", "f_dc_2"]
    q = tmp_path / "m.ply"
    q.write_bytes(o_ply.header_bytes(names, 1) + np.zeros(6, "<f4").tobytes())
    with pytest.raises(ValueError, match="no field of name z"):
        plyio.load_ply(str(q), 0)
