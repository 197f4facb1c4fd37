"""GPU parity of the PLY layer (blitzgs_amd.plyio, blitzgs_amd/csrc/plyio.hip)
through the C ABI.

* save_ply on the GPU writes the same bytes as the CPU restatement of the
  reference's save_ply (oracle/o_ply.py), for SH degrees 0 / 1 / 3, with and
  without lod_level, at record counts around the kernel's 128-row blocks;
* load_ply on the GPU returns bit for bit the oracle's tensors for files in
  the reference's layout, with shuffled property order, extra properties and
  elements, double / big-endian / ascii bodies, more properties than the
  kernel's direct path takes, and several staging chunks;
* at config 2's size (6M SH-degree-3 Gaussians) unpack matches the
  reference's torch expressions (slices, view, transpose) and pack inverts it;
* argument errors of the C ABI.
Values are compared as bit patterns (special values included): the path only
moves them.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from blitzgs_amd import _lib, plyio
from oracle import o_ply

pytestmark = pytest.mark.gpu


def scene(P, K, seed, lod=False):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    s = dict(xyz=f(P, 3), features_dc=f(P, 1, 3), features_rest=f(P, K, 3), opacity=f(P, 1), scaling=f(P, 3),
             rotation=f(P, 4), lod_level=rng.integers(-5, 30, P).astype(np.int8) if lod else None)
    if P >= 4:   # special values travel unchanged
        s["xyz"][0] = [-0.0, np.inf, -np.inf]
        s["xyz"][1] = [np.nan, 1e-45, -1e-40]
        s["opacity"][2] = np.finfo(np.float32).max
    return s


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.int32) if a.dtype == np.float32 else a


def assert_same(got, ref):
    for k in ("xyz", "features_dc", "features_rest", "opacity", "scaling", "rotation"):
        g = getattr(got, k)
        assert g.is_cuda and g.dtype == torch.float32 and g.is_contiguous(), k
        assert tuple(g.shape) == ref[k].shape, k
        np.testing.assert_array_equal(bits(g.cpu().numpy()), bits(ref[k]), err_msg=k)
    if ref["lod_level"] is None:
        assert got.lod_level is None
    else:
        assert got.lod_level.dtype == torch.int8
        np.testing.assert_array_equal(got.lod_level.cpu().numpy(), ref["lod_level"])


def to_gpu(s):
    return {k: (torch.from_numpy(v).cuda() if v is not None else None) for k, v in s.items()}


def save_both(tmp_path, s, tag):
    a, b = tmp_path / f"{tag}_gpu.ply", tmp_path / f"{tag}_ref.ply"
    t = to_gpu(s)
    plyio.save_ply(str(a), t["xyz"], t["features_dc"], t["features_rest"], t["opacity"], t["scaling"],
                   t["rotation"], t["lod_level"])
    o_ply.save_ply(str(b), s["xyz"], s["features_dc"], s["features_rest"], s["opacity"], s["scaling"],
                   s["rotation"], s["lod_level"])
    return a, b


@pytest.mark.parametrize("P", [0, 1, 127, 128, 129, 1000, 50_001])
@pytest.mark.parametrize("K,lod", [(15, False), (15, True), (3, False), (0, True)])
def test_save_bytes_match_oracle(gpu, tmp_path, P, K, lod):
    print(f"save P={P} K={K} lod={lod}", flush=True)
    s = scene(P, K, seed=P + K, lod=lod)
    a, b = save_both(tmp_path, s, "s")
    assert a.read_bytes() == b.read_bytes()


@pytest.mark.parametrize("P", [0, 1, 129, 20_000])
@pytest.mark.parametrize("K,lod", [(15, False), (15, True), (3, True), (0, False)])
def test_load_matches_oracle(gpu, tmp_path, P, K, lod):
    print(f"load P={P} K={K} lod={lod}", flush=True)
    s = scene(P, K, seed=7 + P, lod=lod)
    _, b = save_both(tmp_path, s, "l")
    deg = {0: 0, 3: 1, 15: 3}[K]
    assert_same(plyio.load_ply(str(b), deg), o_ply.load_ply(str(b), deg))


def _write_custom(path, cols, names, types=None, fmt="binary_little_endian"):
    """A PLY file with the given columns (list of 1-D arrays) and property types."""
    P = len(cols[0])
    types = types or ["float"] * len(names)
    hdr = o_ply.header_bytes(names, P, fmt=fmt, types=types, comments=["custom"])
    np_t = {"float": "f4", "double": "f8", "uchar": "u1", "int": "i4", "short": "i2"}
    if fmt == "ascii":
        body = "".join(" ".join(repr(float(c[i])) if t in ("float", "double") else str(int(c[i]))
                                for c, t in zip(cols, types)) + "\n" for i in range(P)).encode()
    else:
        bo = "<" if fmt == "binary_little_endian" else ">"
        dt = np.dtype([(n, bo + np_t[t]) for n, t in zip(names, types)])
        rec = np.empty(P, dtype=dt)
        for n, c in zip(names, cols):
            rec[n] = c
        body = rec.tobytes()
    path.write_bytes(hdr + body)


def _natural(s, lod):
    P = s["xyz"].shape[0]
    K = s["features_rest"].shape[1]
    flat = np.ascontiguousarray(s["features_rest"].transpose(0, 2, 1)).reshape(P, -1)
    cols = [s["xyz"][:, i] for i in range(3)] + [s["features_dc"][:, 0, c] for c in range(3)]
    cols += [flat[:, i] for i in range(3 * K)] + [s["opacity"][:, 0]]
    cols += [s["scaling"][:, i] for i in range(3)] + [s["rotation"][:, i] for i in range(4)]
    names = (["x", "y", "z", "f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{i}" for i in range(3 * K)]
             + ["opacity", "scale_0", "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"])
    if lod:
        cols.append(s["lod_level"].astype(np.float32))
        names.append("lod_level")
    return cols, names


@pytest.mark.parametrize("variant", ["shuffled_extras", "double_le", "big_endian", "ascii", "wide", "int_props"])
def test_load_variants_match_oracle(gpu, tmp_path, variant):
    print(f"variant {variant}", flush=True)
    P = 300 if variant == "ascii" else 5000
    s = scene(P, 15, seed=11, lod=True)
    cols, names = _natural(s, lod=True)
    rng = np.random.default_rng(3)
    types = None
    fmt = "binary_little_endian"
    if variant == "shuffled_extras":
        cols += [rng.standard_normal(P).astype(np.float32), np.zeros(P, np.float32)]
        names += ["red", "nx"]
        perm = rng.permutation(len(names))
        cols, names = [cols[i] for i in perm], [names[i] for i in perm]
    elif variant in ("double_le", "big_endian"):
        cols = [c.astype(np.float64) + 1e-9 for c in cols]     # not float32 values: rounding is exercised
        types = ["double"] * len(names)
        fmt = "binary_little_endian" if variant == "double_le" else "binary_big_endian"
    elif variant == "ascii":
        fmt = "ascii"
        s["xyz"][:3] = 1.0                                     # no inf / nan in text
        cols, names = _natural(s, lod=True)
    elif variant == "wide":
        cols += [rng.standard_normal(P).astype(np.float32) for _ in range(70)]   # 133 properties
        names += [f"extra_{i}" for i in range(70)]
    elif variant == "int_props":
        types = ["float"] * len(names)
        types[-1] = "short"                                    # lod_level stored as an integer
        cols[-1] = s["lod_level"].astype(np.int16)
        cols.append(rng.integers(0, 255, P).astype(np.uint8))
        names.append("alpha")
        types.append("uchar")
    p = tmp_path / f"{variant}.ply"
    _write_custom(p, cols, names, types, fmt)
    ref = o_ply.load_ply(str(p), 3)
    assert_same(plyio.load_ply(str(p), 3), ref)


def test_load_many_chunks(gpu, tmp_path, monkeypatch):
    s = scene(10_007, 15, seed=5, lod=True)
    _, b = save_both(tmp_path, s, "c")
    monkeypatch.setattr(plyio, "_CHUNK_BYTES", 252 * 333)     # 333 records per chunk, ragged last chunk
    assert_same(plyio.load_ply(str(b), 3), o_ply.load_ply(str(b), 3))
    a = tmp_path / "c_gpu2.ply"
    t = to_gpu(s)
    plyio.save_ply(str(a), t["xyz"], t["features_dc"], t["features_rest"], t["opacity"], t["scaling"],
                   t["rotation"], t["lod_level"])
    assert a.read_bytes() == b.read_bytes()


def test_truncated_file_raises(gpu, tmp_path):
    s = scene(500, 15, seed=2)
    _, b = save_both(tmp_path, s, "t")
    data = b.read_bytes()
    b.write_bytes(data[:-100])
    with pytest.raises(ValueError, match="truncated"):
        plyio.load_ply(str(b), 3)


def test_full_size_unpack_and_pack(gpu):
    """Config 2's 6M SH-3 Gaussians: 62-column records in HBM.  Unpack equals
    the reference's load expressions written in torch (column slices, the
    (P,3,15) view transposed to (P,15,3)); pack gives the records back with
    zero normals."""
    P, n = 6_000_000, 62
    print(f"full size P={P}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    rec = torch.randn((P, n), device="cuda", generator=g)
    names = plyio.construct_list_of_attributes(torch.empty(0, 1, 3), torch.empty(0, 15, 3), torch.empty(0, 3),
                                               torch.empty(0, 4))
    idx = {nm: i for i, nm in enumerate(names)}
    cm = [[0, 1, 2], [6, 7, 8], [idx[f"f_rest_{c * 15 + k}"] for k in range(15) for c in range(3)], [54],
          [55, 56, 57], [58, 59, 60, 61]]
    xyz, dc, rest, op, sc, rot = plyio.unpack_records(rec, cm, [(3,), (1, 3), (15, 3), (1,), (3,), (4,)])
    torch.cuda.synchronize()
    assert torch.equal(xyz, rec[:, 0:3])
    assert torch.equal(dc, rec[:, 6:9].reshape(P, 3, 1).transpose(1, 2))
    assert torch.equal(rest, rec[:, 9:54].reshape(P, 3, 15).transpose(1, 2))
    assert torch.equal(op, rec[:, 54:55]) and torch.equal(sc, rec[:, 55:58]) and torch.equal(rot, rec[:, 58:62])
    back, nm2 = plyio.pack_records(xyz, dc, rest, op, sc, rot)
    assert nm2 == names
    exp = rec.clone()
    exp[:, 3:6] = 0
    assert torch.equal(back, exp)


def test_file_round_trip_1m(gpu, tmp_path):
    P = 1_000_000
    print(f"file round trip P={P}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1)
    r = lambda *s: torch.randn(s, device="cuda", generator=g)
    xyz, dc, rest, op, sc, rot = r(P, 3), r(P, 1, 3), r(P, 15, 3), r(P, 1), r(P, 3), r(P, 4)
    lod = torch.randint(-10, 40, (P,), device="cuda", generator=g).to(torch.int8)
    p = tmp_path / "big.ply"
    names = plyio.save_ply(str(p), xyz, dc, rest, op, sc, rot, lod)
    assert p.stat().st_size == len(plyio.ply_header(names, P)) + P * 63 * 4
    got = plyio.load_ply(str(p), 3)
    for a, b in zip(got[:6], (xyz, dc, rest, op, sc, rot)):
        assert torch.equal(a, b)
    assert torch.equal(got.lod_level, lod) and got.active_sh_degree == 3


def test_capi_argument_errors(gpu):
    lib = _lib.load()
    x = torch.zeros((256, 4), device="cuda")
    rec = torch.zeros((256, 8), device="cuda")
    st = _lib.stream_of()

    def spec(*ws):
        arr = (_lib.PlyTensor * len(ws))()
        for i, w in enumerate(ws):
            arr[i].ptr, arr[i].width, arr[i].type = x.data_ptr(), w, 0
        return arr

    cm = lambda *v: (C.c_int32 * len(v))(*v)
    assert lib.gs_ply_unpack(256, _lib.ptr(rec), 8, 1, spec(4), cm(0, 1, 2, 8), st) != 0
    assert b"colmap[3]" in lib.gs_last_error()
    assert lib.gs_ply_unpack(256, _lib.ptr(rec), 121, 1, spec(4), cm(0, 1, 2, 3), st) != 0
    assert b"rec_cols" in lib.gs_last_error()
    assert lib.gs_ply_pack(256, 1, spec(4), cm(0, 1, 1, 3), 8, _lib.ptr(rec), st) != 0
    assert b"two tensor columns" in lib.gs_last_error()
    assert lib.gs_ply_unpack(256, _lib.ptr(rec), 8, 1, spec(0), cm(0), st) != 0
    assert b"width" in lib.gs_last_error()
    assert lib.gs_ply_unpack(256, _lib.ptr(rec), 8, 9, spec(*[1] * 9), cm(*range(8), 0), st) != 0
    assert b"n_tensors" in lib.gs_last_error()
    # unpack may read one record column into two tensor columns
    y = torch.empty((256, 2), device="cuda")
    arr = (_lib.PlyTensor * 1)()
    arr[0].ptr, arr[0].width, arr[0].type = y.data_ptr(), 2, 0
    rec2 = torch.arange(256 * 8, dtype=torch.float32, device="cuda").reshape(256, 8)
    assert lib.gs_ply_unpack(256, _lib.ptr(rec2), 8, 1, arr, cm(5, 5), st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, rec2[:, [5, 5]])
