"""Trained-scene PLY files: save_ply / load_ply of the Gaussian parameters.

Mirrors BlitzGS scene/gaussian_model.py:
  :434-446  construct_list_of_attributes
  :447-520  save_ply  -- x y z, zero normals, f_dc_*, f_rest_* (features
            transposed to (P, 3, K) and flattened), opacity, scale_*, rot_*,
            optional lod_level; every value float32, one binary little-endian
            'vertex' element, written by plyfile in the reference
  :522-575  load_ply  -- reads those properties by name (f_rest_*, scale_*,
            rot* sorted by their trailing integer), reshapes f_rest to
            (P, 3, (max_sh_degree+1)^2 - 1) and transposes it back; float32
            tensors on the GPU, lod_level as int8

Design: the host only moves bytes.  Loading reads the vertex records in
64 MiB chunks into two pinned buffers (file read of one chunk overlaps the
host->device copy of the other) and one gs_ply_unpack launch splits the
records into the six parameter tensors with the SH transposes.  Saving is the
mirror: one gs_ply_pack launch builds the records in HBM, then chunked
device->host copies overlap the file writes.  Files that are not float32
little-endian records (ascii, big-endian, double or integer properties, more
than 120 properties) are decoded on the host first, converting each needed
property to float64 and then float32 as the reference's staging arrays do,
and go through the same kernel.
"""
import os
from typing import NamedTuple, Optional

import numpy as np
import torch

from . import _lib

PLY_TYPES = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}
_MAX_COLS = 120            # gs_ply_pack / gs_ply_unpack limit on record and tensor columns
_CHUNK_BYTES = 64 << 20    # host staging chunk


class PlyGaussians(NamedTuple):
    """What load_ply puts on the model (gaussian_model.py:554-560): float32
    tensors xyz (P,3), features_dc (P,1,3), features_rest (P,K,3), opacity
    (P,1), scaling (P,S), rotation (P,R); lod_level int8 (P,) or None;
    active_sh_degree = max_sh_degree."""
    xyz: torch.Tensor
    features_dc: torch.Tensor
    features_rest: torch.Tensor
    opacity: torch.Tensor
    scaling: torch.Tensor
    rotation: torch.Tensor
    lod_level: Optional[torch.Tensor]
    active_sh_degree: int


class PlyHeader(NamedTuple):
    format: str                 # ascii | binary_little_endian | binary_big_endian
    elements: list              # [(name, count, [(property, numpy type code or None for a list)])]
    body_offset: int            # byte offset of the first element's data


def construct_list_of_attributes(features_dc, features_rest, scaling, rotation):
    """gaussian_model.py:434-446."""
    names = ["x", "y", "z", "nx", "ny", "nz"]
    names += ["f_dc_{}".format(i) for i in range(features_dc.shape[1] * features_dc.shape[2])]
    names += ["f_rest_{}".format(i) for i in range(features_rest.shape[1] * features_rest.shape[2])]
    names.append("opacity")
    names += ["scale_{}".format(i) for i in range(scaling.shape[1])]
    names += ["rot_{}".format(i) for i in range(rotation.shape[1])]
    return names


def ply_header(names, count):
    """Header as plyfile writes one float32 'vertex' element in native (little-endian) order."""
    lines = ["ply", "format binary_little_endian 1.0", "element vertex {}".format(count)]
    lines += ["property float {}".format(n) for n in names]
    lines.append("end_header")
    return ("\n".join(lines) + "\n").encode("ascii")


def read_ply_header(path_or_file):
    """Parse a PLY header (PLY 1.0 grammar: format, comment, obj_info, element, property lines)."""
    fh = open(path_or_file, "rb") if isinstance(path_or_file, (str, os.PathLike)) else path_or_file
    try:
        if fh.readline().rstrip(b"\r\n") != b"ply":
            raise ValueError("not a PLY file (missing 'ply' magic line)")
        fmt, elements = None, []
        while True:
            line = fh.readline()
            if not line:
                raise ValueError("PLY header is not terminated by end_header")
            tok = line.decode("ascii").split()
            if not tok or tok[0] in ("comment", "obj_info"):
                continue
            if tok[0] == "format":
                if len(tok) != 3 or tok[2] != "1.0":
                    raise ValueError("unsupported PLY format line: {}".format(line))
                fmt = tok[1]
            elif tok[0] == "element":
                elements.append((tok[1], int(tok[2]), []))
            elif tok[0] == "property":
                if not elements:
                    raise ValueError("PLY property before any element")
                if tok[1] == "list":
                    elements[-1][2].append((tok[4], None))
                else:
                    if tok[1] not in PLY_TYPES:
                        raise ValueError("unknown PLY property type {}".format(tok[1]))
                    elements[-1][2].append((tok[2], PLY_TYPES[tok[1]]))
            elif tok[0] == "end_header":
                break
            else:
                raise ValueError("unexpected PLY header line: {}".format(line))
        if fmt not in ("ascii", "binary_little_endian", "binary_big_endian"):
            raise ValueError("unknown PLY format {}".format(fmt))
        if not elements:
            raise ValueError("PLY file has no element")
        return PlyHeader(fmt, elements, fh.tell())
    finally:
        if fh is not path_or_file:
            fh.close()


# ------------------------------------------------------------------ kernels

def _device_of(*ts):
    for t in ts:
        if t is not None and t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("blitzgs_amd.plyio: no HIP device")
    return torch.device("cuda", torch.cuda.current_device())


def _specs(tensors):
    arr = (_lib.PlyTensor * len(tensors))()
    for i, (t, w) in enumerate(tensors):
        arr[i].ptr = t.data_ptr()
        arr[i].width = w
        arr[i].type = 1 if t.dtype == torch.int8 else 0
    return arr


def pack_records(xyz, features_dc, features_rest, opacity, scaling, rotation, lod_level=None):
    """gs_ply_pack: the (P, n) float32 vertex records of save_ply on the GPU, and their names."""
    dev = _device_of(xyz)
    P = xyz.shape[0]
    K1, C1 = features_dc.shape[1], features_dc.shape[2]
    K, C = features_rest.shape[1], features_rest.shape[2]
    S, R = scaling.shape[1], rotation.shape[1]
    names = construct_list_of_attributes(features_dc, features_rest, scaling, rotation)
    if lod_level is not None:
        names = names + ["lod_level"]
    n = len(names)
    if n > _MAX_COLS:
        raise ValueError("{} PLY properties exceed the kernel's {} columns".format(n, _MAX_COLS))
    prep = lambda t: t.detach().to(dev, torch.float32).contiguous()
    tensors, colmap = [], []
    base_dc = 6
    base_rest = base_dc + K1 * C1
    base_op = base_rest + K * C
    tensors.append((prep(xyz), 3))
    colmap += [0, 1, 2]
    if K1 * C1:
        tensors.append((prep(features_dc), K1 * C1))
        colmap += [base_dc + c * K1 + k for k in range(K1) for c in range(C1)]   # (P,K,C) -> transpose(1,2)
    if K * C:
        tensors.append((prep(features_rest), K * C))
        colmap += [base_rest + c * K + k for k in range(K) for c in range(C)]
    tensors.append((prep(opacity), 1))
    colmap.append(base_op)
    if S:
        tensors.append((prep(scaling), S))
        colmap += [base_op + 1 + i for i in range(S)]
    if R:
        tensors.append((prep(rotation), R))
        colmap += [base_op + 1 + S + i for i in range(R)]
    if lod_level is not None:
        tensors.append((lod_level.detach().to(dev, torch.int8).reshape(P).contiguous(), 1))
        colmap.append(n - 1)
    for t, w in tensors:
        if t.shape[0] != P or t.numel() != P * w:
            raise ValueError("PLY field of shape {} does not hold {} rows of {} values".format(tuple(t.shape), P, w))
    rec = torch.empty((P, n), dtype=torch.float32, device=dev)
    cm = np.ctypeslib.as_ctypes(np.asarray(colmap, dtype=np.int32))
    with torch.cuda.device(dev):
        _lib.check(_lib.load().gs_ply_pack(P, len(tensors), _specs(tensors), cm, n, _lib.ptr(rec),
                                           _lib.stream_of(dev)), "gs_ply_pack")
    return rec, names


def unpack_records(rec, colmap_by_tensor, shapes, lod=False):
    """gs_ply_unpack of (P, n) float32 records: tensor i takes record columns
    colmap_by_tensor[i] (row-major over its shape[1:]); the last tensor is int8 if lod."""
    P = rec.shape[0]
    dev = rec.device
    outs = []
    for i, shp in enumerate(shapes):
        dt = torch.int8 if (lod and i == len(shapes) - 1) else torch.float32
        outs.append(torch.empty((P,) + tuple(shp), dtype=dt, device=dev))
    tensors, colmap = [], []
    for t, cols in zip(outs, colmap_by_tensor):
        if len(cols):
            tensors.append((t, len(cols)))
            colmap += list(cols)
    if P and tensors:
        cm = np.ctypeslib.as_ctypes(np.asarray(colmap, dtype=np.int32))
        with torch.cuda.device(dev):
            _lib.check(_lib.load().gs_ply_unpack(P, _lib.ptr(rec), rec.shape[1], len(tensors), _specs(tensors), cm,
                                                 _lib.stream_of(dev)), "gs_ply_unpack")
    return outs


# ------------------------------------------------------------------ save / load

def save_ply(path, xyz, features_dc, features_rest, opacity, scaling, rotation, lod_level=None):
    """gaussian_model.py:447-520 (the single-process branch: the file holds the
    tensors given).  Tensors may live on any device; the records are built on
    the GPU."""
    rec, names = pack_records(xyz, features_dc, features_rest, opacity, scaling, rotation, lod_level)
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    P, n = rec.shape
    row_bytes = 4 * n
    rpc = max(1, _CHUNK_BYTES // row_bytes)
    flat = rec.view(-1)
    bufs = [torch.empty(min(rpc, max(P, 1)) * n, dtype=torch.float32, pin_memory=True) for _ in range(2)]
    pending = []
    with open(path, "wb") as fh:
        fh.write(ply_header(names, P))
        for i, r0 in enumerate(range(0, P, rpc)):
            nr = min(rpc, P - r0)
            b = bufs[i % 2]
            b[:nr * n].copy_(flat[r0 * n:(r0 + nr) * n], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            pending.append((ev, b, nr))
            if len(pending) == 2:
                e0, b0, n0 = pending.pop(0)
                e0.synchronize()
                fh.write(memoryview(b0.numpy()[:n0 * n]))
        for e0, b0, n0 in pending:
            e0.synchronize()
            fh.write(memoryview(b0.numpy()[:n0 * n]))
    return names


def _sorted_names(names, prefix):
    """gaussian_model.py:532-552: properties with the prefix, by trailing integer."""
    return sorted([n for n in names if n.startswith(prefix)], key=lambda x: int(x.split("_")[-1]))


def _read_records_fast(fh, hdr, P, n, dev):
    """float32 little-endian records straight from the file to HBM (chunked, double-buffered)."""
    rec = torch.empty((P, n), dtype=torch.float32, device=dev)
    flat = rec.view(-1)
    row_bytes = 4 * n
    rpc = max(1, _CHUNK_BYTES // row_bytes)
    bufs = [torch.empty(min(rpc, max(P, 1)) * n, dtype=torch.float32, pin_memory=True) for _ in range(2)]
    evs = [None, None]
    fh.seek(hdr.body_offset)
    for i, r0 in enumerate(range(0, P, rpc)):
        nr = min(rpc, P - r0)
        k = i % 2
        if evs[k] is not None:
            evs[k].synchronize()
        view = bufs[k].numpy()[:nr * n].view(np.uint8)
        got = fh.readinto(memoryview(view))
        if got != nr * row_bytes:
            raise ValueError("PLY file is truncated: vertex data ends after {} of {} records".format(
                r0 + got // row_bytes, P))
        flat[r0 * n:(r0 + nr) * n].copy_(bufs[k][:nr * n], non_blocking=True)
        evs[k] = torch.cuda.Event()
        evs[k].record()
    for e in evs:
        if e is not None:
            e.synchronize()
    return rec


def _read_vertex_host(fh, hdr):
    """The first element as a numpy structured array (any format; scalar properties)."""
    name, count, props = hdr.elements[0]
    if any(t is None for _, t in props):
        raise ValueError("list properties in the PLY '{}' element are not supported".format(name))
    fh.seek(hdr.body_offset)
    if hdr.format == "ascii":
        dt = np.dtype([(p, t) for p, t in props])
        out = np.empty(count, dtype=dt)
        for i in range(count):
            tok = fh.readline().split()
            if len(tok) < len(props):
                raise ValueError("PLY ascii vertex {} has {} values, expected {}".format(i, len(tok), len(props)))
            for (p, t), v in zip(props, tok):
                out[p][i] = np.float64(v.decode()).astype(t) if t[0] == "f" else int(v)
        return out
    bo = "<" if hdr.format == "binary_little_endian" else ">"
    dt = np.dtype([(p, bo + t) for p, t in props])
    buf = fh.read(count * dt.itemsize)
    if len(buf) != count * dt.itemsize:
        raise ValueError("PLY file is truncated")
    return np.frombuffer(buf, dtype=dt, count=count)


def load_ply(path, max_sh_degree, device=None, with_lod=True):
    """gaussian_model.py:522-575: read a trained scene; returns PlyGaussians."""
    hdr = read_ply_header(path)
    _, P, props = hdr.elements[0]
    names = [p for p, _ in props]
    index = {p: i for i, p in enumerate(names)}

    def col(p):
        if p not in index:
            raise ValueError("no field of name {}".format(p))
        return index[p]

    K = (max_sh_degree + 1) ** 2 - 1
    rest = _sorted_names(names, "f_rest_")
    if len(rest) != 3 * K:
        raise ValueError("cannot reshape {} f_rest properties into (3, {})".format(len(rest), K))
    scale = _sorted_names(names, "scale_")
    rot = _sorted_names(names, "rot")
    lod = with_lod and "lod_level" in index
    wanted = [[col("x"), col("y"), col("z")],
              [col("f_dc_{}".format(c)) for c in range(3)],
              [col(rest[c * K + k]) for k in range(K) for c in range(3)],   # (P,3,K) -> transpose(1,2)
              [col("opacity")],
              [col(s) for s in scale],
              [col(r) for r in rot]]
    shapes = [(3,), (1, 3), (K, 3), (1,), (len(scale),), (len(rot),)]
    if lod:
        wanted.append([col("lod_level")])
        shapes.append(())
    dev = torch.device(device) if device is not None else _device_of()
    fast = (hdr.format == "binary_little_endian" and all(t == "f4" for _, t in props)
            and len(names) <= _MAX_COLS)
    with open(path, "rb") as fh:
        if fast:
            rec = _read_records_fast(fh, hdr, P, len(names), dev)
            cm = wanted
        else:
            v = _read_vertex_host(fh, hdr)
            used = sorted({c for cols in wanted for c in cols})
            where = {c: j for j, c in enumerate(used)}
            host = np.empty((P, len(used)), dtype=np.float32)
            for j, c in enumerate(used):
                host[:, j] = np.asarray(v[names[c]]).astype(np.float64).astype(np.float32)
            if lod:   # the int8 cast reads the property's own value, not its float32 rounding
                host[:, where[col("lod_level")]] = np.asarray(v["lod_level"]).astype(np.int8)
            rec = torch.from_numpy(host).to(dev)
            cm = [[where[c] for c in cols] for cols in wanted]
    outs = unpack_records(rec, cm, shapes, lod=lod)
    return PlyGaussians(outs[0], outs[1], outs[2], outs[3], outs[4], outs[5], outs[6] if lod else None,
                        max_sh_degree)
