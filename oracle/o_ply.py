"""numpy restatement of the reference's PLY save / load (TEST INFRASTRUCTURE ONLY).

Only tests/ and bench.py's cpu_baseline leg use this module, as the checker
and the timed CPU baseline; the product (blitzgs_amd) never imports it.

The reference (BlitzGS scene/gaussian_model.py) writes and reads the trained
scene with the plyfile package, which is absent here (blitzgs_environment.yml:19
lists it without a version).  What the reference relies on from it is the PLY
1.0 file layout (Turk's format, as plyfile writes it):

  ply\n
  format binary_little_endian 1.0\n          (plyfile's native byte order)
  element vertex <P>\n
  property float <name>\n                    (one per attribute, 'f4' -> float)
  ...
  end_header\n
  <P records of the properties back to back, little-endian>

and, for reading, the general grammar: ascii / binary_little_endian /
binary_big_endian bodies, scalar property types char uchar short ushort int
uint float double (and their int8 ... float64 aliases), comment / obj_info
lines, further elements after the first.

Functions follow:
  attribute_names   gaussian_model.py:434-446  construct_list_of_attributes
  save_ply          gaussian_model.py:447-520  (single-rank branch; the gather
                                                to rank 0 is not part of the file)
  load_ply          gaussian_model.py:522-575
"""
import numpy as np

PLY_SCALARS = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}


def attribute_names(dc_shape, rest_shape, n_scale, n_rot, lod=False):
    """gaussian_model.py:434-446 (+ the 'lod_level' column save_ply appends at :508-510).
    dc_shape / rest_shape are the (K, 3) trailing shapes of features_dc / features_rest."""
    names = ["x", "y", "z", "nx", "ny", "nz"]
    names += [f"f_dc_{i}" for i in range(dc_shape[0] * dc_shape[1])]
    names += [f"f_rest_{i}" for i in range(rest_shape[0] * rest_shape[1])]
    names.append("opacity")
    names += [f"scale_{i}" for i in range(n_scale)]
    names += [f"rot_{i}" for i in range(n_rot)]
    if lod:
        names.append("lod_level")
    return names


def header_bytes(names, count, fmt="binary_little_endian", types=None, comments=()):
    lines = ["ply", f"format {fmt} 1.0"]
    lines += [f"comment {c}" for c in comments]
    lines.append(f"element vertex {count}")
    for i, n in enumerate(names):
        lines.append(f"property {types[i] if types else 'float'} {n}")
    lines.append("end_header")
    return ("\n".join(lines) + "\n").encode("ascii")


def _sh_flat(f):
    """(P, K, 3) -> (P, 3*K) as .transpose(1, 2).flatten(start_dim=1) (gaussian_model.py:491-492)."""
    return np.ascontiguousarray(np.transpose(f, (0, 2, 1))).reshape(f.shape[0], f.shape[1] * f.shape[2])


def save_ply(path, xyz, f_dc, f_rest, opacity, scale, rot, lod=None):
    """gaussian_model.py:486-517: every attribute as float32 'f4' in one 'vertex' element."""
    P = xyz.shape[0]
    cols = [xyz, np.zeros_like(xyz), _sh_flat(f_dc), _sh_flat(f_rest), opacity, scale, rot]
    if lod is not None:
        cols.append(np.asarray(lod).astype(np.float32).reshape(-1, 1))
    rec = np.concatenate([np.asarray(c, dtype=np.float32).reshape(P, int(np.prod(np.shape(c)[1:]))) for c in cols],
                         axis=1)
    names = attribute_names(f_dc.shape[1:], f_rest.shape[1:], scale.shape[1], rot.shape[1], lod is not None)
    assert rec.shape[1] == len(names)
    with open(path, "wb") as fh:
        fh.write(header_bytes(names, P))
        fh.write(rec.astype("<f4").tobytes())
    return names


def read_header(fh):
    """Parse a PLY header; returns (format, elements, body offset) with elements a
    list of (name, count, [(prop, numpy type or None for a list property)])."""
    magic = fh.readline()
    if magic.rstrip(b"\r\n") != b"ply":
        raise ValueError("not a PLY file")
    fmt, elements = None, []
    while True:
        line = fh.readline()
        if not line:
            raise ValueError("PLY header has no end_header")
        tok = line.decode("ascii").split()
        if not tok:
            continue
        if tok[0] == "format":
            fmt = tok[1]
        elif tok[0] == "element":
            elements.append((tok[1], int(tok[2]), []))
        elif tok[0] == "property":
            if tok[1] == "list":
                elements[-1][2].append((tok[4], None))
            else:
                elements[-1][2].append((tok[2], PLY_SCALARS[tok[1]]))
        elif tok[0] == "end_header":
            break
    if fmt not in ("ascii", "binary_little_endian", "binary_big_endian"):
        raise ValueError(f"unknown PLY format {fmt}")
    return fmt, elements, fh.tell()


def read_vertex(path):
    """The first element of a PLY file as a numpy structured array."""
    with open(path, "rb") as fh:
        fmt, elements, off = read_header(fh)
        name, count, props = elements[0]
        if any(t is None for _, t in props):
            raise ValueError("list properties in the first element are not supported")
        if fmt == "ascii":
            dt = np.dtype([(n, t) for n, t in props])
            out = np.empty(count, dtype=dt)
            for i in range(count):
                vals = fh.readline().split()
                out[i] = tuple(np.array(v.decode(), dtype=np.float64).astype(t) if t[0] == "f" else int(v)
                               for v, (_, t) in zip(vals, props))
            return out
        bo = "<" if fmt == "binary_little_endian" else ">"
        dt = np.dtype([(n, bo + t) for n, t in props])
        data = np.frombuffer(fh.read(count * dt.itemsize), dtype=dt, count=count)
        return data


def _sorted_names(props, prefix):
    """gaussian_model.py:532-552: names with the prefix, sorted by their trailing integer."""
    return sorted([n for n in props if n.startswith(prefix)], key=lambda x: int(x.split("_")[-1]))


def load_ply(path, max_sh_degree):
    """gaussian_model.py:522-575 up to the tensors: float64 staging arrays, then float32.
    Returns xyz (P,3), features_dc (P,1,3), features_rest (P,K,3), opacity (P,1),
    scaling (P,S), rotation (P,R) float32 and lod_level int8 (P,) or None."""
    v = read_vertex(path)
    props = list(v.dtype.names)
    P = v.shape[0]
    xyz = np.stack((np.asarray(v["x"]), np.asarray(v["y"]), np.asarray(v["z"])), axis=1)
    opac = np.asarray(v["opacity"])[..., np.newaxis]
    dc = np.zeros((P, 3, 1))
    for c in range(3):
        dc[:, c, 0] = np.asarray(v[f"f_dc_{c}"])
    rest_names = _sorted_names(props, "f_rest_")
    rest = np.zeros((P, len(rest_names)))
    for i, n in enumerate(rest_names):
        rest[:, i] = np.asarray(v[n])
    rest = rest.reshape((P, 3, (max_sh_degree + 1) ** 2 - 1))
    scale_names = _sorted_names(props, "scale_")
    scales = np.zeros((P, len(scale_names)))
    for i, n in enumerate(scale_names):
        scales[:, i] = np.asarray(v[n])
    rot_names = _sorted_names(props, "rot")
    rots = np.zeros((P, len(rot_names)))
    for i, n in enumerate(rot_names):
        rots[:, i] = np.asarray(v[n])
    f32 = lambda a: np.ascontiguousarray(np.asarray(a, dtype=np.float64).astype(np.float32))
    lod = np.asarray(v["lod_level"]).astype(np.int8) if "lod_level" in props else None
    return {"xyz": f32(xyz), "features_dc": f32(np.transpose(dc, (0, 2, 1))),
            "features_rest": f32(np.transpose(rest, (0, 2, 1))), "opacity": f32(opac), "scaling": f32(scales),
            "rotation": f32(rots), "lod_level": lod}
