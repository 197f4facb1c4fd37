"""ctypes binding of libblitzgs_amd.so (the C ABI declared in include/blitzgs_amd.h).

The library is built in-tree by blitzgs_amd.build (or __graft_entry__.build()).
There is no fallback path: if the library or a HIP device is missing, every
operator raises.
"""
import ctypes as C
import os

from . import build as _build

_lib = None

_c = C.c_void_p
_i = C.c_int
_f = C.c_float
_i64 = C.c_int64
_sz = C.c_size_t


class RowField(C.Structure):
    """gs_row_field (include/blitzgs_amd.h)."""
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p), ("src_stride", C.c_int64), ("dst_stride", C.c_int64),
                ("width", C.c_int32), ("src_type", C.c_int32), ("dst_type", C.c_int32)]


class PlyTensor(C.Structure):
    """gs_ply_tensor (include/blitzgs_amd.h)."""
    _fields_ = [("ptr", C.c_void_p), ("width", C.c_int32), ("type", C.c_int32)]


class AdamGroup(C.Structure):
    """gs_adam_group (include/blitzgs_amd.h)."""
    _fields_ = [("param", C.c_void_p), ("grad", C.c_void_p), ("exp_avg", C.c_void_p), ("exp_avg_sq", C.c_void_p),
                ("M", C.c_int64), ("lr", C.c_float), ("eps", C.c_float)]


_SIGS = {
    "gs_version": (_i, []),
    "gs_last_error": (C.c_char_p, []),
    "gs_preprocess_forward": (_i, [_i, _i, _i, _c, _c, _c, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i,
                                   _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_preprocess_backward": (_i, [_i, _i, _i, _c, _c, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i,
                                    _c, _c, _c, _c, _i, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_preprocess_record_bytes": (_i64, [_i]),
    "gs_preprocess_forward_rec": (_i, [_i, _i, _i, _c, _c, _c, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i,
                                       _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_preprocess_backward_rec": (_i, [_i, _i, _i, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i,
                                        _c, _c, _i, _c, _c, _c, _c, _c, _c, _c, _i, _c]),
    "gs_preprocess_backward_rec_acc": (_i, [_i, _i, _i, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i,
                                            _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_render_accumulators": (_i, [_c, _i, _i, _i, _i64, C.POINTER(_c), C.POINTER(_c)]),
    "gs_render_geom_bytes": (_sz, [_i, _i, _i]),
    "gs_render_binning_bytes": (_sz, [_i64]),
    "gs_render_img_bytes": (_sz, [_i, _i]),
    "gs_render_forward_count": (_i, [_i, _i, _i, _c, _c, _c, _c, C.POINTER(_i64), _i, _c]),
    "gs_render_forward": (_i, [_i, _i64, _i, _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c,
                               _c, _i, _c, _i64, _c]),
    "gs_render_forward_reserved": (_i, [_i, _i64, _i, _i] + [_c] * 15 + [C.POINTER(_i64), _i, _c, _i64, _c]),
    "gs_render_backward": (_i, [_i, _i64, _i, _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _i, _c, _c, _c, _c,
                                _i64, _c]),
    "gs_render_geo_forward": (_i, [_i, _i64, _i, _i, _f, _f, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_render_forward_geo": (_i, [_i, _i64, _i, _i] + [_c] * 15 + [_f, _f, _c, _c, _c, _i, _c]),
    "gs_render_forward_reserved_geo": (_i, [_i, _i64, _i, _i] + [_c] * 15 + [C.POINTER(_i64), _f, _f, _c, _c,
                                                                             _c, _i, _c]),
    "gs_render_backward_geo": (_i, [_i, _i64, _i, _i, _c, _f, _f] + [_c] * 13 + [_i, _c, _c, _c, _c, _c, _i64,
                                                                               _c]),
    "gs_render_buffer_views": (_i, [_i64, _i, _i, _c, _c, C.POINTER(_c), C.POINTER(_c), C.POINTER(_c),
                                    C.POINTER(_c), C.POINTER(_c), C.POINTER(_c)]),
    "gs_render_point_list": (_i, [_i, _i64, _i, _i, _c, _c, _c, _c, _c]),
    "gs_knn_workspace_bytes": (_sz, [_i]),
    "gs_knn_meandist3": (_i, [_i, _c, _c, _c, _c]),
    "gs_knn_meandist3_noalloc": (_i, [_i, _c, _c, _c]),
    "gs_ssim_forward": (_i, [_i, _i, _i, _i, _f, _f, _c, _c, _c, _c, _c, _c, _c]),
    "gs_ssim_backward": (_i, [_i, _i, _i, _i, _f, _f, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_adam_update": (_i, [_c, _c, _c, _c, _c, _f, _f, _f, _f, _i64, _i64, _c]),
    "gs_adam_update_groups": (_i, [_i, C.POINTER(AdamGroup), _i64, _c, _f, _f, _c]),
    "gs_preprocess_forward_full": (_i, [_i, _i, _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _f, _c, _c, _c, _f, _f, _i,
                                        _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_render_full_count": (_i, [_i, _i, _i, _c, _c, _c, _c, _c, C.POINTER(_i64), _c]),
    "gs_render_full_forward": (_i, [_i, _i64, _i, _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_render_full_forward_reserved": (_i, [_i, _i64, _i, _i] + [_c] * 14 + [C.POINTER(_i64), _c]),
    "gs_render_full_depth": (_i, [_i, _i64, _i, _i] + [_c] * 21 + [_c]),
    "gs_render_full_backward": (_i, [_i, _i64, _i, _i, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_preprocess_backward_full": (_i, [_i, _i, _i, _c, _c, _c, _c, _c, _c, _c, _f, _c, _c, _c, _f, _f, _i, _i, _c,
                                         _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c, _c]),
    "gs_mark_visible": (_i, [_i, _c, _c, _c, _c, _c]),
    "gs_local2j_ids_bool": (_i, [_i, _i, _i, _i, _i, _c, _c, _c, _i, _c, _c]),
    "gs_local2j_workspace_bytes": (_sz, [_i, _i]),
    "gs_local2j_count": (_i, [_i, _i, _i, _i, _i, _c, _c, _c, _i, _c, _c, _c, _c]),
    "gs_local2j_write": (_i, [_i, _i, _i, _i, _i, _c, _c, _c, _i, _c, _c, _i64, _c]),
    "gs_move_rows": (_i, [_i64, _c, _i64, _c, _i64, _i, C.POINTER(RowField), _i, _c]),
    "gs_ply_unpack": (_i, [_i64, _c, C.c_int32, C.c_int32, C.POINTER(PlyTensor), C.POINTER(C.c_int32), _c]),
    "gs_ply_pack": (_i, [_i64, C.c_int32, C.POINTER(PlyTensor), C.POINTER(C.c_int32), C.c_int32, _c, _c]),
    "gs_diag_math": (_i, [_i, _i, _c, _c, _c]),
    "gs_timing_enable": (_i, [_i]),
    "gs_timing_reset": (_i, []),
    "gs_timing_read": (_i, [_i, C.c_char_p, C.POINTER(C.c_double), C.POINTER(_i)]),
}


def lib_path():
    """The in-tree library, or the file named by BLITZGS_AMD_LIB (another build
    of the same sources, e.g. for side-by-side benchmarking)."""
    return os.environ.get("BLITZGS_AMD_LIB") or _build.LIB


def load():
    """Load (once) and return the ctypes library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(f"blitzgs_amd: {path} is not built; run blitzgs_amd.build.build() "
                           "(or __graft_entry__.build()) first")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return list(_SIGS)


def check(rc, what):
    if rc != 0:
        msg = load().gs_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def debug_sync(debug, what):
    """The reference's debug mode (CHECK_CUDA, _f/cuda_rasterizer/auxiliary.h:186-193):
    wait for the device after a call and raise RuntimeError if it failed."""
    if not debug:
        return
    import torch
    try:
        torch.cuda.synchronize()
    except RuntimeError as e:
        raise RuntimeError(f"{what}: {e}") from e


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def stream_of(device=None):
    import torch
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def timing_enable(on=True, stages_only=False):
    """on: time every kernel launch and the stages (stages_only: the stages
    alone, without per-kernel events in the way); off: nothing."""
    rc = load().gs_timing_enable((2 if stages_only else 1) if on else 0)
    if rc != 0:
        raise RuntimeError(f"gs_timing_enable failed ({rc})")


def timing_reset():
    load().gs_timing_reset()


def timing_read(max_entries=64):
    """{kernel name: (total_ms, launches)} accumulated since the last reset."""
    names = C.create_string_buffer(64 * max_entries)
    tot = (C.c_double * max_entries)()
    cnt = (C.c_int * max_entries)()
    n = load().gs_timing_read(max_entries, names, tot, cnt)
    out = {}
    for i in range(min(n, max_entries)):
        nm = names.raw[64 * i:64 * i + 64].split(b"\0", 1)[0].decode()
        out[nm] = (tot[i], cnt[i])
    return out


class InstanceReserve:
    """Per-device estimate of the next forward's instance count R: a slowly
    decaying maximum of the recent counts.  The reserved capacity (10 % above
    it) sizes the binning buffer before R is known, so that the forward is one
    library call with no host round trip between the count and the
    duplication; a forward with more instances is redone at the exact size."""

    HEADROOM = 1.10
    DECAY = 0.98
    MIN_CAPACITY = 4096

    def __init__(self):
        self._est = {}
        self._per_gaussian = {}

    def capacity(self, dev):
        e = self._est.get(dev)
        return None if e is None else min(int(e * self.HEADROOM) + self.MIN_CAPACITY, 2 ** 32 - 1)

    def update(self, dev, R, P=None):
        self._est[dev] = max(int(R), int(self._est.get(dev, 0) * self.DECAY))
        if P:
            self._per_gaussian[dev] = R / P

    # Region side of the split path's binning: 4x4-tile regions when the last
    # forward on the device had this many or more tile instances per Gaussian
    # (large Gaussians: fewer region entries, lists still short enough to
    # sort on chip), else the default.  The choice never changes a result.
    REGION4_MIN_INSTANCES = 12.0

    def region_side(self, dev):
        r = self._per_gaussian.get(dev)
        return 4 if r is not None and r >= self.REGION4_MIN_INSTANCES else 0

    def reset(self):
        self._est.clear()
        self._per_gaussian.clear()


RESERVE = InstanceReserve()
