"""Gaussian -> rank routing and the screen-space row exchange of the
image-distributed training step.

Mirrors BlitzGS:
  diff-gaussian-rasterization_f/rasterize_points.cu:212-367
      _C.get_local2j_ids_bool / _C.get_local2j_ids_bool_adjust_mode6
  gaussian_renderer/workload_division.py:145-167, 430-468, 682-704
      DivisionStrategy*.get_local2j_ids: the bool matrix, then one nonzero() per rank
  gaussian_renderer/__init__.py:22-189
      all_to_all_communication_final: per destination rank torch.cat(fields, 1)[ids]
      (pack), all_to_all, split + cat per camera, radii .float() -> .int() (unpack);
      autograd carries the gradients of the six differentiable fields back.

All device work runs in libblitzgs_amd.so (blitzgs_amd/csrc/route.hip):
gs_local2j_ids_bool (the bool matrix), gs_local2j_count / gs_local2j_write
(every rank's id list from one counting and one writing pass, one host read of
the counts instead of one per rank) and gs_move_rows (pack, unpack and the
gradient scatter, one launch each).

Only the single-process exchange is built: with one rank the all-to-all hands
each camera's packed rows back to the same process, so pack and unpack fuse
into one gather per camera.  A process group of more than one rank raises.
"""
import torch

from . import _lib

INTERVAL = 0   # GS_ROUTE_INTERVAL: table = world + 1 tile indices
RECT = 1       # GS_ROUTE_RECT: table = world rows of (y_l, y_r, x_l, x_r)


def _dev(t, name, dtype):
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise RuntimeError(f"{name} must be a HIP device tensor")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")
    return t.contiguous()


def _table(table, device):
    if not isinstance(table, torch.Tensor):
        table = torch.tensor(table, dtype=torch.int32)
    return table.to(device=device, dtype=torch.int32).contiguous()


def _inputs(means2D, radii, table):
    m2d = _dev(means2D, "means2D", torch.float32)
    if m2d.dim() != 2 or m2d.size(1) != 2:
        raise RuntimeError(f"means2D must be (P, 2), got {tuple(m2d.shape)}")
    r = _dev(radii, "radii", torch.int32).reshape(-1)
    if r.numel() != m2d.size(0):
        raise RuntimeError("radii must have one entry per Gaussian")
    return m2d, r, _table(table, m2d.device)


def _avoid(args):
    return bool(args["avoid_pixel_all2all"]) if args is not None else False


def _bool_matrix(mode, H, W, world, means2D, radii, table, avoid):
    m2d, r, tab = _inputs(means2D, radii, table)
    P = m2d.size(0)
    need = world + 1 if mode == INTERVAL else 4 * world
    if tab.numel() < need:
        raise RuntimeError(f"routing table has {tab.numel()} entries, {need} needed")
    out = torch.empty((P, world), dtype=torch.bool, device=m2d.device)
    _lib.check(_lib.load().gs_local2j_ids_bool(mode, P, int(H), int(W), int(world), _lib.ptr(m2d), _lib.ptr(r),
                                               _lib.ptr(tab), int(avoid), _lib.ptr(out), _lib.stream_of(m2d.device)),
               "gs_local2j_ids_bool")
    return out


def get_local2j_ids_bool(image_height, image_width, mp_rank, mp_world_size, means2D, radii, dist_global_strategy,
                         args=None):
    """The reference's _C.get_local2j_ids_bool (rasterize_points.cu:258-289):
    (P, mp_world_size) bool, rank rk gets Gaussian i when the row-major tile
    span of its rect meets [strategy[rk], strategy[rk+1])."""
    return _bool_matrix(INTERVAL, image_height, image_width, mp_world_size, means2D, radii, dist_global_strategy,
                        _avoid(args))


def get_local2j_ids_bool_adjust_mode6(image_height, image_width, mp_rank, mp_world_size, means2D, radii, rectangles,
                                      args=None):
    """The reference's _C.get_local2j_ids_bool_adjust_mode6
    (rasterize_points.cu:337-367): rank rk owns the tile rectangle
    rectangles[rk] = (y_l, y_r, x_l, x_r)."""
    return _bool_matrix(RECT, image_height, image_width, mp_world_size, means2D, radii, rectangles, _avoid(args))


def local2j_ids(means2D, radii, image_height, image_width, table, world_size, mode=INTERVAL,
                avoid_pixel_all2all=False, want_bool=False):
    """Every rank's send ids at once: returns (list of int64 id tensors, one per
    rank, ascending -- what local2j_ids_bool[:, rk].nonzero() gives -- and the
    bool matrix or None).  One host read of the counts in all."""
    ids, cnt, out_bool = local2j_ids_concat(means2D, radii, image_height, image_width, table, world_size, mode,
                                            avoid_pixel_all2all, want_bool)
    return list(torch.split(ids, cnt)), out_bool


def local2j_ids_concat(means2D, radii, image_height, image_width, table, world_size, mode=INTERVAL,
                       avoid_pixel_all2all=False, want_bool=False):
    """As local2j_ids, with the id lists left concatenated rank after rank:
    returns (int64 ids, per-rank counts as a list of ints, bool matrix or None)."""
    m2d, r, tab = _inputs(means2D, radii, table)
    P, world = m2d.size(0), int(world_size)
    need = world + 1 if mode == INTERVAL else 4 * world
    if tab.numel() < need:
        raise RuntimeError(f"routing table has {tab.numel()} entries, {need} needed")
    dev = m2d.device
    lib = _lib.load()
    ws = torch.empty(max(int(lib.gs_local2j_workspace_bytes(P, world)), 4), dtype=torch.uint8, device=dev)
    counts = torch.empty(world + 1, dtype=torch.int64, device=dev)
    out_bool = torch.empty((P, world), dtype=torch.bool, device=dev) if want_bool else None
    s = _lib.stream_of(dev)
    args = (mode, P, int(image_height), int(image_width), world, _lib.ptr(m2d), _lib.ptr(r), _lib.ptr(tab),
            int(bool(avoid_pixel_all2all)))
    _lib.check(lib.gs_local2j_count(*args, _lib.ptr(out_bool), _lib.ptr(counts), _lib.ptr(ws), s), "gs_local2j_count")
    cnt = counts.cpu().tolist()
    ids = torch.empty(cnt[world], dtype=torch.int64, device=dev)
    _lib.check(lib.gs_local2j_write(*args, _lib.ptr(ws), _lib.ptr(ids), cnt[world], s), "gs_local2j_write")
    return ids, cnt[:world], out_bool


# ---------------------------------------------------------------- row mover

def _rows2d(t):
    """(P, w) view of a field whose elements are contiguous within a row."""
    if t.dim() == 1:
        t = t.unsqueeze(1)
    elif t.dim() > 2:
        t = t.reshape(t.size(0), -1)
    if t.stride(1) != 1 and t.size(1) > 1:
        t = t.contiguous()
    return t


_TYPES = {torch.float32: 0, torch.int32: 1}


def _field(src, dst):
    if src.dtype not in _TYPES or dst.dtype not in _TYPES:
        raise RuntimeError(f"row fields must be float32 or int32, got {src.dtype} -> {dst.dtype}")
    if src.size(1) != dst.size(1):
        raise RuntimeError("source and destination widths differ")
    return _lib.RowField(src=src.data_ptr(), dst=dst.data_ptr(), src_stride=src.stride(0), dst_stride=dst.stride(0),
                         width=src.size(1), src_type=_TYPES[src.dtype], dst_type=_TYPES[dst.dtype])


def move_rows(n_rows, pairs, src_rows=None, dst_rows=None, accumulate=False):
    """One gs_move_rows launch: row r of every (src, dst) pair moves from
    source row src_rows[r] (or r) to destination row dst_rows[r] (or r).
    Map entries outside the sources' / destinations' rows read as zero / are
    skipped (all sources, and all destinations, must have the same rows)."""
    if not pairs:
        return
    dev = pairs[0][1].device
    for s, d in pairs:
        if not (s.is_cuda and d.is_cuda):
            raise RuntimeError("row fields must be HIP device tensors")
    n_src = {s.size(0) for s, _ in pairs}
    n_dst = {d.size(0) for _, d in pairs}
    if len(n_src) != 1 or len(n_dst) != 1:
        raise RuntimeError("row fields of one move must have the same number of rows on each side")
    maps = []
    for m in (src_rows, dst_rows):
        if m is not None:
            m = _dev(m, "row map", torch.int64).reshape(-1)
            if m.numel() < n_rows:
                raise RuntimeError("row map shorter than n_rows")
        maps.append(m)
    fields = (_lib.RowField * len(pairs))(*[_field(s, d) for s, d in pairs])
    _lib.check(_lib.load().gs_move_rows(int(n_rows), _lib.ptr(maps[0]), n_src.pop(), _lib.ptr(maps[1]), n_dst.pop(),
                                        len(pairs), fields, int(bool(accumulate)), _lib.stream_of(dev)),
               "gs_move_rows")


def pack_rows(ids, tensors):
    """torch.cat([t.reshape(P, -1).float() for t in tensors], 1)[ids] in one
    launch (the send buffer of one destination rank)."""
    srcs = [_rows2d(t) for t in tensors]
    width = sum(s.size(1) for s in srcs)
    n = int(ids.numel())
    out = torch.empty((n, width), dtype=torch.float32, device=srcs[0].device)
    pairs, c = [], 0
    for s in srcs:
        pairs.append((s, out[:, c:c + s.size(1)]))
        c += s.size(1)
    move_rows(n, pairs, src_rows=ids)
    return out


def unpack_rows(buf, widths, dtypes):
    """Split received rows into contiguous per-field tensors (torch.split +
    .contiguous(), with .int() for int32 fields), one launch."""
    n = buf.size(0)
    outs, pairs, c = [], [], 0
    for w, dt in zip(widths, dtypes):
        o = torch.empty((n, w), dtype=dt, device=buf.device)
        pairs.append((buf[:, c:c + w], o))
        outs.append(o)
        c += w
    if c != buf.size(1):
        raise RuntimeError("field widths do not add up to the row width")
    move_rows(n, pairs)
    return outs


def scatter_rows(ids, rows, P, out=None, accumulate=False):
    """Backward of a gather: zero-filled (P, w) tensors with rows[r] at ids[r]
    (index_put_ of the reference's autograd), or added into `out`."""
    rows = [_rows2d(g) for g in rows]
    if out is None:
        out = [torch.zeros((P, g.size(1)), dtype=g.dtype, device=g.device) for g in rows]
    move_rows(int(ids.numel()), list(zip(rows, out)), dst_rows=ids, accumulate=accumulate)
    return out


class _LocalExchange(torch.autograd.Function):
    """One camera's screen-space exchange when this process is the only rank:
    gathers rows ids of the eight fields into contiguous tensors; the backward
    scatters the gradients of the six differentiable fields to the source rows
    (zeros elsewhere)."""

    @staticmethod
    def forward(ctx, ids, means2D, rgb, conic_opacity, radii, depths, means3D, scales, rotation):
        srcs = [_rows2d(t) for t in (means2D, rgb, conic_opacity, radii, depths, means3D, scales, rotation)]
        n = int(ids.numel())
        outs = [torch.empty((n, s.size(1)), dtype=s.dtype, device=s.device) for s in srcs]
        move_rows(n, list(zip(srcs, outs)), src_rows=ids)
        ctx.save_for_backward(ids)
        ctx.P = means2D.size(0)
        ctx.shapes = [tuple(t.shape[1:]) for t in (means2D, rgb, conic_opacity, means3D, scales, rotation)]
        radii_o, depths_o = outs[3].reshape(n), outs[4].reshape(n)
        ctx.mark_non_differentiable(radii_o, depths_o)
        o = [outs[0], outs[1], outs[2], outs[5], outs[6], outs[7]]
        return (o[0], o[1], o[2], radii_o, depths_o, o[3], o[4], o[5])

    @staticmethod
    def backward(ctx, g_m2d, g_rgb, g_con, g_radii, g_depths, g_m3d, g_sc, g_rot):
        (ids,) = ctx.saved_tensors
        grads = [g_m2d, g_rgb, g_con, g_m3d, g_sc, g_rot]
        live = [k for k, g in enumerate(grads) if g is not None]
        res = [None] * 6
        if live:
            outs = scatter_rows(ids, [grads[k].float() for k in live], ctx.P)
            for k, o in zip(live, outs):
                res[k] = o.reshape((ctx.P,) + ctx.shapes[k])
        return (None, res[0], res[1], res[2], None, None, res[3], res[4], res[5])


def _single_process():
    d = torch.distributed
    if d.is_available() and d.is_initialized() and d.get_world_size() > 1:
        raise NotImplementedError("the screen-space all-to-all between GPUs is not part of this build; "
                                  "all_to_all_communication_final runs with one process only")


def all_to_all_communication_final(batched_rasterizers, batched_screenspace_params, batched_cuda_args,
                                   batched_strategies):
    """Single-process counterpart of gaussian_renderer/__init__.py:22-189: same
    arguments, same 10-tuple.  Each strategy's get_local2j_ids gives the send
    ids (rank 0's list is the whole exchange); each camera's fields are then
    gathered in one launch, and autograd returns their gradients to the
    source rows."""
    _single_process()
    outs = [[] for _ in range(8)]
    sizes, send_ids = [], []
    for k, rast in enumerate(batched_rasterizers):
        means2D, rgb, conic_opacity, radii, depths, means3D, scales, rotation = batched_screenspace_params[k]
        local2j_ids, _ = batched_strategies[k].get_local2j_ids(means2D, radii, rast.raster_settings,
                                                               batched_cuda_args[k])
        ids = local2j_ids[0] if len(local2j_ids) else torch.empty(0, dtype=torch.int64, device=means2D.device)
        if rgb.dim() > 2:
            rgb = rgb.contiguous().view(rgb.shape[0], -1)
        res = _LocalExchange.apply(ids, means2D, rgb, conic_opacity, radii.int(), depths.float(), means3D, scales,
                                   rotation)
        for j in range(8):
            outs[j].append(res[j])
        sizes.append(int(ids.numel()))
        send_ids.append(ids)
    gpui_to_gpuj_imgk_size = [[sizes]]
    local_to_gpuj_camk_send_ids = [send_ids]
    return (*outs, gpui_to_gpuj_imgk_size, local_to_gpuj_camk_send_ids)
