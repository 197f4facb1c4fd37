"""Training checkpoints in the reference's tuple format and file naming.

Mirrors BlitzGS:
  scene/gaussian_model.py:94-136  capture / restore: the model tuple
      (active_sh_degree, _xyz, _features_dc, _features_rest, _scaling,
       _rotation, _opacity, max_radii2D, xyz_gradient_accum, denom,
       optimizer.state_dict(), spatial_lr_scale, _lod_level, octree_state)
      restore accepts the 12-entry form too (the two LOD entries optional)
  train_internal.py:481-493  one file per rank,
      <folder>/chkpnt_ws=<world size>_rk=<global rank>.pth holding
      (model tuple, iteration to resume from)
  utils/general_utils.py:547-736  load_checkpoint on a possibly different
      world size: the same number of files -> this rank's file; more files
      (a multiple) -> this rank merges files rank, rank+N, ... by
      concatenating the per-Gaussian tensors (merge_multiple_checkpoints);
      fewer files (a divisor) -> this rank takes part rank // n_files of
      file rank % n_files, parts of N // n_files + 1 rows
      (get_part_of_checkpoints); then optional drop_duplicate_gaussians
      (rows 0 .. floor(P * coeff) - 1 taken modulo P).  Merged and split
      tuples carry opt_dict None and 12 entries, as the reference's do.

Files are read with torch.load(weights_only=True): the tuple holds only
tensors, Parameters, numbers, None and the optimizer's state dict, all of
which the restricted unpickler accepts.
"""
import os

import torch
import torch.nn as nn

CHECKPOINT_NAME = "chkpnt_ws={}_rk={}.pth"


def capture(active_sh_degree, xyz, features_dc, features_rest, scaling, rotation, opacity, max_radii2D,
            xyz_gradient_accum, denom, optimizer_state, spatial_lr_scale, lod_level=None, octree_state=None):
    """gaussian_model.py:94-111: the 14-entry model tuple."""
    return (active_sh_degree, xyz, features_dc, features_rest, scaling, rotation, opacity, max_radii2D,
            xyz_gradient_accum, denom, optimizer_state, spatial_lr_scale, lod_level, octree_state)


def restore(model_args):
    """gaussian_model.py:113-136 without the optimizer set-up: the tuple's
    entries by name; lod_level / octree_state are None when absent."""
    (active_sh_degree, xyz, features_dc, features_rest, scaling, rotation, opacity, max_radii2D,
     xyz_gradient_accum, denom, opt_dict, spatial_lr_scale, *optional) = model_args
    out = dict(active_sh_degree=active_sh_degree, xyz=xyz, features_dc=features_dc, features_rest=features_rest,
               scaling=scaling, rotation=rotation, opacity=opacity, max_radii2D=max_radii2D,
               xyz_gradient_accum=xyz_gradient_accum, denom=denom, opt_dict=opt_dict,
               spatial_lr_scale=spatial_lr_scale, lod_level=None, octree_state=None)
    if len(optional) >= 2 and optional[1] is not None:
        out["lod_level"], out["octree_state"] = optional[0], optional[1]
    elif len(optional) >= 1 and optional[0] is not None:
        out["lod_level"] = optional[0]
    return out


def checkpoint_path(folder, world_size, rank):
    return os.path.join(folder, CHECKPOINT_NAME.format(world_size, rank))


def save_checkpoint(folder, model_params, iteration, world_size=1, rank=0):
    """train_internal.py:481-493: torch.save((model tuple, iteration), chkpnt_ws=N_rk=i.pth)."""
    os.makedirs(folder, exist_ok=True)
    path = checkpoint_path(folder, world_size, rank)
    torch.save((model_params, iteration), path)
    return path


def _load(path, map_location):
    return torch.load(path, map_location=map_location, weights_only=True)


def _param(t):
    return nn.Parameter(t.requires_grad_(True))


def _tuple12(active_sh_degree, per_gaussian, spatial_lr_scale):
    xyz, fdc, frest, sc, rot, op, mr, acc, den = per_gaussian
    return (active_sh_degree, _param(xyz), _param(fdc), _param(frest), _param(sc), _param(rot), _param(op),
            mr, acc, den, None, spatial_lr_scale)


def merge_multiple_checkpoints(checkpoint_files, map_location=None):
    """general_utils.py:547-595: concatenate the per-Gaussian entries 1..9 of
    several files in the order given; the iteration is the last file's;
    spatial_lr_scale is the first file's LAST tuple entry, as the reference
    takes it (for the 14-entry tuple that entry is the octree state)."""
    all_params, it = [], 0
    for f in checkpoint_files:
        params, it = _load(f, map_location)
        all_params.append(params)
    cat = [torch.cat([p[i].detach() for p in all_params], dim=0) for i in range(1, 10)]
    return _tuple12(all_params[0][0], cat, all_params[0][-1]), it


def get_part_of_checkpoints(checkpoint_file, num_parts, part_id, map_location=None):
    """general_utils.py:598-637: rows [part_id * (P // num_parts + 1), min(next, P))."""
    params, it = _load(checkpoint_file, map_location)
    P = params[1].shape[0]
    per = P // num_parts + 1
    s, e = part_id * per, min((part_id + 1) * per, P)
    rows = [params[i].detach()[s:e] for i in range(1, 10)]
    return _tuple12(params[0], rows, params[11]), it


def drop_duplicate_gaussians(model_params, drop_duplicate_gaussians_coeff):
    """general_utils.py:640-675: keep rows arange(int(P * coeff)) % P."""
    if drop_duplicate_gaussians_coeff == 1.0:
        return model_params
    P = model_params[1].shape[0]
    keep = torch.arange(int(P * drop_duplicate_gaussians_coeff), device=model_params[1].device) % P
    rows = [model_params[i].detach()[keep] for i in range(1, 10)]
    return _tuple12(model_params[0], rows, model_params[11])


def load_checkpoint(start_checkpoint, world_size=1, rank=0, drop_duplicate_gaussians_coeff=1.0, map_location=None):
    """general_utils.py:678-736: this rank's model tuple and start iteration
    from a folder of chkpnt_ws=<n>_rk=<i>.pth files written at any world size n
    that is a multiple or a divisor of world_size (AssertionError otherwise,
    with the reference's messages)."""
    n_files = len(os.listdir(start_checkpoint))
    name = lambda i: checkpoint_path(start_checkpoint, n_files, i)
    if n_files == world_size:
        params, it = _load(name(rank), map_location)
    elif n_files > world_size:
        if n_files % world_size != 0:
            raise AssertionError("The number of files in the checkpoint folder must be a multiple of the number of "
                             "processes.")
        params, it = merge_multiple_checkpoints([name(i) for i in range(rank, n_files, world_size)], map_location)
    else:
        if world_size % n_files != 0:
            raise AssertionError("The number of files in the checkpoint folder must be a divisor of the number of "
                             "processes.")
        params, it = get_part_of_checkpoints(name(rank % n_files), world_size // n_files, rank // n_files,
                                             map_location)
    if drop_duplicate_gaussians_coeff != 1.0:
        params = drop_duplicate_gaussians(params, drop_duplicate_gaussians_coeff)
    return params, it
