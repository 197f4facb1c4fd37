"""CPU checks of the checkpoint layer (blitzgs_amd.checkpoint): the model
tuple, the chkpnt_ws=<n>_rk=<i>.pth naming, and resuming at another world
size (merge of several files, split of one, duplicate dropping), against the
rules of the reference's utils/general_utils.py:547-736 worked out by hand on
per-Gaussian rows whose values name their global row."""
import os

import pytest
import torch

from blitzgs_amd import checkpoint as ck


def shard(rows, sh_rest=15):
    """A model tuple whose per-Gaussian entries hold their global row index."""
    r = torch.as_tensor(rows, dtype=torch.float32)
    P = r.numel()
    col = lambda w: r[:, None].repeat(1, w)
    opt = torch.optim.Adam([torch.nn.Parameter(torch.zeros(P, 3))], lr=1e-3)
    return ck.capture(3, torch.nn.Parameter(col(3)), torch.nn.Parameter(col(3).view(P, 1, 3)),
                      torch.nn.Parameter(col(3 * sh_rest).view(P, sh_rest, 3)), torch.nn.Parameter(col(3)),
                      torch.nn.Parameter(col(4)), torch.nn.Parameter(col(1)), r.clone(), col(1), col(1),
                      opt.state_dict(), 2.5)


def rows_of(params):
    return params[1][:, 0].detach().to(torch.int64).tolist()


def write_ckpt(folder, n_files, per_file, iteration=700):
    # file i holds global rows [i * per_file, (i + 1) * per_file)
    for i in range(n_files):
        ck.save_checkpoint(str(folder), shard(range(i * per_file, (i + 1) * per_file)), iteration, n_files, i)


def test_naming_and_round_trip(tmp_path):
    write_ckpt(tmp_path, 1, 10)
    assert os.listdir(tmp_path) == ["chkpnt_ws=1_rk=0.pth"]
    params, it = ck.load_checkpoint(str(tmp_path), 1, 0)
    assert it == 700 and len(params) == 14
    assert rows_of(params) == list(range(10))
    assert isinstance(params[1], torch.nn.Parameter) and params[1].requires_grad
    assert params[10]["param_groups"][0]["lr"] == 1e-3 and params[11] == 2.5
    assert params[3].shape == (10, 15, 3)


def test_merge_when_more_files_than_ranks(tmp_path):
    write_ckpt(tmp_path, 4, 5)
    # world size 2: rank 0 merges files 0 and 2, rank 1 files 1 and 3
    p0, it = ck.load_checkpoint(str(tmp_path), 2, 0)
    p1, _ = ck.load_checkpoint(str(tmp_path), 2, 1)
    assert it == 700 and len(p0) == 12 and p0[10] is None
    assert rows_of(p0) == [0, 1, 2, 3, 4, 10, 11, 12, 13, 14]
    assert rows_of(p1) == [5, 6, 7, 8, 9, 15, 16, 17, 18, 19]
    for i in range(1, 10):
        assert p0[i].shape[0] == 10
    assert p0[7].tolist() == [0, 1, 2, 3, 4, 10, 11, 12, 13, 14]   # max_radii2D rows follow
    # the reference takes spatial_lr_scale from the last entry of the first
    # file's tuple, which for the 14-entry tuple is the octree state (None)
    assert p0[11] is None


def test_split_when_fewer_files_than_ranks(tmp_path):
    write_ckpt(tmp_path, 2, 10)
    # world size 8 over 2 files: 4 parts per file of 10 // 4 + 1 = 3 rows;
    # rank r reads file r % 2, part r // 2
    got = {r: rows_of(ck.load_checkpoint(str(tmp_path), 8, r)[0]) for r in range(8)}
    assert got[0] == [0, 1, 2] and got[2] == [3, 4, 5] and got[4] == [6, 7, 8] and got[6] == [9]
    assert got[1] == [10, 11, 12] and got[3] == [13, 14, 15] and got[5] == [16, 17, 18] and got[7] == [19]
    p, _ = ck.load_checkpoint(str(tmp_path), 8, 0)
    assert len(p) == 12 and p[11] == 2.5 and p[10] is None


def test_split_can_leave_a_rank_empty(tmp_path):
    write_ckpt(tmp_path, 1, 3)
    # 4 parts of 3 // 4 + 1 = 1 row: ranks 0..2 get one row, rank 3 none
    got = [rows_of(ck.load_checkpoint(str(tmp_path), 4, r)[0]) for r in range(4)]
    assert got == [[0], [1], [2], []]


def test_world_size_mismatch_errors(tmp_path):
    write_ckpt(tmp_path, 3, 2)
    with pytest.raises(AssertionError, match="multiple"):
        ck.load_checkpoint(str(tmp_path), 2, 0)
    with pytest.raises(AssertionError, match="divisor"):
        ck.load_checkpoint(str(tmp_path), 4, 0)


def test_drop_duplicate_gaussians(tmp_path):
    write_ckpt(tmp_path, 1, 4)
    p, _ = ck.load_checkpoint(str(tmp_path), 1, 0, drop_duplicate_gaussians_coeff=1.5)
    assert rows_of(p) == [0, 1, 2, 3, 0, 1]
    p, _ = ck.load_checkpoint(str(tmp_path), 1, 0, drop_duplicate_gaussians_coeff=0.5)
    assert rows_of(p) == [0, 1]
    assert p[3].shape == (2, 15, 3) and p[9].shape == (2, 1)


def test_restore_tuple_forms():
    full = shard(range(3))
    r = ck.restore(full)
    assert r["active_sh_degree"] == 3 and r["spatial_lr_scale"] == 2.5 and r["lod_level"] is None
    lod = torch.tensor([0, 1, 2], dtype=torch.int8)
    r = ck.restore(full[:12] + (lod,))
    assert r["lod_level"] is lod and r["octree_state"] is None
    r = ck.restore(full[:12] + (lod, {"depth": 4}))
    assert r["lod_level"] is lod and r["octree_state"] == {"depth": 4}
    r = ck.restore(full[:12])
    assert r["lod_level"] is None and r["xyz"] is full[1]


def test_files_load_with_weights_only(tmp_path):
    """The files hold nothing the restricted unpickler refuses (Adam state included)."""
    p = torch.nn.Parameter(torch.randn(4, 3))
    opt = torch.optim.Adam([{"params": [p], "lr": 0.01, "name": "xyz"}], eps=1e-15)
    p.grad = torch.randn(4, 3)
    opt.step()
    params = shard(range(4))[:10] + (opt.state_dict(), 1.0, None, None)
    path = ck.save_checkpoint(str(tmp_path), params, 30000)
    got, it = torch.load(path, weights_only=True)
    assert it == 30000
    assert torch.equal(got[10]["state"][0]["exp_avg"], opt.state_dict()["state"][0]["exp_avg"])
    assert got[10]["param_groups"][0]["name"] == "xyz"
