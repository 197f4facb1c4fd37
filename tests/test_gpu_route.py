"""GPU parity of the routing and the screen-space exchange (blitzgs_amd.routing,
blitzgs_amd/csrc/route.hip) through the C ABI.

* the bool matrix (both modes, avoid on and off, 1 to 100 ranks) bit for bit
  against the CPU oracle, on preprocessed Gaussians and on edge inputs (NaN
  and huge means, radius 0, rects outside the image, empty inputs);
* the per-rank id lists against nonzero() of the oracle's matrix;
* pack / unpack / scatter and the one-process exchange against the
  reference's torch expressions (cat + index, split, index_put backward),
  bit for bit (they only move values);
* config 3's 8M Gaussians routed to four tile-row ranks.
"""
import numpy as np
import pytest
import torch

from blitzgs_amd import routing, synth
from oracle import oracle as O
from tests.gpu_helpers import gpu_preprocess, gpu_render_forward, np_, settings_for, to_dev

pytestmark = pytest.mark.gpu


def _edge_inputs(H, W, seed=0, P=20000):
    rng = np.random.default_rng(seed)
    m2d = np.stack([rng.uniform(-200, W + 200, P), rng.uniform(-200, H + 200, P)], 1).astype(np.float32)
    radii = rng.integers(0, 120, P).astype(np.int32)
    radii[rng.random(P) < 0.2] = 0
    m2d[:8] = [[0, 0], [np.nan, 5], [5, np.nan], [1e30, 1e30], [-1e30, 3], [W, H], [W - 0.5, H - 0.5], [16, 16]]
    radii[:8] = [0, 3, 3, 7, 7, 0, 0, 0]
    radii[8:12] = [2 ** 30, 1, 0, 2 ** 31 - 1]
    return m2d, radii


def _strategies(gx, gy):
    T = gx * gy
    yield [0, T]
    yield [0, 40, 41, T // 2, T]
    rows = np.linspace(0, gy, 5).astype(int)
    yield list(rows * gx)
    yield list(np.linspace(0, T, 9).astype(int))
    yield list(np.linspace(0, T, 65).astype(int))


def _rects(gx, gy):
    yield [[0, gy, 0, gx]]
    yield [[0, gy // 2, 0, gx // 3], [0, gy // 2, gx // 3, gx], [gy // 2, gy, 0, gx // 2], [gy // 2, gy, gx // 2, gx]]
    ys = np.linspace(0, gy, 4).astype(int)
    xs = np.linspace(0, gx, 3).astype(int)
    yield [[ys[i], ys[i + 1], xs[j], xs[j + 1]] for i in range(3) for j in range(2)]


@pytest.mark.parametrize("avoid", [False, True])
def test_bool_interval_matches_oracle(gpu, avoid):
    H, W = 700, 1000
    gx, gy = 63, 44
    m2d, radii = _edge_inputs(H, W)
    dm, dr = to_dev(m2d), to_dev(radii)
    args = {"avoid_pixel_all2all": avoid}
    for st in _strategies(gx, gy):
        world = len(st) - 1
        print("interval", avoid, world, flush=True)
        got = np_(routing.get_local2j_ids_bool(H, W, 0, world, dm, dr, torch.tensor(st, dtype=torch.int32,
                                                                                      device="cuda"), args))
        exp = O.local2j_ids_bool(H, W, m2d, radii, st, avoid)
        assert got.shape == exp.shape and got.dtype == np.bool_
        bad = np.flatnonzero(got != exp)
        assert bad.size == 0, (world, bad[:5])


@pytest.mark.parametrize("avoid", [False, True])
def test_bool_rect_matches_oracle(gpu, avoid):
    H, W = 700, 1000
    gx, gy = 63, 44
    m2d, radii = _edge_inputs(H, W, seed=1)
    dm, dr = to_dev(m2d), to_dev(radii)
    for rc in _rects(gx, gy):
        world = len(rc)
        got = np_(routing.get_local2j_ids_bool_adjust_mode6(H, W, 0, world, dm, dr,
                                                            torch.tensor(rc, dtype=torch.int32, device="cuda"),
                                                            {"avoid_pixel_all2all": avoid}))
        exp = O.local2j_ids_bool_rect(H, W, m2d, radii, rc, avoid)
        assert (got == exp).all(), world


def test_bool_many_ranks(gpu):
    # more ranks than the id-list path takes: the bool matrix has no bound
    H, W = 512, 512
    m2d, radii = _edge_inputs(H, W, seed=2, P=5000)
    st = list(np.linspace(0, 32 * 32, 101).astype(int))
    got = np_(routing.get_local2j_ids_bool(H, W, 0, 100, to_dev(m2d), to_dev(radii), st))
    assert (got == O.local2j_ids_bool(H, W, m2d, radii, st)).all()


@pytest.mark.parametrize("mode", [routing.INTERVAL, routing.RECT])
def test_id_lists_match_nonzero(gpu, mode):
    H, W = 700, 1000
    gx, gy = 63, 44
    for seed, P in [(3, 20000), (4, 1), (5, 257), (6, 70000)]:
        m, r = _edge_inputs(H, W, seed=seed, P=max(P, 12))
        m2d, radii = m[:P].copy(), r[:P].copy()
        tables = list(_strategies(gx, gy)) if mode == routing.INTERVAL else list(_rects(gx, gy))
        for tab in tables:
            world = len(tab) - 1 if mode == routing.INTERVAL else len(tab)
            for avoid in (False, True):
                ids, b = routing.local2j_ids(to_dev(m2d), to_dev(radii), H, W, tab, world, mode=mode,
                                             avoid_pixel_all2all=avoid, want_bool=True)
                exp = (O.local2j_ids_bool(H, W, m2d, radii, tab, avoid) if mode == routing.INTERVAL
                       else O.local2j_ids_bool_rect(H, W, m2d, radii, tab, avoid))
                assert (np_(b) == exp).all()
                assert len(ids) == world
                for rk in range(world):
                    e = np.flatnonzero(exp[:, rk])
                    g = np_(ids[rk])
                    assert g.dtype == np.int64 and g.shape == e.shape and (g == e).all(), (seed, world, rk)


def test_id_lists_empty_input(gpu):
    ids, b = routing.local2j_ids(torch.empty((0, 2), device="cuda"), torch.empty(0, dtype=torch.int32, device="cuda"),
                                 64, 64, [0, 8, 16], 2, want_bool=True)
    assert [t.numel() for t in ids] == [0, 0] and b.shape == (0, 2)


def _fields(P, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).cuda()
    return [mk(P, 2), mk(P, 3), mk(P, 4), torch.randint(0, 500, (P,), generator=g, dtype=torch.int32).cuda(),
            mk(P), mk(P, 3), mk(P, 3), mk(P, 4)]


def test_pack_unpack_scatter_match_torch(gpu):
    P = 100003
    f = _fields(P, 7)
    ids = torch.sort(torch.randperm(P, device="cuda")[:60001]).values
    # pack: the reference's cat of the state fields then index
    state = [f[0], f[1], f[2], f[5], f[6], f[7]]
    buf = routing.pack_rows(ids, state)
    ref = torch.cat(state, dim=1)[ids]
    assert torch.equal(buf, ref)
    aux = routing.pack_rows(ids, [f[3], f[4]])
    assert torch.equal(aux, torch.cat([f[3].float().unsqueeze(1), f[4].unsqueeze(1)], 1)[ids])
    # unpack: split + contiguous; radii back to int
    outs = routing.unpack_rows(buf, [2, 3, 4, 3, 3, 4], [torch.float32] * 6)
    for o, r in zip(outs, torch.split(ref, [2, 3, 4, 3, 3, 4], dim=1)):
        assert o.is_contiguous() and torch.equal(o, r)
    r_i, d = routing.unpack_rows(aux, [1, 1], [torch.int32, torch.float32])
    assert torch.equal(r_i.squeeze(1), f[3][ids]) and torch.equal(d.squeeze(1), f[4][ids])
    # scatter: index backward (zeros elsewhere), then accumulate a second rank's rows
    g = torch.randn(ids.numel(), 19, device="cuda")
    sc = routing.scatter_rows(ids, [g[:, :2], g[:, 2:5]], P)
    exp0 = torch.zeros(P, 2, device="cuda").index_put_((ids,), g[:, :2], accumulate=True)
    assert torch.equal(sc[0], exp0)
    ids2 = torch.sort(torch.randperm(P, device="cuda")[:3000]).values
    g2 = torch.randn(ids2.numel(), 2, device="cuda")
    routing.scatter_rows(ids2, [g2], P, out=[sc[0]], accumulate=True)
    assert torch.equal(sc[0], exp0.index_put_((ids2,), g2, accumulate=True))


class _Strategy:
    """A stand-in for the reference's DivisionStrategyFinal with one rank: its
    get_local2j_ids (workload_division.py:682-704) as the reference writes it,
    calling the drop-in _C op."""

    def __init__(self, division_pos, tile_x):
        self.division_pos = division_pos
        self.tile_x = tile_x
        self.world_size = len(division_pos) - 1
        self.rank = 0
        self.gpu_ids = [0]

    def get_local2j_ids(self, means2D, radii, raster_settings, cuda_args):
        from blitzgs_amd import compat_ops as _C
        st = torch.tensor(self.division_pos, dtype=torch.int, device=means2D.device) * self.tile_x
        b = _C.get_local2j_ids_bool(raster_settings.image_height, raster_settings.image_width, self.rank,
                                    self.world_size, means2D, radii, st, cuda_args)
        return [b[:, rk].nonzero(as_tuple=True)[0] for rk in range(self.world_size)], b


class _Rast:
    def __init__(self, rs):
        self.raster_settings = rs


def test_single_process_exchange_matches_reference_flow(gpu):
    scene, cam = synth.config0()
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    P = g["means2D"].size(0)
    gx = (cam["W"] + 15) // 16
    gy = (cam["H"] + 15) // 16
    extra = _fields(P, 9)
    # every third Gaussian culled (radius 0, mean at the origin): routed nowhere
    radii = g["radii"].clone()
    radii[::3] = 0
    m2d = g["means2D"].clone()
    m2d[::3] = 0
    leaves = [m2d.requires_grad_(), g["rgb"].clone().requires_grad_(),
              g["conic_opacity"].clone().requires_grad_(), extra[5].requires_grad_(), extra[6].requires_grad_(),
              extra[7].requires_grad_()]
    params = [leaves[0], leaves[1], leaves[2], radii, g["depths"], leaves[3], leaves[4], leaves[5]]
    strat = _Strategy([0, gy], gx)
    out = routing.all_to_all_communication_final([_Rast(rs)], [params], [{"avoid_pixel_all2all": False}], [strat])
    ids = strat.get_local2j_ids(m2d.detach(), radii, rs, {"avoid_pixel_all2all": False})[0][0]
    assert out[8] == [[[ids.numel()]]] and torch.equal(out[9][0][0], ids)
    assert 0 < ids.numel() <= P - P // 3
    # the reference's one-rank flow (gaussian_renderer/__init__.py:117-189): cat, index, split
    ref_leaves = [t.detach().clone().requires_grad_() for t in leaves]
    cat = torch.cat([ref_leaves[0], ref_leaves[1], ref_leaves[2], ref_leaves[3], ref_leaves[4], ref_leaves[5]], 1)[ids]
    ref = torch.split(cat, [2, 3, 4, 3, 3, 4], dim=1)
    aux = torch.cat([radii.float().unsqueeze(1), g["depths"].unsqueeze(1)], 1)[ids]
    got = [out[0][0], out[1][0], out[2][0], out[5][0], out[6][0], out[7][0]]
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    assert out[3][0].dtype == torch.int32 and torch.equal(out[3][0], aux[:, 0].int())
    assert torch.equal(out[4][0], aux[:, 1])
    # gradients: the same upstream gradients through both graphs
    ups = [torch.randn_like(t) for t in got]
    torch.autograd.backward(got, ups)
    torch.autograd.backward(list(ref), ups)
    for a, b in zip(leaves, ref_leaves):
        assert torch.equal(a.grad, b.grad)


def test_config3_routing_four_row_ranks(gpu):
    scene, cam = synth.config3()
    rs = settings_for(cam)
    g = gpu_preprocess(scene, rs)
    gx = (cam["W"] + 15) // 16
    gy = (cam["H"] + 15) // 16
    rows = [0, 43, 86, 129, gy]
    st = [r * gx for r in rows]
    ids, b = routing.local2j_ids(g["means2D"], g["radii"], cam["H"], cam["W"], st, 4, want_bool=True)
    exp = O.local2j_ids_bool(cam["H"], cam["W"], np_(g["means2D"]), np_(g["radii"]), st)
    bb = np_(b)
    assert (bb == exp).all()
    for rk in range(4):
        e = np.flatnonzero(exp[:, rk])
        assert np_(ids[rk]).shape == e.shape and (np_(ids[rk]) == e).all()
    # every Gaussian the binning lists in rank 1's rows (the config 3 share) is routed to rank 1
    out = gpu_render_forward(rs, g["means2D"], g["depths"], g["radii"], g["conic_opacity"], g["rgb"],
                             compute_locally=scene["compute_locally"])
    listed = np.unique(np_(out["point_list"])[:out["R"]].astype(np.int64))
    assert listed.size > 0 and bb[listed, 1].all()
