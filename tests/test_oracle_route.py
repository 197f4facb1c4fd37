"""Pinning the routing oracle (oracle/o_route.c) without the reference's code.

The reference has no tests or vectors for get_local2j_ids_bool*, so the oracle
is pinned by:
* hand-worked cases of the integer rules (the unsigned tile span read as int,
  the culled Gaussian at the origin, rects clamped at the image border, the
  avoid_pixel_all2all widening below tile 0, the unsigned-versus-int rectangle
  test);
* an independent code path: the binning oracle's tile count (o_binning_count,
  which enumerates the tiles of each rect) with compute_locally set to one
  rank's tiles.  For a rank owning whole tile rows (the strategy
  workload_division.py:682-704 builds: division_pos * TILE_X) or a tile
  rectangle (mode 6), and a Gaussian with a non-empty rect, "routed to the
  rank" must equal "has a tile there" exactly; for an arbitrary tile range the
  route must be a superset (the row-major span covers every tile of the rect).
"""
import numpy as np
import pytest

from oracle import oracle as O


def _rect(p, r, gx, gy):
    """The rect a test expects, worked out in numpy float32 (auxiliary.h:51-61)."""
    p = np.asarray(p, np.float32)
    rf = np.float32(r)
    f = lambda v: int(np.trunc(v))
    c = lambda v, g: min(max(v, 0), g)
    x0 = c(f((p[0] - rf) / np.float32(16)), gx)
    y0 = c(f((p[1] - rf) / np.float32(16)), gy)
    x1 = c(f((((p[0] + rf) + np.float32(16)) - np.float32(1)) / np.float32(16)), gx)
    y1 = c(f((((p[1] + rf) + np.float32(16)) - np.float32(1)) / np.float32(16)), gy)
    return x0, y0, x1, y1


def test_hand_cases_interval():
    H = W = 64                      # 4 x 4 tiles
    m2d = np.array([[0, 0],         # culled at the origin: span end wraps negative -> nowhere
                    [17.5, 17.5],   # radius 0 but rect (1,1)-(2,2): tile 5 -> rank 0
                    [300, 5],       # right of the image, one row: empty span -> nowhere
                    [300, 40],      # right of the image, rows 2..3: span [gx*y0+gx, ...] non-empty
                    [8, 8],         # radius 40: whole image -> both ranks
                    [40, 56]],      # radius 1: tile (2,3) = 14 -> rank 1
                   np.float32)
    radii = np.array([0, 0, 3, 20, 40, 1], np.int32)
    got = O.local2j_ids_bool(H, W, m2d, radii, [0, 8, 16])
    # case 3 worked by hand: x0 = x1 = 4 (clamped), y0 = 1, y1 = 4
    # lo = 1*4 + 4 = 8, hi = 3*4 + 4 - 1 = 15 -> [8, 15] meets rank 1's [8, 16) only
    exp = np.array([[0, 0], [1, 0], [0, 0], [0, 1], [1, 1], [0, 1]], bool)
    assert (got == exp).all(), got


def test_hand_cases_interval_avoid():
    H = W = 64
    m2d = np.array([[17.5, 17.5], [40, 56], [0, 0]], np.float32)
    radii = np.array([0, 1, 0], np.int32)
    # avoid widens [0, 8) to [-5, 13) and [8, 16) to [3, 21)
    got = O.local2j_ids_bool(H, W, m2d, radii, [0, 8, 16], avoid=True)
    exp = np.array([[1, 1], [0, 1], [0, 0]], bool)   # tile 5 in both widened ranges; 14 only in rank 1's
    assert (got == exp).all(), got


def test_hand_cases_rect():
    H = W = 64
    # rank 0: rows [0, 2) x cols [0, 4); rank 1: rows [2, 4) x cols [0, 2); rank 2: rows [2, 4) x cols [2, 4)
    rects = np.array([[0, 2, 0, 4], [2, 4, 0, 2], [2, 4, 2, 4]], np.int32)
    m2d = np.array([[17.5, 17.5],    # rect (1,1)-(2,2) -> rank 0
                    [40, 56],        # rect (2,3)-(3,4) -> rank 2
                    [300, 40],       # x0 = x1 = 4: x_r <= x0 for every rank -> nowhere
                    [0, 0],          # rect (0,0)-(0,0): y1 <= y_l fails for y_l = 0 but x1 <= x_l holds -> nowhere
                    [31.5, 31.5]],   # radius 1: rect (1,1)-(2,2) -> rank 0
                   np.float32)
    radii = np.array([0, 1, 20, 0, 1], np.int32)
    got = O.local2j_ids_bool_rect(H, W, m2d, radii, rects)
    exp = np.array([[1, 0, 0], [0, 0, 1], [0, 0, 0], [0, 0, 0], [1, 0, 0]], bool)
    assert (got == exp).all(), got
    # widened by one tile: rank 0 becomes rows [0, 3) x cols [0, 5), rank 1 rows [1, 5) x cols [0, 3),
    # rank 2 rows [1, 5) x cols [1, 5); the empty rect at x = 4 now lies inside ranks 0 and 2 (x_l < 4 < x_r)
    got = O.local2j_ids_bool_rect(H, W, m2d, radii, rects, avoid=True)
    exp = np.array([[1, 1, 1], [0, 1, 1], [1, 0, 1], [0, 0, 0], [1, 1, 1]], bool)
    assert (got == exp).all(), got


def _scene(P, H, W, seed):
    rng = np.random.default_rng(seed)
    m2d = np.stack([rng.uniform(-100, W + 100, P), rng.uniform(-100, H + 100, P)], 1).astype(np.float32)
    radii = rng.integers(0, 90, P).astype(np.int32)
    radii[rng.random(P) < 0.1] = 0
    return m2d, radii


def _tiles_in(m2d, radii, H, W, mask):
    cnt = np.empty(m2d.shape[0], np.uint32)
    from oracle.oracle import lib, _p
    lib().o_binning_count(m2d.shape[0], W, H, _p(m2d), _p(radii), _p(mask.astype(np.uint8)), _p(cnt))
    return cnt > 0


def _nonempty(m2d, radii, H, W):
    gx, gy = (W + 15) // 16, (H + 15) // 16
    r = np.array([_rect(p, int(rr), gx, gy) for p, rr in zip(m2d, radii)])
    return (radii > 0) & (r[:, 0] < r[:, 2]) & (r[:, 1] < r[:, 3])


@pytest.mark.parametrize("seed", [0, 1])
def test_row_strategy_equals_binning(seed):
    H, W = 600, 900                  # 38 x 57 tiles
    gx, gy = 57, 38
    m2d, radii = _scene(3000, H, W, seed)
    rows = [0, 7, 13, 30, 38]
    strategy = np.array(rows) * gx  # division_pos * TILE_X
    got = O.local2j_ids_bool(H, W, m2d, radii, strategy)
    ne = _nonempty(m2d, radii, H, W)
    assert ne.sum() > 1000
    for rk in range(len(rows) - 1):
        mask = np.zeros((gy, gx), bool)
        mask[rows[rk]:rows[rk + 1]] = True
        has = _tiles_in(m2d, radii, H, W, mask)
        assert (got[ne, rk] == has[ne]).all(), rk


@pytest.mark.parametrize("seed", [2, 3])
def test_tile_range_strategy_covers_binning(seed):
    H, W = 600, 900
    gx, gy = 57, 38
    m2d, radii = _scene(3000, H, W, seed)
    strategy = np.array([0, 100, 120, 1003, 2166])   # rank 1: row 1 cols 43-56 and row 2 cols 0-5
    got = O.local2j_ids_bool(H, W, m2d, radii, strategy)
    ne = _nonempty(m2d, radii, H, W)
    routed_somewhere_strictly_more = 0
    for rk in range(4):
        mask = np.zeros(gx * gy, bool)
        mask[strategy[rk]:strategy[rk + 1]] = True
        has = _tiles_in(m2d, radii, H, W, mask.reshape(gy, gx))
        assert (got[has, rk]).all(), rk        # every rank with a tile of the rect gets the Gaussian
        routed_somewhere_strictly_more += int((got[ne, rk] & ~has[ne]).sum())
    # the span is row-major, so a rect over several rows also reaches a short
    # range that lies between its tiles
    assert routed_somewhere_strictly_more > 0


@pytest.mark.parametrize("seed", [4, 5])
def test_rect_strategy_equals_binning(seed):
    H, W = 600, 900
    gx, gy = 57, 38
    m2d, radii = _scene(3000, H, W, seed)
    rects = np.array([[0, 20, 0, 30], [0, 20, 30, 57], [20, 38, 0, 11], [20, 38, 11, 57]], np.int32)
    got = O.local2j_ids_bool_rect(H, W, m2d, radii, rects)
    ne = _nonempty(m2d, radii, H, W)
    for rk, (yl, yr, xl, xr) in enumerate(rects):
        mask = np.zeros((gy, gx), bool)
        mask[yl:yr, xl:xr] = True
        has = _tiles_in(m2d, radii, H, W, mask)
        assert (got[ne, rk] == has[ne]).all(), rk
    # with the one-tile widening the rank's rectangle grows by one tile per side
    got = O.local2j_ids_bool_rect(H, W, m2d, radii, rects, avoid=True)
    for rk, (yl, yr, xl, xr) in enumerate(rects):
        mask = np.zeros((gy, gx), bool)
        mask[max(yl - 1, 0):yr + 1, max(xl - 1, 0):xr + 1] = True
        has = _tiles_in(m2d, radii, H, W, mask)
        assert (got[ne, rk] == has[ne]).all(), rk


def test_one_rank_everything_with_a_rect():
    H, W = 256, 256
    m2d, radii = _scene(2000, H, W, 6)
    got = O.local2j_ids_bool(H, W, m2d, radii, [0, 256])
    ne = _nonempty(m2d, radii, H, W)
    assert got[ne, 0].all()
