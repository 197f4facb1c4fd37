"""Seeded synthetic Gaussian scenes and cameras for the five benchmark configs.

Cameras follow the reference's conventions (BlitzGS utils/graphics_utils.py:42-76,
scene/cameras.py:111-133): ``viewmatrix`` is getWorld2View2(R, T) transposed,
``projmatrix`` is viewmatrix @ getProjectionMatrix(znear=0.01, zfar=100).T, and
``campos`` is the camera centre.  R is the camera-to-world rotation whose
columns are the camera's x (right), y (down) and z (forward) axes in world
coordinates, T = -R^T C.

Scenes are drawn with numpy ``Generator(PCG64(seed))`` in the fixed order:
means (float64) -> log-scales -> quaternions -> opacity logits (float64) ->
SH (one (P,16,3) float32 standard-normal draw; coefficient 0 is scaled by the
DC standard deviation, the other 15 by the higher-band one) -> dL/dimage
(float32).  Parameters are returned already
activated, as the reference's GaussianModel hands them to the rasterizer
(scene/gaussian_model.py:53-58): scales = exp(log-scale), rotations =
normalised quaternions (r, x, y, z), opacities = sigmoid(logit) with shape
(P, 1), sh = (P, 16, 3).
"""
import math

import numpy as np

ZNEAR, ZFAR = 0.01, 100.0


def projection_matrix(znear, zfar, fovx, fovy):
    """getProjectionMatrix (utils/graphics_utils.py:56-76), float64."""
    tan_y, tan_x = math.tan(fovy / 2), math.tan(fovx / 2)
    top, right = tan_y * znear, tan_x * znear
    bottom, left = -top, -right
    P = np.zeros((4, 4))
    P[0, 0] = 2.0 * znear / (right - left)
    P[1, 1] = 2.0 * znear / (top - bottom)
    P[0, 2] = (right + left) / (right - left)
    P[1, 2] = (top + bottom) / (top - bottom)
    P[3, 2] = 1.0
    P[2, 2] = zfar / (zfar - znear)
    P[2, 3] = -(zfar * znear) / (zfar - znear)
    return P


def world2view(R, t):
    """getWorld2View2 with translate 0, scale 1 (utils/graphics_utils.py:42-53)."""
    Rt = np.zeros((4, 4))
    Rt[:3, :3] = R.T
    Rt[:3, 3] = t
    Rt[3, 3] = 1.0
    return Rt


def make_camera(R, C, W, H, fovx, fovy=None):
    """Camera dict from camera-to-world rotation R (3x3) and centre C."""
    if fovy is None:
        fovy = 2.0 * math.atan(math.tan(fovx / 2) * H / W)
    R = np.asarray(R, np.float64)
    C = np.asarray(C, np.float64)
    t = -R.T @ C
    w2v = world2view(R, t)
    view = w2v.T.astype(np.float32)                      # world_view_transform
    projT = projection_matrix(ZNEAR, ZFAR, fovx, fovy).T.astype(np.float32)
    full = (view @ projT).astype(np.float32)             # full_proj_transform
    campos = np.linalg.inv(view.astype(np.float64))[3, :3].astype(np.float32)
    return dict(W=int(W), H=int(H), fovx=float(fovx), fovy=float(fovy),
                tanfovx=math.tan(fovx * 0.5), tanfovy=math.tan(fovy * 0.5),
                viewmatrix=view, projmatrix=full, campos=campos)


def look_at(C, target, W, H, fovx, up=(0.0, 0.0, 1.0)):
    C = np.asarray(C, np.float64)
    f = np.asarray(target, np.float64) - C
    f /= np.linalg.norm(f)
    r = np.cross(f, np.asarray(up, np.float64))
    if np.linalg.norm(r) < 1e-9:
        r = np.cross(f, np.array([0.0, 1.0, 0.0]))
    r /= np.linalg.norm(r)
    d = np.cross(f, r)
    R = np.stack([r, d, f], axis=1)
    return make_camera(R, C, W, H, fovx)


def _quats(rng, P):
    q = rng.standard_normal((P, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _finish(rng, means, log_mu, log_sd, op_mu, op_sd, P, dc_sd=0.5, rest_sd=0.05, K=16):
    log_scales = rng.normal(log_mu, log_sd, size=(P, 3))
    quats = _quats(rng, P)
    op_logit = rng.normal(op_mu, op_sd, size=(P, 1))
    sh = rng.standard_normal((P, K, 3), dtype=np.float32)
    sh[:, 0, :] *= np.float32(dc_sd)
    sh[:, 1:, :] *= np.float32(rest_sd)
    return dict(means3D=means.astype(np.float32), scales=np.exp(log_scales).astype(np.float32),
                rotations=quats.astype(np.float32), opacities=_sigmoid(op_logit).astype(np.float32),
                sh=sh)


def _ground_plane_means(rng, P):
    """400x400 m plane, height |N(0,15)|, 30% in 200 ball-shaped 10 m clusters."""
    n_cl = int(round(0.3 * P))
    n_bg = P - n_cl
    bg = np.empty((n_bg, 3))
    bg[:, 0:2] = rng.uniform(-200.0, 200.0, size=(n_bg, 2))
    bg[:, 2] = np.abs(rng.normal(0.0, 15.0, size=n_bg))
    centers = np.empty((200, 3))
    centers[:, 0:2] = rng.uniform(-200.0, 200.0, size=(200, 2))
    centers[:, 2] = 10.0
    which = rng.integers(0, 200, size=n_cl)
    d = rng.standard_normal((n_cl, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rad = 10.0 * np.cbrt(rng.uniform(0.0, 1.0, size=(n_cl, 1)))
    cl = centers[which] + d * rad
    return np.concatenate([bg, cl], axis=0)


def aerial_camera(W, H, fovx_deg=60.0, altitude=150.0, tilt_deg=30.0):
    """Camera at `altitude`, optical axis tilted `tilt_deg` off nadir, aimed at the origin."""
    back = altitude * math.tan(math.radians(tilt_deg))
    return look_at((0.0, -back, altitude), (0.0, 0.0, 0.0), W, H, math.radians(fovx_deg))


def config0():
    """16,384 Gaussians in [-1,1]^3, camera at (0,0,-4) looking down +z, 256x256, FoV 60."""
    rng = np.random.Generator(np.random.PCG64(0))
    P = 16384
    means = rng.uniform(-1.0, 1.0, size=(P, 3))
    scene = _finish(rng, means, -4.0, 0.5, 0.0, 1.0, P)
    cam = make_camera(np.eye(3), (0.0, 0.0, -4.0), 256, 256, math.radians(60.0), math.radians(60.0))
    scene["dL_dimage"] = rng.standard_normal((3, 256, 256)).astype(np.float32)
    return scene, cam


def config1(P=1_000_000):
    """64 anisotropic clusters in a 10^3 box, 1920x1080, FoVx 50, radius-8 sphere."""
    rng = np.random.Generator(np.random.PCG64(1))
    centers = rng.uniform(-4.0, 4.0, size=(64, 3))
    axes_sd = np.exp(rng.normal(math.log(0.6), 0.4, size=(64, 3)))
    rots = np.stack([np.linalg.qr(rng.standard_normal((3, 3)))[0] for _ in range(64)])
    which = rng.integers(0, 64, size=P)
    local = rng.standard_normal((P, 3)) * axes_sd[which]
    means = centers[which] + np.einsum("pij,pj->pi", rots[which], local)
    means = np.clip(means, -5.0, 5.0)
    scene = _finish(rng, means, -3.5, 0.7, 0.0, 1.5, P)
    az, el = math.radians(30.0), math.radians(20.0)
    C = 8.0 * np.array([math.cos(el) * math.cos(az), math.cos(el) * math.sin(az), math.sin(el)])
    cam = look_at(C, (0.0, 0.0, 0.0), 1920, 1080, math.radians(50.0))
    scene["target"] = rng.uniform(0.0, 1.0, size=(1, 3, 1080, 1920)).astype(np.float32)
    return scene, cam


def config2(P=6_000_000, W=1600, H=1066, seed=2):
    """City-scale aerial share: 6M Gaussians, 1600x1066, 150 m altitude, 30 deg tilt."""
    rng = np.random.Generator(np.random.PCG64(seed))
    means = _ground_plane_means(rng, P)
    scene = _finish(rng, means, -1.5, 0.8, 0.5, 1.5, P)
    cam = aerial_camera(W, H)
    scene["dL_dimage"] = rng.standard_normal((3, H, W), dtype=np.float32)
    return scene, cam


def config3(P=8_000_000):
    """Workload-division share: 8M Gaussians, 4096x2730, tile rows [43, 86) of 171."""
    scene, cam = config2(P=P, W=4096, H=2730, seed=3)
    gx, gy = (cam["W"] + 15) // 16, (cam["H"] + 15) // 16
    cl = np.zeros((gy, gx), np.uint8)
    rows = tile_row_block(gy, 4, 1)
    cl[rows[0]:rows[1], :] = 1
    scene["compute_locally"] = cl
    return scene, cam


def tile_row_block(n_rows, world_size, rank):
    """Contiguous tile-row block of one rank, ceil(n/W) rows per rank."""
    per = -(-n_rows // world_size)
    lo = min(n_rows, per * rank)
    return lo, min(n_rows, lo + per)


def config4_points(P=10_000_000):
    rng = np.random.Generator(np.random.PCG64(4))
    return _ground_plane_means(rng, P).astype(np.float32)


def config4_images(B=8, H=1080, W=1920, seed=4):
    rng = np.random.Generator(np.random.PCG64(seed + 100))
    a = rng.uniform(0.0, 1.0, size=(B, 3, H, W)).astype(np.float32)
    b = rng.uniform(0.0, 1.0, size=(B, 3, H, W)).astype(np.float32)
    return a, b


def small_scene(P, seed, W=64, H=48, extent=1.0, log_mu=-2.5, log_sd=0.4, op_mu=0.0, op_sd=1.0,
                cam_dist=4.0, fov_deg=60.0):
    """Small scene for parity tests: means in [-extent, extent]^3 in front of a
    camera at distance cam_dist looking along +z."""
    rng = np.random.Generator(np.random.PCG64(seed))
    means = rng.uniform(-extent, extent, size=(P, 3))
    scene = _finish(rng, means, log_mu, log_sd, op_mu, op_sd, P)
    cam = make_camera(np.eye(3), (0.0, 0.0, -cam_dist), W, H, math.radians(fov_deg))
    scene["dL_dimage"] = rng.standard_normal((3, H, W)).astype(np.float32)
    return scene, cam


CONFIGS = {0: config0, 1: config1, 2: config2, 3: config3}
