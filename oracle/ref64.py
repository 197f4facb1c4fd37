"""Float64 numpy twin of the rasterizer forward (TEST INFRASTRUCTURE ONLY).

An independent restatement written from the mathematics rather than from the
reference's code layout, used to pin the fp32 C oracle:
  * 3D covariance  Sigma = R(q) S^2 R(q)^T with the textbook quaternion
    rotation matrix (BlitzGS utils/general_utils.py:448-483 builds the same);
  * EWA projection (Zwicker et al. 2002): Sigma2 = J W Sigma W^T J^T + 0.3 I
    with the perspective Jacobian J at the view-space mean, whose x/z and y/z
    are clamped to +-1.3 tan(fov/2) (_f/cuda_rasterizer/forward.cu:83-122);
  * real spherical harmonics up to degree 3, restated from
    utils/sh_utils.py:57-120 (eval_sh), colour = max(SH + 0.5, 0);
  * front-to-back alpha compositing with the reference's skip / stop rules
    (_r/cuda_rasterizer/forward.cu:328-396).
Everything is float64 so finite differences of it pin the fp32 backward.
"""
import math

import numpy as np

C0 = 0.28209479177387814
C1 = 0.4886025119029199
C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
      0.5462742152960396)
C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
      -0.4570457994644658, 1.445305721320277, -0.5900435899266435)


def quat_to_rot(q):
    """Rotation matrix of quaternion (w, x, y, z), applied without normalising."""
    w, x, y, z = q[..., 0], q[..., 1], q[..., 2], q[..., 3]
    R = np.empty(q.shape[:-1] + (3, 3))
    R[..., 0, 0] = 1 - 2 * (y * y + z * z)
    R[..., 0, 1] = 2 * (x * y - w * z)
    R[..., 0, 2] = 2 * (x * z + w * y)
    R[..., 1, 0] = 2 * (x * y + w * z)
    R[..., 1, 1] = 1 - 2 * (x * x + z * z)
    R[..., 1, 2] = 2 * (y * z - w * x)
    R[..., 2, 0] = 2 * (x * z - w * y)
    R[..., 2, 1] = 2 * (y * z + w * x)
    R[..., 2, 2] = 1 - 2 * (x * x + y * y)
    return R


def eval_sh(deg, sh, dirs):
    """sh: (P, K, 3), dirs: (P, 3) unit vectors -> (P, 3)."""
    x, y, z = dirs[:, 0:1], dirs[:, 1:2], dirs[:, 2:3]
    r = C0 * sh[:, 0]
    if deg > 0:
        r = r - C1 * y * sh[:, 1] + C1 * z * sh[:, 2] - C1 * x * sh[:, 3]
    if deg > 1:
        xx, yy, zz, xy, yz, xz = x * x, y * y, z * z, x * y, y * z, x * z
        r = (r + C2[0] * xy * sh[:, 4] + C2[1] * yz * sh[:, 5] + C2[2] * (2 * zz - xx - yy) * sh[:, 6]
             + C2[3] * xz * sh[:, 7] + C2[4] * (xx - yy) * sh[:, 8])
    if deg > 2:
        r = (r + C3[0] * y * (3 * xx - yy) * sh[:, 9] + C3[1] * xy * z * sh[:, 10]
             + C3[2] * y * (4 * zz - xx - yy) * sh[:, 11] + C3[3] * z * (2 * zz - 3 * xx - 3 * yy) * sh[:, 12]
             + C3[4] * x * (4 * zz - xx - yy) * sh[:, 13] + C3[5] * z * (xx - yy) * sh[:, 14]
             + C3[6] * x * (xx - 3 * yy) * sh[:, 15])
    return r


def project(cam, means3D, scales, rotations, opacities, sh, scale_modifier=1.0, sh_degree=3):
    """Screen-space parameters in float64.  Returns dict with means2D (px),
    conic (a, b, c), opacity, rgb, depth, valid (near-cull pass), cov2D."""
    m = np.asarray(means3D, np.float64)
    V = np.asarray(cam["viewmatrix"], np.float64).reshape(4, 4).T     # world -> view (math)
    PM = np.asarray(cam["projmatrix"], np.float64).reshape(4, 4).T    # world -> clip (math)
    W, H = cam["W"], cam["H"]
    tx, ty = cam["tanfovx"], cam["tanfovy"]
    fx, fy = W / (2 * tx), H / (2 * ty)
    hom = np.concatenate([m, np.ones((m.shape[0], 1))], axis=1)
    pv = hom @ V.T
    ph = hom @ PM.T
    pw = 1.0 / (ph[:, 3] + 1e-7)
    ndc = ph[:, :2] * pw[:, None]
    means2D = np.stack([((ndc[:, 0] + 1.0) * W - 1.0) * 0.5, ((ndc[:, 1] + 1.0) * H - 1.0) * 0.5], 1)
    R = quat_to_rot(np.asarray(rotations, np.float64))
    s = scale_modifier * np.asarray(scales, np.float64)
    Sigma = np.einsum("pij,pj,pkj->pik", R, s * s, R)
    t = pv[:, :3].copy()
    limx, limy = 1.3 * tx, 1.3 * ty
    t[:, 0] = np.clip(t[:, 0] / t[:, 2], -limx, limx) * t[:, 2]
    t[:, 1] = np.clip(t[:, 1] / t[:, 2], -limy, limy) * t[:, 2]
    J = np.zeros((m.shape[0], 2, 3))
    J[:, 0, 0] = fx / t[:, 2]
    J[:, 0, 2] = -fx * t[:, 0] / t[:, 2] ** 2
    J[:, 1, 1] = fy / t[:, 2]
    J[:, 1, 2] = -fy * t[:, 1] / t[:, 2] ** 2
    Wr = V[:3, :3]
    T = J @ Wr
    cov2 = T @ Sigma @ np.swapaxes(T, 1, 2)
    a = cov2[:, 0, 0] + 0.3
    b = cov2[:, 0, 1]
    c = cov2[:, 1, 1] + 0.3
    det = a * c - b * b
    conic = np.stack([c / det, -b / det, a / det], 1)
    dirs = m - np.asarray(cam["campos"], np.float64)[None]
    dirs = dirs / np.linalg.norm(dirs, axis=1, keepdims=True)
    rgb = np.maximum(eval_sh(sh_degree, np.asarray(sh, np.float64), dirs) + 0.5, 0.0)
    op = np.asarray(opacities, np.float64).reshape(-1)
    valid = pv[:, 2] > 0.2
    with np.errstate(invalid="ignore", divide="ignore"):
        extent = np.where(op > 1.0 / 255.0,
                          np.minimum(3.33, np.sqrt(2.0 * np.log(np.maximum(op * 255.0, 1e-300)))), 3.33)
    mid = 0.5 * (a + c)
    lam = mid + np.sqrt(np.maximum(0.01, mid * mid - det))
    radius = extent * np.sqrt(lam)
    return dict(means2D=means2D, conic=conic, opacity=op, rgb=rgb, depth=pv[:, 2], valid=valid,
                cov2D=np.stack([a, b, c], 1), radius=radius, extent=extent)


def render(W, H, bg, means2D, conic, opacity, rgb, ranges, point_list, compute_locally=None,
           signature=False):
    """Front-to-back compositing over the given per-tile sorted lists, float64.
    Returns the (3, H, W) image and the per-pixel final transmittance (and,
    with signature=True, a hash of which (pixel, Gaussian) pairs blended, so
    finite differences can detect a threshold crossing)."""
    sig = 0
    gx, gy = (W + 15) // 16, (H + 15) // 16
    img = np.zeros((3, H, W))
    finalT = np.zeros((H, W))
    bg = np.asarray(bg, np.float64)
    for t in range(gx * gy):
        if compute_locally is not None and not compute_locally.reshape(-1)[t]:
            continue
        tx0, ty0 = (t % gx) * 16, (t // gx) * 16
        xs = np.arange(tx0, min(tx0 + 16, W))
        ys = np.arange(ty0, min(ty0 + 16, H))
        px, py = np.meshgrid(xs.astype(np.float64), ys.astype(np.float64))
        px, py = px.reshape(-1), py.reshape(-1)
        Tr = np.ones(px.shape)
        Cc = np.zeros((3,) + px.shape)
        alive = np.ones(px.shape, bool)
        for k in range(int(ranges[t, 0]), int(ranges[t, 1])):
            g = int(point_list[k])
            dx, dy = means2D[g, 0] - px, means2D[g, 1] - py
            a, b, c = conic[g]
            power = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
            alpha = np.minimum(0.99, opacity[g] * np.exp(np.minimum(power, 0.0)))
            use = alive & (power <= 0.0) & (alpha >= 1.0 / 255.0)
            test = Tr * (1.0 - alpha)
            stop = use & (test < 1e-4)
            alive = alive & ~stop
            use = use & ~stop
            if signature:
                sig = (sig * 1000003 + int(np.flatnonzero(use).sum()) * 7919 + int(use.sum()) * (g + 1)) % (1 << 61)
            w = np.where(use, alpha * Tr, 0.0)
            Cc += rgb[g][:, None] * w[None]
            Tr = np.where(use, test, Tr)
            if not alive.any():
                break
        out = Cc + Tr[None] * bg[:, None]
        img[:, ys[0]:ys[-1] + 1, xs[0]:xs[-1] + 1] = out.reshape(3, len(ys), len(xs))
        finalT[ys[0]:ys[-1] + 1, xs[0]:xs[-1] + 1] = Tr.reshape(len(ys), len(xs))
    if signature:
        return img, finalT, sig
    return img, finalT
