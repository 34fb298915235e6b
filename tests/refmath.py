"""Independent fp64 re-derivations used to pin the golden model.

Written from the underlying mathematics rather than from the oracle's code:
  - real spherical harmonics from their closed-form normalisation constants;
  - the 2DGS splat homography T = A * P * [t_u t_v p] (Huang et al. 2024,
    Eq. 8-10) and the ray-splat intersection solved as a 2x2 linear system;
  - front-to-back alpha compositing with the fork's skip rules
    (msplat_metal.metal:663-721);
  - SSIM (Wang et al. 2004) with an explicit 2D 11x11 Gaussian window and
    zero padding, plus L1.
Only used on tiny inputs (pure Python / numpy loops).
"""
from __future__ import annotations

import math

import numpy as np

PI = math.pi


def sh_constants():
    """Closed-form real-SH normalisations in the order msplat evaluates them."""
    c0 = 1.0 / (2.0 * math.sqrt(PI))
    c1 = math.sqrt(3.0 / (4.0 * PI))
    a = 0.5 * math.sqrt(15.0 / PI)
    c2 = [a, -a, 0.25 * math.sqrt(5.0 / PI), -a, 0.25 * math.sqrt(15.0 / PI)]
    b = 0.25 * math.sqrt(35.0 / (2.0 * PI))
    d = 0.25 * math.sqrt(21.0 / (2.0 * PI))
    c3 = [-b, 0.5 * math.sqrt(105.0 / PI), -d, 0.25 * math.sqrt(7.0 / PI), -d, 0.25 * math.sqrt(105.0 / PI), -b]
    return c0, c1, c2, c3


def sh_basis(d: np.ndarray, degree: int) -> np.ndarray:
    """Real SH basis values [.., (degree+1)^2] at unit directions d [.., 3]."""
    c0, c1, c2, c3 = sh_constants()
    x, y, z = d[..., 0], d[..., 1], d[..., 2]
    out = [np.full_like(x, c0)]
    if degree >= 1:
        out += [-c1 * y, c1 * z, -c1 * x]
    if degree >= 2:
        xx, yy, zz = x * x, y * y, z * z
        out += [c2[0] * x * y, c2[1] * y * z, c2[2] * (2 * zz - xx - yy), c2[3] * x * z, c2[4] * (xx - yy)]
    if degree >= 3:
        xx, yy, zz = x * x, y * y, z * z
        out += [c3[0] * y * (3 * xx - yy), c3[1] * x * y * z, c3[2] * y * (4 * zz - xx - yy),
                c3[3] * z * (2 * zz - 3 * xx - 3 * yy), c3[4] * x * (4 * zz - xx - yy), c3[5] * z * (xx - yy),
                c3[6] * x * (xx - 3 * yy)]
    return np.stack(out, -1)


def rotation(q) -> np.ndarray:
    """Rotation matrix of the quaternion (w, x, y, z) after normalisation."""
    w, x, y, z = np.asarray(q, np.float64) / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def project(mean, log_scale, quat, projmat, W, H, cx, cy):
    """Returns (T [3,3], normal [3]): T maps (u, v, 1) on the splat plane to
    homogeneous pixel coordinates (pixel centres at integers)."""
    R = rotation(quat)
    s = np.exp(np.asarray(log_scale, np.float64))
    M = np.zeros((4, 3))
    M[:3, 0] = R[:, 0] * s[0]
    M[:3, 1] = R[:, 1] * s[1]
    M[:3, 2] = mean
    M[3, 2] = 1.0
    A = np.array([[W / 2.0, 0, 0, cx - 0.5], [0, H / 2.0, 0, cy - 0.5], [0, 0, 0, 1.0]])
    T = A @ np.asarray(projmat, np.float64).reshape(4, 4) @ M
    return T, R[:, 2]


def sh_color(mean, cam_pos, fdc, frest, degree):
    d = np.asarray(mean, np.float64) - np.asarray(cam_pos, np.float64)
    d /= np.linalg.norm(d)
    coeffs = np.concatenate([np.asarray(fdc, np.float64)[None], np.asarray(frest, np.float64).reshape(-1, 3)])
    basis = sh_basis(d, degree)
    return basis @ coeffs[: basis.shape[-1]]


def _extreme(fn, theta0, width, rounds=4, samples=257):
    """Maximises fn(theta) [m, k] over each row's window around theta0 by
    repeated grid zooming; returns the maxima [m]."""
    best_t = theta0
    for _ in range(rounds):
        ts = best_t[:, None] + np.linspace(-width, width, samples)[None, :]
        v = fn(ts)
        i = np.argmax(v, axis=1)
        best_t = ts[np.arange(len(ts)), i]
        width = 2.0 * width / (samples - 1)
    return fn(best_t[:, None])[:, 0]


def circle_footprint(T, r=3.0, samples=4096):
    """Bounding box of the circle u^2 + v^2 = r^2 mapped through the
    homographies T [m,3,3] to pixels: (centre [m,2], half extent [m,2]).
    Only valid where the whole circle is in front (T[2] . (u,v,1) > 0)."""
    T = np.asarray(T, np.float64)

    def coord(ts, row):
        u, v = r * np.cos(ts), r * np.sin(ts)
        h = T[:, row, 0, None] * u + T[:, row, 1, None] * v + T[:, row, 2, None]
        w = T[:, 2, 0, None] * u + T[:, 2, 1, None] * v + T[:, 2, 2, None]
        return h / w

    grid = np.linspace(0.0, 2 * np.pi, samples, endpoint=False)[None, :].repeat(len(T), 0)
    out_c, out_e = [], []
    for row in (0, 1):
        vals = coord(grid, row)
        hi = _extreme(lambda ts: coord(ts, row), grid[0, np.argmax(vals, 1)], 2 * np.pi / samples)
        lo = -_extreme(lambda ts: -coord(ts, row), grid[0, np.argmin(vals, 1)], 2 * np.pi / samples)
        out_c.append(0.5 * (hi + lo))
        out_e.append(0.5 * (hi - lo))
    return np.stack(out_c, 1), np.stack(out_e, 1)


def composite(px, py, splats, background, near=0.2, far=100.0):
    """Front-to-back compositing of one pixel over `splats` (already in
    depth order): each a dict(T, xy, opac_logit, color_raw, normal).
    Returns dict of the per-pixel outputs and `lowpass`, the number of
    contributing splats that took the screen-space low-pass branch."""
    Tr = 1.0
    col = np.zeros(3)
    dep = 0.0
    nrm = np.zeros(3)
    M1 = M2 = dist = 0.0
    med = 0.0
    lowpass_used = 0
    for s in splats:
        T = s["T"]
        k = T[0] - px * T[2]
        l = T[1] - py * T[2]
        A2 = np.array([[k[0], k[1]], [l[0], l[1]]])
        if abs(np.linalg.det(A2)) == 0.0:
            continue
        u, v = np.linalg.solve(A2, -np.array([k[2], l[2]]))
        rho3 = u * u + v * v
        d = np.asarray(s["xy"], np.float64) - (px, py)
        rho2 = 2.0 * (d @ d)
        depth = T[2] @ (u, v, 1.0)
        if depth < near:
            continue
        opa = 1.0 / (1.0 + math.exp(-s["opac_logit"]))
        alpha = min(0.99, opa * math.exp(-0.5 * min(rho3, rho2)))
        if alpha < 1.0 / 255.0:
            continue
        if Tr * (1.0 - alpha) <= 1e-4:
            break
        lowpass_used += int(rho3 > rho2)
        w = alpha * Tr
        m = far / (far - near) * (1.0 - near / depth)
        dist += (m * m * (1.0 - Tr) + M2 - 2.0 * m * M1) * w
        M1 += m * w
        M2 += m * m * w
        if Tr > 0.5:
            med = depth
        col += np.maximum(np.asarray(s["color_raw"], np.float64) + 0.5, 0.0) * w
        dep += depth * w
        nrm += np.asarray(s["normal"], np.float64) * w
        Tr *= 1.0 - alpha
    return dict(img=col + np.asarray(background, np.float64) * Tr, depth=dep, normal=nrm, alpha=1.0 - Tr,
                median=med, distortion=dist, lowpass=lowpass_used)


def gaussian_window() -> np.ndarray:
    x = np.arange(11) - 5.0
    g = np.exp(-x * x / (2.0 * 1.5 * 1.5))
    g /= g.sum()
    return np.outer(g, g)


def blur2d(img: np.ndarray) -> np.ndarray:
    """Explicit 2D 11x11 window, zero padding, per channel."""
    w = gaussian_window()
    H, W = img.shape[:2]
    pad = np.zeros((H + 10, W + 10) + img.shape[2:])
    pad[5:5 + H, 5:5 + W] = img
    out = np.zeros_like(img, dtype=np.float64)
    for dy in range(11):
        for dx in range(11):
            out += w[dy, dx] * pad[dy:dy + H, dx:dx + W]
    return out


def ssim_map(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    C1, C2 = 0.01 ** 2, 0.03 ** 2
    mu1, mu2 = blur2d(a), blur2d(b)
    s11 = blur2d(a * a) - mu1 * mu1
    s22 = blur2d(b * b) - mu2 * mu2
    s12 = blur2d(a * b) - mu1 * mu2
    return ((2 * mu1 * mu2 + C1) * (2 * s12 + C2)) / ((mu1 * mu1 + mu2 * mu2 + C1) * (s11 + s22 + C2))


def loss(img, gt, lam=0.2):
    img = img.astype(np.float64)
    gt = gt.astype(np.float64)
    return (1.0 - lam) * np.abs(img - gt).mean() + lam * (1.0 - ssim_map(img, gt).mean())


# ---- 3DGS (EWA splatting, Zwicker et al. 2002; Kerbl et al. 2023) ----------
def ewa_project(mean, log_scale, quat, viewmat, projmat, fx, fy, W, H, cx, cy):
    """fp64 projection of a 3D Gaussian: (xy [2], cov2d [2,2], conic [2,2],
    depth).  The 2D covariance is J W Sigma W^T J^T + 0.3 I with the
    perspective Jacobian J at the view-space mean (its x/z, y/z clamped to
    1.3 tan(fov/2), as the reference's helper does), Sigma = R S S^T R^T."""
    V = np.asarray(viewmat, np.float64).reshape(4, 4)
    P = np.asarray(projmat, np.float64).reshape(4, 4)
    m = np.asarray(mean, np.float64)
    pv = V[:3, :3] @ m + V[:3, 3]
    R = rotation(quat)
    S = np.diag(np.exp(np.asarray(log_scale, np.float64)))
    Sigma = R @ S @ S.T @ R.T
    tx, ty = 0.5 * W / fx, 0.5 * H / fy
    x = pv[2] * np.clip(pv[0] / pv[2], -1.3 * tx, 1.3 * tx)
    y = pv[2] * np.clip(pv[1] / pv[2], -1.3 * ty, 1.3 * ty)
    z = pv[2]
    J = np.array([[fx / z, 0.0, -fx * x / (z * z)], [0.0, fy / z, -fy * y / (z * z)]])
    Wr = V[:3, :3]
    cov2d = J @ Wr @ Sigma @ Wr.T @ J.T + 0.3 * np.eye(2)
    h = P @ np.append(m, 1.0)
    xy = np.array([0.5 * W * h[0] / (h[3] + 1e-6) + cx - 0.5, 0.5 * H * h[1] / (h[3] + 1e-6) + cy - 0.5])
    return xy, cov2d, np.linalg.inv(cov2d), z


def composite3d(px, py, splats, background):
    """fp64 front-to-back compositing of 3D Gaussians at pixel (px, py):
    alpha = min(0.99, sigmoid(opacity) exp(-0.5 d^T C d)), d = centre -
    pixel; skipped when the exponent is positive or alpha < 1/255, stopping
    before the transmittance falls to 1e-4 (the fork's blending rules)."""
    T = 1.0
    col = np.zeros(3)
    for s in splats:
        d = np.asarray(s["xy"], np.float64) - np.array([px, py])
        C = np.asarray(s["conic"], np.float64)
        rho = d @ C @ d
        if rho < 0:
            continue
        alpha = min(0.99, 1.0 / (1.0 + math.exp(-s["opac_logit"])) * math.exp(-0.5 * rho))
        if alpha < 1.0 / 255.0:
            continue
        nT = T * (1.0 - alpha)
        if nT <= 1e-4:
            break
        col += np.maximum(np.asarray(s["color_raw"], np.float64) + 0.5, 0.0) * alpha * T
        T = nT
    return col + np.asarray(background, np.float64) * T, T
