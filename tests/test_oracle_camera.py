"""Pins the golden model's camera set-up and splat footprint against models
that share no code or formula with it:

  orc_prepare_cam (core/src/model.cpp:500-544)
      -> a pinhole camera written from cam_to_world: X_c = F R^T (X - t)
         with F = diag(1, -1, -1) (OpenGL -> OpenCV), pixel =
         f * X_c / Z_c + c - 0.5 (pixel centres at integers).  The oracle's
         projmat, pushed through the NDC -> pixel map of
         compute_transmat_2dgs (msplat_metal.metal:226-295), must land on
         the same pixel; its viewmat must give X_c and its depth Z_c.
  compute_aabb_2dgs (msplat_metal.metal:302-330, radius rule :1470-1478)
      -> the circle u^2 + v^2 = 9 on the splat plane, sampled densely and
         mapped through the splat's homography T to pixels: the centre of
         its bounding box is xys, ceil(max(extent, 3 * 0.707106)) is the
         radius.

Each check is shown to be live: a planted slip (fovX and fovY swapped, the
y/z flip dropped, a cutoff of 2 instead of 3) is rejected.
"""
import math

import numpy as np
import pytest

from msplat import synthetic as S
import refmath as R
from scenes import adversarial

F_CV = np.diag([1.0, -1.0, -1.0])


def _rand_rotation(rng):
    q = rng.normal(size=4)
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _cameras():
    """Orbit cameras of the workloads plus off-axis cameras with W != H,
    fx != fy and a principal point away from the image centre."""
    cams = []
    for c in S.orbit_cameras(5, 4.0, 20.0, 1297, 840):
        cams.append((c.cam_to_world.astype(np.float64), c.fx, c.fy, c.cx, c.cy, c.width, c.height))
    rng = np.random.default_rng(5)
    for k in range(6):
        c2w = np.eye(4)
        c2w[:3, :3] = _rand_rotation(rng)
        c2w[:3, 3] = rng.uniform(-3, 3, 3)
        W, H = int(rng.integers(64, 2000)), int(rng.integers(48, 1500))
        fx, fy = rng.uniform(0.4, 2.0) * W, rng.uniform(0.4, 2.0) * H
        cx, cy = W * rng.uniform(0.3, 0.7), H * rng.uniform(0.3, 0.7)
        cams.append((c2w, fx, fy, cx, cy, W, H))
    return cams


def _pinhole(c2w, fx, fy, cx, cy, X):
    """(pixel [n,2], Z_c [n]) of world points X [n,3] under the pinhole model."""
    R, t = c2w[:3, :3], c2w[:3, 3]
    Xc = (F_CV @ R.T @ (X - t).T).T
    return np.stack([fx * Xc[:, 0] / Xc[:, 2] + cx - 0.5, fy * Xc[:, 1] / Xc[:, 2] + cy - 0.5], 1), Xc


def _via_projmat(projmat, W, H, cx, cy, X):
    """Pixels of X through a row-major world -> clip matrix and the NDC ->
    pixel map halfW * x_clip / w_clip + (cx - 0.5) of the projection."""
    P = np.asarray(projmat, np.float64).reshape(4, 4)
    clip = (P @ np.c_[X, np.ones(len(X))].T).T
    return np.stack([0.5 * W * clip[:, 0] / clip[:, 3] + cx - 0.5,
                     0.5 * H * clip[:, 1] / clip[:, 3] + cy - 0.5], 1), clip[:, 3]


def _points_in_view(c2w, fx, fy, cx, cy, W, H, n, rng):
    """World points whose pinhole pixel lies in the image at depths 0.2..50."""
    R, t = c2w[:3, :3], c2w[:3, 3]
    px = rng.uniform(-0.5, W - 0.5, n)
    py = rng.uniform(-0.5, H - 0.5, n)
    z = np.exp(rng.uniform(math.log(0.2), math.log(50.0), n))
    Xc = np.stack([(px - cx + 0.5) / fx * z, (py - cy + 0.5) / fy * z, z], 1)
    return (R @ F_CV @ Xc.T).T + t


def _projmat_error(cam, c2w, fx, fy, cx, cy, W, H, X, projmat=None):
    """Largest pixel error of the projmat path against the pinhole, in units
    of a per-point bound: 1e-4 px plus the fp32 rounding the set-up carries
    (about 1e-6 relative on the camera-space coordinates, so the error
    scales with f * (1 + |t| + |X|) / Z, and on the offset from the
    principal point)."""
    pix, Xc = _pinhole(c2w, fx, fy, cx, cy, X)
    got, w = _via_projmat(cam.projmat if projmat is None else projmat, W, H, cx, cy, X)
    f = max(fx, fy)
    size = 1.0 + np.abs(c2w[:3, 3]).max() + np.abs(X).max(1)
    tol = 1e-4 + 1e-6 * (f * size / Xc[:, 2] + np.abs(pix - np.array([cx, cy])).max(1))
    return (np.abs(got - pix).max(1) / tol).max(), Xc, w


def test_prepare_cam_is_a_pinhole_camera(orc):
    rng = np.random.default_rng(1)
    for c2w, fx, fy, cx, cy, W, H in _cameras():
        cam = orc.prepare_cam(c2w.astype(np.float32), fx, fy, cx, cy, W, H)
        c2w32 = c2w.astype(np.float32).astype(np.float64)
        X = _points_in_view(c2w32, fx, fy, cx, cy, W, H, 4000, rng)
        err, Xc, w = _projmat_error(cam, c2w32, fx, fy, cx, cy, W, H, X)
        assert err <= 1.0, (W, H, err)
        # the clip w is the camera-space depth, and the viewmat is R^T, -R^T t
        # in OpenCV axes
        V = np.asarray(cam.viewmat, np.float64).reshape(4, 4)
        assert np.abs(w - Xc[:, 2]).max() <= 2e-5 * Xc[:, 2].max()
        assert np.abs((V @ np.c_[X, np.ones(len(X))].T).T[:, :3] - Xc).max() <= 2e-5 * np.abs(Xc).max()
        assert np.allclose(cam.cam_pos, c2w32[:3, 3], rtol=0, atol=0)
        assert (cam.tiles_x, cam.tiles_y) == ((W + 15) // 16, (H + 15) // 16)


def test_prepare_cam_check_is_live(orc):
    """Slips of prepare_cam that the pinhole check must reject: fovX and
    fovY swapped (W != H), and a projection without the y/z flip."""
    rng = np.random.default_rng(2)
    c2w, fx, fy, cx, cy, W, H = _cameras()[-1]
    assert abs(W / fx - H / fy) > 0.05
    cam = orc.prepare_cam(c2w.astype(np.float32), fx, fy, cx, cy, W, H)
    c2w32 = c2w.astype(np.float32).astype(np.float64)
    X = _points_in_view(c2w32, fx, fy, cx, cy, W, H, 1000, rng)
    P = np.asarray(cam.projmat, np.float64).reshape(4, 4)
    swapped = P.copy()
    sx, sy = 2 * fx / W, 2 * fy / H
    swapped[0] *= sy / sx
    swapped[1] *= sx / sy
    assert _projmat_error(cam, c2w32, fx, fy, cx, cy, W, H, X, swapped)[0] > 100.0
    noflip = P.copy()
    noflip[1] *= -1.0
    noflip[3] *= -1.0
    assert _projmat_error(cam, c2w32, fx, fy, cx, cy, W, H, X, noflip)[0] > 100.0


def test_points_behind_the_camera_are_culled(orc):
    """Splats at camera depth <= clip_thresh (0.01) get radius 0 and no tile;
    the same splats just in front of it are kept."""
    c2w, fx, fy, cx, cy, W, H = _cameras()[7]
    cam = orc.prepare_cam(c2w.astype(np.float32), fx, fy, cx, cy, W, H)
    R, t = c2w[:3, :3], c2w[:3, 3]
    n = 64
    z = np.r_[np.linspace(-3.0, 0.0, n // 2), np.linspace(0.05, 2.0, n // 2)]
    Xc = np.stack([0.01 * z, 0.01 * z, z], 1)
    means = ((R @ F_CV @ Xc.T).T + t).astype(np.float32)
    scene = S.make_scene(1, n=n, width=W, height=H)
    params = dict(means=means, scales=np.full((n, 2), -4.0, np.float32), quats=scene.quats,
                  opacities=scene.opacities, features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = orc.project_fwd(params, cam, 0, 0)
    depth = Xc[:, 2]
    assert np.all(proj["radii"][depth <= 0.01] == 0)
    assert np.all(proj["radii"][depth > 0.05] > 0)
    assert np.allclose(proj["depths"][depth > 0.05], depth[depth > 0.05], rtol=2e-5)


# ------------------------------------------------------------- AABB ------
def _aabb_scenes():
    out = []
    s = S.make_scene(2, n=3000, width=333, height=217, num_cameras=2)
    out.append(("blob", s))
    out.append(("adversarial", adversarial(3000, 31, width=200, height=136)))
    s = S.make_scene(1, n=2000, width=256, height=256)
    out.append(("uniform", s))
    return out


def _footprint_mismatches(T, xys, radii, ctr, ext):
    """(centre wrong, radius wrong, radius ambiguous) per splat.  The fp32
    half extent sqrt(c^2 - f.(T0*T0)) cancels when the centre c is large
    against the extent: its error is about 3e-7 * c^2 / extent, so a radius
    whose exact extent lies that close to an integer is ambiguous."""
    scale = np.maximum(1.0, np.abs(ext).max(1))
    ctr_bad = np.abs(xys - ctr).max(1) > 1e-3 * scale
    want = np.maximum(ext.max(1), 3.0 * 0.707106)
    amb = 1e-6 * scale + 3e-7 * (ctr * ctr).max(1) / np.maximum(ext.max(1), 1.0)
    near_int = np.abs(want - np.round(want)) <= amb
    rad_bad = (radii != np.ceil(want)) & ~near_int
    return ctr_bad, rad_bad, near_int


@pytest.mark.parametrize("name,scene", _aabb_scenes())
def test_aabb_is_the_footprint_of_the_3_sigma_circle(orc, name, scene):
    c = scene.cameras[0]
    cam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                  features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = orc.project_fwd(params, cam, scene.sh_degree, scene.sh_degree)
    T = proj["transmats"].reshape(-1, 3, 3).astype(np.float64)
    vis = proj["radii"] > 0
    # an ellipse only when the whole 3-sigma circle is in front of the camera
    front = T[:, 2, 2] > 3.0 * np.hypot(T[:, 2, 0], T[:, 2, 1]) * (1 + 1e-6)
    sel = np.flatnonzero(vis & front)
    assert sel.size > 200, sel.size
    ctr, ext = R.circle_footprint(T[sel])
    ctr_bad, rad_bad, amb = _footprint_mismatches(T[sel], proj["xys"][sel], proj["radii"][sel], ctr, ext)
    assert ctr_bad.sum() == 0, (name, np.abs(proj["xys"][sel] - ctr).max())
    assert rad_bad.sum() == 0, name
    assert amb.mean() < 0.02, (name, amb.mean())
    # live: an oracle with a cutoff of 2 would be rejected on most splats
    ctr2, ext2 = R.circle_footprint(T[sel], r=2.0)
    ctr_bad2, rad_bad2, _ = _footprint_mismatches(T[sel], ctr2, np.ceil(np.maximum(ext2.max(1), 2 * 0.707106)),
                                               ctr, ext)
    assert rad_bad2.mean() > 0.3 and (ctr_bad2 | rad_bad2).mean() > 0.3, name
