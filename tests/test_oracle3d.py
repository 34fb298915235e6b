"""The golden model's 3DGS mode, pinned by independent fp64 derivations:

  projection     -> refmath.ewa_project (matrix-form EWA: J W Sigma W^T J^T
                    + 0.3 I, explicit inverse, homogeneous projection) and a
                    closed form for a Gaussian on the optical axis;
  compositing    -> refmath.composite3d, and a single-Gaussian closed form;
  raster bwd     -> central finite differences of that fp64 compositing;
  project bwd    -> central finite differences of refmath.ewa_project and
                    the real-SH colour.
The fork's own 3DGS compositing kernel was removed, so these pins, not a
reference run, are what fixes the mode (its helpers, msplat_metal.metal:
152-459 and 1059-1374, are transcribed in the oracle).
"""
import math

import numpy as np
import pytest

import refmath as R


def _scene3d(seed=0, n=6, W=48, H=40, spread=0.25, log_s=(-2.2, -1.6)):
    """n 3D Gaussians in front of a camera 3 units away (OpenGL pose)."""
    rng = np.random.default_rng(seed)
    p = dict(means=np.column_stack([rng.uniform(-spread, spread, n), rng.uniform(-spread, spread, n),
                                    rng.uniform(-0.4, 0.4, n)]),
             scales=rng.uniform(log_s[0], log_s[1], (n, 3)),
             quats=rng.normal(0, 1, (n, 4)),
             opacities=rng.uniform(-1.0, 1.0, (n, 1)),
             features_dc=rng.uniform(-1.2, 1.2, (n, 3)),
             features_rest=rng.normal(0, 0.15, (n, 15, 3)))
    p["quats"] /= np.linalg.norm(p["quats"], axis=1, keepdims=True)
    p = {k: v.astype(np.float32) for k, v in p.items()}
    c2w = np.eye(4, dtype=np.float32)
    c2w[2, 3] = 3.0
    f = 1.1 * W
    return p, dict(c2w=c2w, fx=f, fy=f * 1.05, cx=W / 2 + 0.7, cy=H / 2 - 0.4, W=W, H=H)


def _cam(orc, c):
    return orc.prepare_cam(c["c2w"], c["fx"], c["fy"], c["cx"], c["cy"], c["W"], c["H"])


def test_project3d_matches_fp64_ewa(orc):
    p, c = _scene3d(1, n=40, W=96, H=72, spread=0.6)
    cam = _cam(orc, c)
    out = orc.project3d_fwd(p, cam, 3, 3)
    vis = np.flatnonzero(out["radii"] > 0)
    assert vis.size >= 30
    for i in vis:
        xy, cov2d, conic, z = R.ewa_project(p["means"][i], p["scales"][i], p["quats"][i], cam.viewmat, cam.projmat,
                                            c["fx"], c["fy"], c["W"], c["H"], c["cx"], c["cy"])
        assert np.abs(out["xys"][i] - xy).max() < 2e-4
        assert out["depths"][i] == pytest.approx(z, rel=1e-6)
        c2 = np.array([cov2d[0, 0], cov2d[0, 1], cov2d[1, 1]])
        assert np.abs(out["cov2d"][i] - c2).max() <= 2e-5 * np.abs(c2).max()
        cn = np.array([conic[0, 0], conic[0, 1], conic[1, 1]])
        assert np.abs(out["conics"][i] - cn).max() <= 2e-4 * np.abs(cn).max()
        # 3-sigma radius of the larger eigenvalue, the reference's formula
        b = 0.5 * (c2[0] + c2[2])
        lam = b + math.sqrt(max(0.1, b * b - np.linalg.det(cov2d)))
        r = 3.0 * math.sqrt(lam)
        if abs(r - round(r)) > 1e-3:
            assert out["radii"][i] == math.ceil(r)
        col = R.sh_color(p["means"][i], cam.cam_pos, p["features_dc"][i], p["features_rest"][i], 3)
        assert np.abs(out["colors"][i] - col).max() < 2e-5


def test_project3d_on_axis_closed_form(orc):
    """An isotropic Gaussian of scale s on the optical axis at depth z:
    centre (cx - 0.5, cy - 0.5), cov2d = diag((fx s / z)^2, (fy s / z)^2) +
    0.3, conic its inverse; slips in the Jacobian's focal lengths or the
    low-pass term fail it."""
    p, c = _scene3d(0, n=1)
    s = 0.07
    p["means"][0] = [0.0, 0.0, 0.5]
    p["scales"][0] = [math.log(s)] * 3
    cam = _cam(orc, c)
    out = orc.project3d_fwd(p, cam, 3, 0)
    z = 3.0 - 0.5
    vx, vy = (c["fx"] * s / z) ** 2 + 0.3, (c["fy"] * s / z) ** 2 + 0.3
    assert np.abs(out["xys"][0] - [c["cx"] - 0.5, c["cy"] - 0.5]).max() < 1e-4
    assert out["cov2d"][0] == pytest.approx([vx, 0.0, vy], rel=1e-5, abs=1e-6)
    assert out["conics"][0] == pytest.approx([1 / vx, 0.0, 1 / vy], rel=1e-5, abs=1e-7)
    # compute_cov2d_bounds floors the eigenvalue gap at sqrt(0.1)
    b = 0.5 * (vx + vy)
    assert out["radii"][0] == math.ceil(3 * math.sqrt(b + math.sqrt(max(0.1, b * b - vx * vy))))


def _render3d(orc, p, c, bg):
    cam = _cam(orc, c)
    proj = orc.project3d_fwd(p, cam, 3, 3)
    bins = orc.bin_sort(proj, cam)
    fwd = orc.raster3d_fwd(proj, bins, cam, p["opacities"], bg)
    return cam, proj, bins, fwd


def _fp64_render3d(proj, bins, cam, bg, op, xy_over=None, conic_over=None, op_over=None, col_over=None):
    H, W = cam.height, cam.width
    img = np.zeros((H, W, 3))
    for py in range(H):
        for px in range(W):
            t = (py // 16) * cam.tiles_x + px // 16
            lst = bins["ids"][bins["tile_offsets"][t]:bins["tile_offsets"][t + 1]]
            sp = []
            for g in lst:
                cn = conic_over[g] if conic_over is not None else proj["conics"][g].astype(np.float64)
                sp.append(dict(xy=xy_over[g] if xy_over is not None else proj["xys"][g],
                               conic=np.array([[cn[0], cn[1]], [cn[1], cn[2]]]),
                               opac_logit=op_over[g] if op_over is not None else float(op[g, 0]),
                               color_raw=col_over[g] if col_over is not None else proj["colors"][g]))
            img[py, px] = R.composite3d(px, py, sp, bg)[0]
    return img


def test_raster3d_forward_matches_fp64_compositing(orc):
    p, c = _scene3d(2, n=8)
    bg = np.float32([0.3, 0.1, 0.6])
    cam, proj, bins, fwd = _render3d(orc, p, c, bg)
    ref = _fp64_render3d(proj, bins, cam, bg, p["opacities"])
    assert bins["num_intersections"] > 8
    assert np.abs(fwd["out_img"] - ref).max() < 2e-5


def test_raster3d_single_gaussian_closed_form(orc):
    p, c = _scene3d(3, n=1, W=32, H=32)
    p["means"][0] = [0.02, -0.01, 0.0]
    p["opacities"][0] = 1.3
    bg = np.float32([0.2, 0.2, 0.2])
    cam, proj, bins, fwd = _render3d(orc, p, c, bg)
    C = proj["conics"][0].astype(np.float64)
    Cm = np.array([[C[0], C[1]], [C[1], C[2]]])
    col = np.maximum(proj["colors"][0].astype(np.float64) + 0.5, 0)
    op = 1 / (1 + math.exp(-1.3))
    ys, xs = np.mgrid[0:32, 0:32]
    d = np.stack([proj["xys"][0, 0] - xs, proj["xys"][0, 1] - ys], -1).astype(np.float64)
    a = np.minimum(0.99, op * np.exp(-0.5 * np.einsum("hwi,ij,hwj->hw", d, Cm, d)))
    a = np.where(a >= 1 / 255, a, 0.0)
    # only pixels in the splat's tiles see it
    r = proj["rect"][0]
    inr = (xs // 16 >= r[0]) & (xs // 16 < r[2]) & (ys // 16 >= r[1]) & (ys // 16 < r[3])
    a = np.where(inr, a, 0.0)
    exp_img = a[..., None] * col + (1 - a[..., None]) * bg
    assert np.abs(fwd["out_img"] - exp_img).max() < 3e-6
    assert np.abs(fwd["final_T"] - (1 - a)).max() < 3e-6


def test_raster3d_backward_matches_finite_differences(orc):
    p, c = _scene3d(4, n=5, W=36, H=30)
    bg = np.float32([0.4, 0.5, 0.3])
    cam, proj, bins, fwd = _render3d(orc, p, c, bg)
    H, W = cam.height, cam.width
    rng = np.random.default_rng(9)
    up = (rng.normal(size=(H, W, 3)) * 0.01).astype(np.float32)
    g = orc.raster3d_bwd(proj, bins, fwd, cam, p["opacities"], bg, up)
    n = proj["radii"].shape[0]
    xy0 = [proj["xys"][i].astype(np.float64) for i in range(n)]
    cn0 = [proj["conics"][i].astype(np.float64) for i in range(n)]
    op0 = [float(p["opacities"][i, 0]) for i in range(n)]
    co0 = [proj["colors"][i].astype(np.float64) for i in range(n)]

    def L(xy=xy0, cn=cn0, op=op0, co=co0):
        return float((_fp64_render3d(proj, bins, cam, bg, p["opacities"], xy, cn, op, co) * up).sum())

    def fd(lst, i, k, h):
        a = [x.copy() if hasattr(x, "copy") else x for x in lst]
        b = [x.copy() if hasattr(x, "copy") else x for x in lst]
        if isinstance(a[i], float):
            a[i] += h
            b[i] -= h
        else:
            a[i][k] += h
            b[i][k] -= h
        return a, b

    scale = max(1.0, float(np.abs(g).max()))
    for i in range(n):
        if proj["radii"][i] == 0:
            continue
        for k in range(2):
            a, b = fd(xy0, i, k, 1e-5)
            f = (L(xy=a) - L(xy=b)) / 2e-5
            assert g[i, k] == pytest.approx(f, rel=3e-3, abs=3e-7 * scale), ("xy", i, k)
        for k in range(3):
            h = 1e-6 * max(1.0, abs(cn0[i][k]))
            a, b = fd(cn0, i, k, h)
            f = (L(cn=a) - L(cn=b)) / (2 * h)
            # the off-diagonal entry is the derivative by one of the two
            # symmetric matrix entries (half the scalar's)
            want = 0.5 * f if k == 1 else f
            assert g[i, 2 + k] == pytest.approx(want, rel=3e-3, abs=3e-7 * scale), ("conic", i, k)
        a, b = fd(op0, i, 0, 1e-6)
        f = (L(op=a) - L(op=b)) / 2e-6
        assert g[i, 5] == pytest.approx(f, rel=3e-3, abs=1e-7), ("opacity", i)
        for ch in range(3):
            a, b = fd(co0, i, ch, 1e-6)
            f = (L(co=a) - L(co=b)) / 2e-6
            assert g[i, 6 + ch] == pytest.approx(f, rel=3e-3, abs=1e-7), ("color", i, ch)


def test_project3d_backward_matches_finite_differences(orc):
    p, c = _scene3d(5, n=10, W=96, H=72, spread=0.5)
    cam = _cam(orc, c)
    proj = orc.project3d_fwd(p, cam, 3, 3)
    vis = np.flatnonzero(proj["radii"] > 0)
    assert vis.size >= 6
    rng = np.random.default_rng(3)
    g9 = rng.normal(size=(len(proj["radii"]), 9)).astype(np.float32)
    out = orc.project3d_bwd(p, cam, 3, 3, proj["radii"], g9)

    def L(i, mean, ls, q, fdc, frest):
        xy, _, conic, _ = R.ewa_project(mean, ls, q, cam.viewmat, cam.projmat, c["fx"], c["fy"], c["W"], c["H"],
                                        c["cx"], c["cy"])
        col = R.sh_color(mean, cam.cam_pos, fdc, frest, 3)
        # g9[3] is the derivative by one symmetric entry: the scalar's is 2 g9[3]
        return float(xy @ g9[i, :2] + conic[0, 0] * g9[i, 2] + 2 * conic[0, 1] * g9[i, 3] + conic[1, 1] * g9[i, 4]
                     + col @ g9[i, 6:9])

    for i in vis[:6]:
        base = [p["means"][i].astype(np.float64), p["scales"][i].astype(np.float64),
                p["quats"][i].astype(np.float64), p["features_dc"][i].astype(np.float64),
                p["features_rest"][i].astype(np.float64)]

        def fd(which, k, h=1e-6):
            a = [b.copy() for b in base]
            b_ = [b.copy() for b in base]
            a[which].reshape(-1)[k] += h
            b_[which].reshape(-1)[k] -= h
            return (L(i, *a) - L(i, *b_)) / (2 * h)

        for k in range(3):
            f = fd(0, k)
            assert out["dmeans"][i, k] == pytest.approx(f, rel=3e-3, abs=3e-4 * max(1.0, abs(f))), ("mean", i, k)
        for k in range(3):
            f = fd(1, k)
            assert out["dscales"][i, k] == pytest.approx(f, rel=3e-3, abs=2e-4), ("scale", i, k)
        qn = base[2] / np.linalg.norm(base[2])
        gq = out["dquats"][i].astype(np.float64)
        gq_tan = (gq - qn * (qn @ gq)) / np.linalg.norm(base[2])
        fdq = np.array([fd(2, k) for k in range(4)])
        assert np.abs(gq_tan - fdq).max() <= 3e-3 * np.abs(fdq).max() + 2e-4, ("quat", i)
        for k in range(3):
            assert out["dfdc"][i, k] == pytest.approx(fd(3, k), rel=2e-3, abs=1e-6)
        for k in (0, 7, 20, 44):
            assert out["dfrest"][i].reshape(-1)[k] == pytest.approx(fd(4, k), rel=2e-3, abs=1e-6)
        # the densification statistic is dL/dxy in NDC units
        assert out["dmean2d"][i] == pytest.approx([g9[i, 0] * c["W"] / 2, g9[i, 1] * c["H"] / 2], rel=1e-6)


# ---- densification with three scales --------------------------------------
STRIDES3 = (3, 3, 4, 3, 45, 1)


def _dens_inputs(n=64, seed=5):
    rng = np.random.default_rng(seed)
    cap = 4 * n + 8
    p = dict(means=rng.uniform(-1, 1, (n, 3)), scales=rng.uniform(-4.5, -2.5, (n, 3)),
             quats=rng.normal(0, 1, (n, 4)), features_dc=rng.normal(0, 1, (n, 3)),
             features_rest=rng.normal(0, 0.1, (n, 45)), opacities=rng.uniform(-1, 3, (n, 1)))
    keys = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")
    params = []
    for k, s in zip(keys, STRIDES3):
        a = np.zeros(cap * s, np.float32)
        a[: n * s] = p[k].astype(np.float32).reshape(-1)
        params.append(a)
    m6 = [np.zeros(cap * s, np.float32) for s in STRIDES3]
    v6 = [np.zeros(cap * s, np.float32) for s in STRIDES3]
    stats = dict(grad_norm=rng.uniform(0, 0.004, n).astype(np.float32), vis=np.ones(n, np.float32),
                 max2d=rng.uniform(0, 0.1, n).astype(np.float32))
    rs = rng.normal(0, 1, (2 * n, 3)).astype(np.float32)
    return n, cap, params, m6, v6, stats, rs


def _quat_R(q):
    w, x, y, z = np.asarray(q, np.float64) / np.linalg.norm(np.asarray(q, np.float64))
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def test_densify3d_children_sampled_along_three_axes(orc):
    """Every split child sits at parent + R (r * exp(s)) with all three
    axes (the surfel form drops the third), carries the parent's scales
    minus log 1.6 on all three, and the split parent is culled."""
    n, cap, params, m6, v6, stats, rs = _dens_inputs()
    stats["grad_norm"][:] = 0.004  # all high-gradient
    stats["max2d"][:] = 0.0  # no split by screen size
    p0 = [a.copy() for a in params]
    new = orc.densify(n, cap, params, m6, v6, 45, stats, rs, size_thresh=0.05, check_huge=0, cull_alpha=0.0,
                      half_max_dim=100.0, scale_dim=3)
    sc0 = p0[1][: 3 * n].reshape(n, 3).astype(np.float64)
    large = np.exp(sc0).max(axis=1) > 0.05
    split = large
    ns, nd = int(split.sum()), int((~large).sum())
    assert 0 < ns < n and nd > 0
    assert new == n - ns + 2 * ns + nd
    # compaction keeps order: survivors (non-split originals), then children, then dups
    means = params[0][: 3 * new].reshape(new, 3).astype(np.float64)
    scales = params[1][: 3 * new].reshape(new, 3).astype(np.float64)
    m_orig = p0[0][: 3 * n].reshape(n, 3).astype(np.float64)
    q_orig = p0[2][: 4 * n].reshape(n, 4)
    base = n - ns
    ords = np.flatnonzero(split)
    third = []
    for o, i in enumerate(ords):
        R = _quat_R(q_orig[i])
        for k in range(2):
            c = base + 2 * o + k
            local = R.T @ (means[c] - m_orig[i])
            want = rs[2 * o + k].astype(np.float64) * np.exp(sc0[i])
            assert np.allclose(local, want, rtol=2e-4, atol=2e-6 * np.abs(m_orig[i]).max()), (i, k)
            third.append(abs(want[2]))
            assert np.allclose(scales[c], sc0[i] - math.log(1.6), atol=1e-6)
    assert max(third) > 1e-3  # the third axis moved children


def test_densify3d_third_scale_classifies_and_culls(orc):
    """A splat small in two axes but large in the third is split (large), not
    duplicated; with check_huge it is culled by the third scale alone."""
    n, cap, params, m6, v6, stats, rs = _dens_inputs(n=8)
    sc = params[1][: 3 * n].reshape(n, 3)
    sc[:, :] = np.log(0.001)
    sc[0, 2] = np.log(0.5)
    stats["grad_norm"][:] = 0.004
    stats["max2d"][:] = 0.0
    a = [x.copy() for x in params]
    new = orc.densify(n, cap, a, [x.copy() for x in m6], [x.copy() for x in v6], 45, stats, rs, size_thresh=0.02,
                      check_huge=0, cull_alpha=0.0, half_max_dim=100.0, scale_dim=3)
    assert new == (n - 1) + 2 + (n - 1)  # one split (two children), seven dups
    b = [x.copy() for x in params]
    sc_b = b[1][: 3 * n].reshape(n, 3)
    sc_b[0, 2] = np.log(0.9)
    stats["grad_norm"][:] = 0.0  # no densification, cull only
    new = orc.densify(n, cap, b, [x.copy() for x in m6], [x.copy() for x in v6], 45, stats, rs, check_huge=1,
                      cull_scale=0.5, cull_alpha=0.0, half_max_dim=100.0, scale_dim=3)
    assert new == n - 1
    assert np.array_equal(b[0][: 3 * (n - 1)], params[0][3: 3 * n])


def test_densify3d_reduces_to_surfels_when_the_third_scale_vanishes(orc):
    """With exp(third scale) = 0 the 3-scale densify equals the surfel one
    bit for bit on every other buffer (the offsets' third term is exactly 0)."""
    n, cap, params, m6, v6, stats, rs = _dens_inputs(n=96, seed=9)
    sc3 = params[1][: 3 * n].reshape(n, 3)
    sc3[:, 2] = -200.0
    assert orc.expf(-200.0) == 0.0
    two = [a.copy() for a in params]
    two[1] = np.zeros(cap * 2, np.float32)
    two[1][: 2 * n] = sc3[:, :2].reshape(-1)
    m2 = [np.zeros(cap * s, np.float32) for s in (3, 2, 4, 3, 45, 1)]
    v2 = [np.zeros(cap * s, np.float32) for s in (3, 2, 4, 3, 45, 1)]
    three = [a.copy() for a in params]
    n3 = orc.densify(n, cap, three, m6, v6, 45, stats, rs, half_max_dim=300.0, scale_dim=3)
    n2 = orc.densify(n, cap, two, m2, v2, 45, stats, rs, half_max_dim=300.0, scale_dim=2)
    assert n3 == n2 and n3 != n
    for g in (0, 2, 3, 4, 5):
        s = STRIDES3[g]
        assert np.array_equal(three[g][: n3 * s], two[g][: n3 * s]), g
    s3 = three[1][: 3 * n3].reshape(n3, 3)
    assert np.array_equal(s3[:, :2].reshape(-1), two[1][: 2 * n3])
