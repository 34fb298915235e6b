"""Pins the CPU golden model against what the mathematics fixes, so that a
plausible slip (a dropped term, a wrong sign or index, a transposed operand)
fails here.  The reference publishes no golden vectors for this path and its
Metal kernels cannot run on Linux, so each check is independent of the
oracle's code:

  exp            -> libm fp64 exp, ulp bound
  SH             -> closed-form real-SH constants + orthonormality on the sphere
  SSIM window    -> the reference's own tabulated weights (fixture) and the
                    closed form
  SSIM/L1 fwd    -> brute-force 2D 11x11 window in fp64
  loss bwd       -> central finite differences of the fp64 loss
  raster fwd     -> fp64 compositing with the intersection solved as a 2x2
                    linear system
  raster bwd     -> central finite differences of that fp64 forward
  project fwd    -> fp64 homography T = A P [t_u t_v p] and SH colour
  project bwd    -> central finite differences of the fp64 projection
  binning/sort   -> brute-force rectangle enumeration + lexicographic sort
  Adam           -> one-step closed form and an fp64 recurrence
  densify        -> a serial numpy restatement with stable partition
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import refmath as R

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- exp ----
def test_expf_within_one_ulp_of_libm(orc):
    x = np.concatenate([np.linspace(-103.9, 88.7, 400_001, dtype=np.float32),
                        np.float32([-0.0, 0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0, 88.0, -87.0, -100.0])])
    y = orc.expf_array(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    tiny = np.float64(np.finfo(np.float32).smallest_subnormal)
    err = np.abs(y - ref) / np.maximum(ulp, tiny)
    assert err.max() <= 1.0, float(err.max())


def test_expf_special_values(orc):
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-200.0) == 0.0
    assert math.isinf(orc.expf(100.0))
    assert math.isnan(orc.expf(float("nan")))
    assert orc.expf(-103.0) > 0.0  # subnormal range is kept


def test_gauss_accuracy(orc):
    """The rasterizer's Gaussian falloff exp(-rho / 2): within 8 ulp of exp
    where alpha can reach 1/255 (rho <= 11.2), within the rounding of its
    exponent up to rho = 160, exact at 0, clamped (never below 4e-38)
    further out, NaN treated like +inf, and monotone."""
    rho = np.linspace(0.0, 11.2, 400_001, dtype=np.float32)
    y = orc.gauss_array(rho).astype(np.float64)
    ref = np.exp(-0.5 * rho.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(y - ref) / ulp).max() <= 8.0
    # further out the exponent t = -rho log2(e) / 2 dominates: its rounding
    # (half an ulp of t) and the float log2(e) (1.34e-8 relative), each
    # times ln 2, relative
    rho = np.linspace(0.0, 160.0, 200_001, dtype=np.float32)
    y = orc.gauss_array(rho).astype(np.float64)
    ref = np.exp(-0.5 * rho.astype(np.float64))
    t = rho.astype(np.float64) * 0.72134752
    t_ulp = np.spacing(t.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y - ref) / ref <= 2.5e-7 + 0.4 * t_ulp + 1.0e-8 * t)
    assert orc.gauss(0.0) == 1.0
    # a plausible slip in the reduction (a dropped halving, a wrong-sign
    # exponent) is far outside these bounds
    assert abs(orc.gauss(2.0) - np.exp(-1.0)) <= 2e-7 * np.exp(-1.0)
    assert orc.gauss(1e9) >= 4e-38
    assert orc.gauss(float("inf")) >= 4e-38
    assert orc.gauss(float("nan")) == orc.gauss(float("inf"))
    # monotone non-increasing in rho on a dense grid (no reduction seams)
    rho = np.linspace(0.0, 40.0, 1_000_001, dtype=np.float32)
    y = orc.gauss_array(rho)
    assert np.all(np.diff(y.astype(np.float64)) <= 0.0)


# ----------------------------------------------------------------- SH ----
def test_sh_basis_is_orthonormal():
    # closed-form constants must give an orthonormal basis on the sphere
    n = 400_000
    i = np.arange(n) + 0.5
    z = 1 - 2 * i / n
    phi = np.pi * (1 + 5 ** 0.5) * i
    d = np.stack([np.sqrt(1 - z * z) * np.cos(phi), np.sqrt(1 - z * z) * np.sin(phi), z], -1)
    B = R.sh_basis(d, 3)
    gram = (B.T @ B) * (4 * np.pi / n)
    assert np.abs(gram - np.eye(16)).max() < 2e-3


def test_project_forward_matches_fp64_derivation(orc):
    from msplat import synthetic as S
    scene = S.make_scene(2, n=200, width=96, height=64, num_cameras=3)
    for ci in range(3):
        c = scene.cameras[ci]
        cam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
        params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                      features_dc=scene.features_dc, features_rest=scene.features_rest)
        proj = orc.project_fwd(params, cam, 3, 3)
        vis = np.flatnonzero(proj["radii"] > 0)
        assert vis.size > 50
        for i in vis:
            T, nrm = R.project(scene.means[i], scene.scales[i], scene.quats[i], cam.projmat, c.width, c.height,
                               c.cx, c.cy)
            scale = np.abs(T).max()
            assert np.abs(proj["transmats"][i].reshape(3, 3) - T).max() <= 2e-5 * scale
            assert np.abs(proj["normal_opac"][i, :3] - nrm).max() <= 2e-6
            col = R.sh_color(scene.means[i], cam.cam_pos, scene.features_dc[i], scene.features_rest[i], 3)
            assert np.abs(proj["colors"][i] - col).max() <= 2e-5
            assert np.abs(proj["xys"][i] - R.circle_footprint(T[None])[0][0]).max() <= 2e-3
            assert proj["depths"][i] == pytest.approx(T[2, 2], rel=1e-5)


def test_sh_degree_zero_is_c0_times_dc(orc):
    from msplat import synthetic as S
    scene = S.make_scene(1, n=300, width=64, height=64)
    c = scene.cameras[0]
    cam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                  features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = orc.project_fwd(params, cam, 0, 0)
    vis = proj["radii"] > 0
    c0 = np.float32(R.sh_constants()[0])
    assert np.array_equal(proj["colors"][vis], (c0 * scene.features_dc[vis]).astype(np.float32))


# --------------------------------------------------------------- SSIM ----
def test_ssim_window_matches_reference_table(orc):
    table = json.loads((GOLDEN / "ssim_window.json").read_text())["weights"]
    w = orc.ssim_window()
    assert np.abs(w - np.float32(table)).max() <= 1e-9
    x = np.arange(11) - 5.0
    g = np.exp(-x * x / 4.5)
    assert np.allclose(w, g / g.sum(), rtol=0, atol=2e-8)  # half a float32 ulp


@pytest.mark.parametrize("H,W", [(19, 23), (8, 40), (1, 1), (30, 30)])
def test_ssim_forward_matches_bruteforce(orc, H, W):
    from msplat import synthetic as S
    rng = S.SplitMix64(H * 100 + W)
    img = rng.uniform(H * W * 3).reshape(H, W, 3)
    gt = rng.uniform(H * W * 3).reshape(H, W, 3)
    loss, dL, _, ssim_sum = orc.loss_fwd_bwd(img, gt)
    ref_ssim = R.ssim_map(img, gt).sum()
    assert ssim_sum == pytest.approx(ref_ssim, rel=1e-5, abs=1e-5)
    assert loss == pytest.approx(R.loss(img, gt), rel=1e-5)


def test_loss_backward_matches_finite_differences(orc):
    from msplat import synthetic as S
    H, W = 14, 17
    rng = S.SplitMix64(3)
    img = rng.uniform(H * W * 3).reshape(H, W, 3).astype(np.float64)
    gt = rng.uniform(H * W * 3).reshape(H, W, 3).astype(np.float64)
    _, dL, _, _ = orc.loss_fwd_bwd(img, gt)
    eps = 1e-6
    picks = [(0, 0, 0), (5, 7, 1), (13, 16, 2), (7, 0, 0), (2, 9, 2), (10, 3, 1)]
    for (y, x, c) in picks:
        assert abs(img[y, x, c] - gt[y, x, c]) > 10 * eps
        a, b = img.copy(), img.copy()
        a[y, x, c] += eps
        b[y, x, c] -= eps
        fd = (R.loss(a, gt) - R.loss(b, gt)) / (2 * eps)
        assert dL[y, x, c] == pytest.approx(fd, rel=2e-3, abs=1e-9), (y, x, c)


# ------------------------------------------------- rasterize fwd / bwd ----
def _tiny_scene(seed=0, n=5, W=40, H=32):
    """A handful of large, moderately tilted splats in front of a camera, so
    almost every pair takes the ray-splat branch and no pixel saturates."""
    from msplat import synthetic as S
    rng = S.SplitMix64(seed)
    scene = S.make_scene(1, n=n, width=W, height=H)
    scene.means[:] = np.column_stack([rng.uniform(n, -0.25, 0.25), rng.uniform(n, -0.2, 0.2),
                                      rng.uniform(n, -0.5, 0.5)]).astype(np.float32)
    scene.scales[:] = rng.uniform(2 * n, -1.9, -1.4).reshape(n, 2).astype(np.float32)
    q = np.column_stack([np.ones(n), rng.uniform(3 * n, -0.3, 0.3).reshape(n, 3)])
    scene.quats[:] = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    scene.opacities[:] = rng.uniform(n, -1.5, 0.5).reshape(n, 1).astype(np.float32)
    scene.features_dc[:] = ((rng.uniform(3 * n) - 0.5) / 0.2820948).reshape(n, 3).astype(np.float32)
    return scene


def _fp64_render(scene, proj, bins, cam, T_over=None, opac_over=None, col_over=None, nrm_over=None):
    W, H = cam.width, cam.height
    outs = {k: np.zeros((H, W) + s) for k, s in
            dict(img=(3,), depth=(), normal=(3,), alpha=(), median=(), distortion=()).items()}
    lowpass = np.zeros((H, W), bool)
    for py in range(H):
        for px in range(W):
            t = (py // 16) * cam.tiles_x + px // 16
            lst = bins["ids"][bins["tile_offsets"][t]:bins["tile_offsets"][t + 1]]
            splats = []
            for g in lst:
                splats.append(dict(
                    T=(T_over[g] if T_over is not None else proj["transmats"][g].reshape(3, 3).astype(np.float64)),
                    xy=proj["xys"][g],
                    opac_logit=(opac_over[g] if opac_over is not None else float(proj["normal_opac"][g, 3])),
                    color_raw=(col_over[g] if col_over is not None else proj["colors"][g]),
                    normal=(nrm_over[g] if nrm_over is not None else proj["normal_opac"][g, :3])))
            o = R.composite(px, py, splats, scene.background)
            lowpass[py, px] = o["lowpass"] > 0
            for k in outs:
                outs[k][py, px] = o[k]
    return outs, lowpass


def test_raster_forward_matches_fp64_compositing(orc):
    scene = _tiny_scene(1, n=6)
    cam, proj, bins, fwd = orc.render(scene)
    outs, _ = _fp64_render(scene, proj, bins, cam)
    assert np.abs(fwd["out_img"] - outs["img"]).max() < 2e-5
    assert np.abs(fwd["out_depth"] - outs["depth"]).max() < 2e-4
    assert np.abs(fwd["out_alpha"] - outs["alpha"]).max() < 2e-5
    assert np.abs(fwd["out_normal"] - outs["normal"]).max() < 2e-5
    assert np.abs(fwd["out_distortion"] - outs["distortion"]).max() < 1e-5


def _fp64_pixel(px, py, T, xy, opac_logit, color_raw, bg, near=0.2):
    """Vectorised fp64 front-to-back compositing of one pixel over splats in
    list order (the rules of refmath.composite): returns (colour, number
    blended, smallest relative margin of any alpha / termination decision)."""
    k = T[:, 0] - px * T[:, 2]
    l = T[:, 1] - py * T[:, 2]
    det = k[:, 0] * l[:, 1] - k[:, 1] * l[:, 0]
    ok = det != 0.0
    det = np.where(ok, det, 1.0)
    u = (-k[:, 2] * l[:, 1] + k[:, 1] * l[:, 2]) / det
    v = (-k[:, 0] * l[:, 2] + k[:, 2] * l[:, 0]) / det
    d = xy - np.array([px, py])
    rho = np.minimum(u * u + v * v, 2.0 * (d * d).sum(1))
    depth = T[:, 2, 0] * u + T[:, 2, 1] * v + T[:, 2, 2]
    alpha = np.minimum(0.99, 1.0 / (1.0 + np.exp(-opac_logit)) * np.exp(-0.5 * rho))
    thr = 1.0 / 255.0
    use = ok & (depth >= near) & (alpha >= thr)
    a = np.where(use, alpha, 0.0)
    Tb = np.concatenate([[1.0], np.cumprod(1.0 - a)[:-1]])  # transmittance before each splat
    stop = use & (Tb * (1.0 - a) <= 1e-4)
    end = int(np.argmax(stop)) if stop.any() else len(a)
    w = (a * Tb)[:end]
    col = (np.maximum(color_raw[:end] + 0.5, 0.0) * w[:, None]).sum(0) + bg * Tb[end] if end < len(a) else \
        (np.maximum(color_raw + 0.5, 0.0) * w[:, None]).sum(0) + bg * np.prod(1.0 - a)
    margins = [np.abs(alpha[ok & (depth >= near)] - thr).min(initial=1.0) / thr]
    if use.any():
        margins.append((np.abs(Tb * (1.0 - a) - 1e-4)[use]).min() / 1e-4)
    return col, int(use[:end].sum()), min(margins)


def test_raster_forward_matches_fp64_compositing_deep_lists(orc):
    """Pixels that blend hundreds of splats: the golden model's fp32
    compositing (the kernels' arithmetic) against fp64 compositing of the
    same splats, to the 1e-4 image bar.  Pixels where any alpha or
    termination decision lies within 1e-5 relative of its threshold (a
    decision fp32 rounding may flip) are excluded and counted."""
    from msplat import synthetic as S
    rng = np.random.default_rng(3)
    n = 20_000
    scene = S.make_scene(1, n=n, width=64, height=48)
    scene.means[:] = rng.uniform(-1.2, 1.2, (n, 3)).astype(np.float32)
    scene.scales[:] = rng.normal(-1.6, 0.2, (n, 2)).astype(np.float32)
    scene.opacities[:] = rng.normal(-4.3, 0.3, (n, 1)).astype(np.float32)
    cam, proj, bins, fwd = orc.render(scene)
    H, W = cam.height, cam.width
    pix = rng.choice(H * W, 300, replace=False)
    diffs, blended, skipped = [], [], 0
    for p in pix:
        py, px = divmod(int(p), W)
        t = (py // 16) * cam.tiles_x + px // 16
        lst = bins["ids"][bins["tile_offsets"][t]:bins["tile_offsets"][t + 1]]
        T = proj["transmats"][lst].reshape(-1, 3, 3).astype(np.float64)
        col, nb, margin = _fp64_pixel(px, py, T, proj["xys"][lst].astype(np.float64),
                                      proj["normal_opac"][lst, 3].astype(np.float64),
                                      proj["colors"][lst].astype(np.float64), scene.background.astype(np.float64))
        if margin < 1e-5:
            skipped += 1
            continue
        diffs.append(np.abs(fwd["out_img"][py, px] - col).max())
        blended.append(nb)
    blended = np.array(blended)
    print(f"[deep] {len(diffs)} pixels, blended splats median {np.median(blended):.0f} max {blended.max()}, "
          f"max |diff| {max(diffs):.3g}, {skipped} pixels at a threshold tie")
    assert np.median(blended) >= 100  # realistic list depth
    assert skipped <= 6
    assert max(diffs) < 1e-4


def test_raster_single_fronto_parallel_splat_closed_form(orc):
    """A splat facing the camera centred on a pixel: alpha there is
    min(0.99, sigmoid(o)) and the pixel is c*alpha + bg*(1-alpha)."""
    from msplat import synthetic as S
    scene = S.make_scene(1, n=1, width=33, height=33)  # principal point on pixel 16
    scene.means[:] = 0.0
    scene.quats[:] = np.float32([1, 0, 0, 0])
    scene.scales[:] = np.float32(-3.0)
    scene.opacities[:] = np.float32(0.3)
    scene.features_dc[:] = np.float32([0.5, -0.2, 0.9])
    cam, proj, bins, fwd = orc.render(scene)
    cx, cy = int(round(proj["xys"][0, 0])), int(round(proj["xys"][0, 1]))
    assert abs(proj["xys"][0, 0] - cx) < 1e-4 and abs(proj["xys"][0, 1] - cy) < 1e-4
    a = min(0.99, 1.0 / (1.0 + math.exp(-0.3)))
    col = np.maximum(0.2820948 * scene.features_dc[0] + 0.5, 0)
    exp = col * a + scene.background * (1 - a)
    assert np.abs(fwd["out_img"][cy, cx] - exp).max() < 1e-5
    assert fwd["final_idx"][cy, cx, 0] == 1


def test_raster_empty_tiles_are_background(orc):
    from msplat import synthetic as S
    scene = S.make_scene(1, n=4, width=64, height=48)
    scene.means[:] = np.float32([0.0, 0.0, 10.0])  # behind the camera (camera at z=3 looks down -z)
    cam, proj, bins, fwd = orc.render(scene)
    assert bins["num_intersections"] == 0
    assert np.array_equal(fwd["out_img"], np.broadcast_to(scene.background, fwd["out_img"].shape))
    assert np.all(fwd["final_Ts"][..., 0] == 1.0) and np.all(fwd["final_idx"][..., 0] == 0)


def test_raster_backward_matches_finite_differences(orc):
    scene = _tiny_scene(2, n=5, W=36, H=30)
    cam, proj, bins, fwd = orc.render(scene)
    H, W = cam.height, cam.width
    from msplat import synthetic as S
    rng = S.SplitMix64(11)
    up = dict(img=rng.normal(H * W * 3).reshape(H, W, 3) * 0.01, depth=rng.normal(H * W).reshape(H, W) * 0.01,
              alpha=rng.normal(H * W).reshape(H, W) * 0.01, normal=rng.normal(H * W * 3).reshape(H, W, 3) * 0.01,
              median=rng.normal(H * W).reshape(H, W) * 0.01, distortion=rng.normal(H * W).reshape(H, W) * 0.1)
    # On the low-pass branch the reference passes depth gradients to T with
    # the ray-splat point held fixed (msplat_metal.metal:1957-1965), which is
    # not the derivative of the forward; keep depth-type upstream gradients
    # off the pixels where such a pair contributes, so the check is exact.
    _, lp0 = _fp64_render(scene, proj, bins, cam)
    for k in ("depth", "median", "distortion"):
        up[k][lp0] = 0.0
    up = {k: v.astype(np.float32) for k, v in up.items()}
    g = orc.raster_bwd(proj, bins, fwd, cam, scene.background, up["img"], up["depth"], up["alpha"], up["normal"],
                       up["median"], up["distortion"])
    n = scene.n
    T0 = [proj["transmats"][i].reshape(3, 3).astype(np.float64) for i in range(n)]
    op0 = [float(proj["normal_opac"][i, 3]) for i in range(n)]
    co0 = [proj["colors"][i].astype(np.float64) for i in range(n)]
    nr0 = [proj["normal_opac"][i, :3].astype(np.float64) for i in range(n)]

    def L(Tm, op, co, nr):
        outs, lp = _fp64_render(scene, proj, bins, cam, Tm, op, co, nr)
        assert np.array_equal(lp, lp0), "a perturbation moved a pair across the low-pass switch"
        return sum(float((outs[k] * up[k]).sum()) for k in up)

    for i in range(n):
        Ti = T0[i]
        for (r, c) in [(0, 0), (1, 1), (2, 2), (0, 2), (1, 2), (2, 0)]:
            h = 1e-6 * max(1.0, abs(Ti[r, c]))
            Tp = [t.copy() for t in T0]
            Tm = [t.copy() for t in T0]
            Tp[i][r, c] += h
            Tm[i][r, c] -= h
            fd = (L(Tp, op0, co0, nr0) - L(Tm, op0, co0, nr0)) / (2 * h)
            assert g[i, 3 * r + c] == pytest.approx(fd, rel=3e-3, abs=3e-7 * max(1.0, np.abs(g[:, :9]).max())), \
                (i, r, c)
        h = 1e-6
        opp, opm = list(op0), list(op0)
        opp[i] += h
        opm[i] -= h
        fd = (L(T0, opp, co0, nr0) - L(T0, opm, co0, nr0)) / (2 * h)
        assert g[i, 12] == pytest.approx(fd, rel=3e-3, abs=1e-7), ("opacity", i)
        for ch in range(3):
            cp = [c.copy() for c in co0]
            cm = [c.copy() for c in co0]
            cp[i][ch] += h
            cm[i][ch] -= h
            fd = (L(T0, op0, cp, nr0) - L(T0, op0, cm, nr0)) / (2 * h)
            assert g[i, 13 + ch] == pytest.approx(fd, rel=3e-3, abs=1e-7), ("color", i, ch)
            npp = [c.copy() for c in nr0]
            nm = [c.copy() for c in nr0]
            npp[i][ch] += h
            nm[i][ch] -= h
            fd = (L(T0, op0, co0, npp) - L(T0, op0, co0, nm)) / (2 * h)
            assert g[i, 9 + ch] == pytest.approx(fd, rel=3e-3, abs=1e-7), ("normal", i, ch)


# -------------------------------------------------------- project bwd ----
def test_project_backward_matches_finite_differences(orc):
    from msplat import synthetic as S
    scene = S.make_scene(2, n=12, width=96, height=64, num_cameras=1)
    c = scene.cameras[0]
    cam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                  features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = orc.project_fwd(params, cam, 3, 3)
    vis = np.flatnonzero(proj["radii"] > 0)
    assert vis.size >= 4
    rng = S.SplitMix64(21)
    g16 = rng.normal(scene.n * 16).reshape(scene.n, 16).astype(np.float32)
    out = orc.project_bwd(params, cam, 3, 3, proj["radii"], g16)

    def L(i, mean, ls, q, fdc, frest):
        T, nrm = R.project(mean, ls, q, cam.projmat, c.width, c.height, c.cx, c.cy)
        col = R.sh_color(mean, cam.cam_pos, fdc, frest, 3)
        return float((T.reshape(9) * g16[i, :9]).sum() + (nrm * g16[i, 9:12]).sum() + (col * g16[i, 13:16]).sum())

    for i in vis[:6]:
        base = [scene.means[i].astype(np.float64), scene.scales[i].astype(np.float64),
                scene.quats[i].astype(np.float64), scene.features_dc[i].astype(np.float64),
                scene.features_rest[i].astype(np.float64)]

        def fd(which, k, h=1e-6):
            p = [b.copy() for b in base]
            m = [b.copy() for b in base]
            p[which].reshape(-1)[k] += h
            m[which].reshape(-1)[k] -= h
            return (L(i, *p) - L(i, *m)) / (2 * h)

        for k in range(3):
            assert out["dmeans"][i, k] == pytest.approx(fd(0, k), rel=2e-3, abs=2e-4), ("mean", i, k)
        for k in range(2):
            assert out["dscales"][i, k] == pytest.approx(fd(1, k), rel=2e-3, abs=2e-4), ("scale", i, k)
        # the reference differentiates w.r.t. the normalised quaternion; the
        # tangential part is what a finite difference of the raw one sees
        qn = base[2] / np.linalg.norm(base[2])
        gq = out["dquats"][i].astype(np.float64)
        gq_tan = (gq - qn * (qn @ gq)) / np.linalg.norm(base[2])
        fdq = np.array([fd(2, k) for k in range(4)])
        assert np.abs(gq_tan - fdq).max() <= 2e-3 * np.abs(fdq).max() + 2e-4, ("quat", i)
        for k in range(3):
            assert out["dfdc"][i, k] == pytest.approx(fd(3, k), rel=2e-3, abs=1e-6)
        for k in (0, 7, 20, 44):
            assert out["dfrest"][i].reshape(-1)[k] == pytest.approx(fd(4, k), rel=2e-3, abs=1e-6)


# ---------------------------------------------------------- binning ----
def test_binning_and_sort_match_bruteforce(orc):
    from msplat import synthetic as S
    scene = S.make_scene(2, n=3000, width=200, height=136, num_cameras=1)
    c = scene.cameras[0]
    cam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                  features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = orc.project_fwd(params, cam, 3, 3)
    bins = orc.bin_sort(proj, cam)
    TX, TY = cam.tiles_x, cam.tiles_y
    xy = proj["xys"].astype(np.float32)
    r = proj["radii"].astype(np.float32)
    f2i = lambda v: np.trunc(np.clip(v, -2147483648.0, 2147483520.0)).astype(np.int64)
    x0 = np.clip(f2i(xy[:, 0] / np.float32(16) - r / np.float32(16)), 0, TX)
    x1 = np.clip(f2i(xy[:, 0] / np.float32(16) + r / np.float32(16) + np.float32(1)), 0, TX)
    y0 = np.clip(f2i(xy[:, 1] / np.float32(16) - r / np.float32(16)), 0, TY)
    y1 = np.clip(f2i(xy[:, 1] / np.float32(16) + r / np.float32(16) + np.float32(1)), 0, TY)
    keys = proj["depths"].view(np.uint32).astype(np.uint64) << np.uint64(32)
    for t in range(TX * TY):
        tx, ty = t % TX, t // TX
        members = np.flatnonzero((proj["radii"] > 0) & (x0 <= tx) & (tx < x1) & (y0 <= ty) & (ty < y1))
        order = members[np.argsort(keys[members] | members.astype(np.uint64), kind="stable")]
        got = bins["ids"][bins["tile_offsets"][t]:bins["tile_offsets"][t + 1]]
        assert np.array_equal(got, order), t
    assert np.array_equal(np.diff(bins["tile_offsets"]), bins["tile_counts"])


# --------------------------------------------------------------- Adam ----
def test_adam_first_step_closed_form(orc):
    from msplat import synthetic as S
    rng = S.SplitMix64(4)
    n = 10_000
    p0 = rng.normal(n)
    g = rng.normal(n) * 1e-2
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    lr = 0.01
    bc1, bc2 = 1 - 0.9, 1 - 0.999
    orc.adam(p, g.astype(np.float32), m, v, np.float32(lr / bc1), 0.9, 0.999, np.float32(math.sqrt(bc2)), 1e-8)
    # first step from zero moments: m = (1-b1) g, v = (1-b2) g^2, so
    # p1 = p0 - s (1-b1) g / (sqrt(1-b2) |g| / bc2_sqrt + eps), with the
    # float32 constants the kernel receives (1 - 0.999f is not 0.001)
    g = g.astype(np.float32).astype(np.float64)
    b1, b2 = float(np.float32(0.9)), float(np.float32(0.999))
    s, bcs = float(np.float32(lr / bc1)), float(np.float32(math.sqrt(bc2)))
    exp = p0.astype(np.float64) - s * (1 - b1) * g / (math.sqrt(1 - b2) * np.abs(g) / bcs + 1e-8)
    # the step passes through eight float32 roundings (m, v, sqrt, /, +eps, *,
    # /, -) of at most half an ulp each: 4 ulp of the larger operand of the
    # final subtraction (p0 - step can cancel)
    scale = np.maximum(np.abs(p0), np.abs(p0 - exp)).astype(np.float32)
    assert np.all(np.abs(p - exp) <= 4 * np.spacing(scale))


def test_adam_matches_fp64_recurrence(orc):
    from msplat import synthetic as S
    rng = S.SplitMix64(5)
    n = 2000
    p = rng.normal(n)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    pd, md, vd = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 6):
        g = (rng.normal(n) * 1e-3).astype(np.float32)
        bc1, bc2 = 1 - 0.9 ** t, 1 - 0.999 ** t
        orc.adam(p, g, m, v, np.float32(0.005 / bc1), 0.9, 0.999, np.float32(math.sqrt(bc2)), 1e-8)
        md = 0.9 * md + 0.1 * g
        vd = 0.999 * vd + 0.001 * g.astype(np.float64) ** 2
        pd = pd - 0.005 / bc1 * md / (np.sqrt(vd) / math.sqrt(bc2) + 1e-8)
    assert np.abs(p - pd).max() < 1e-6


# ------------------------------------------------------------ densify ----
def _densify_numpy(n, params, m6, v6, strides, stats, rs, th):
    """Serial restatement of msplat_densify (msplat_metal.mm:1339-1594) with
    stable compaction, in float64 for the arithmetic."""
    P = [np.asarray(a, np.float64).reshape(-1, s) for a, s in zip(params, strides)]
    M = [np.asarray(a, np.float64).reshape(-1, s) for a, s in zip(m6, strides)]
    V = [np.asarray(a, np.float64).reshape(-1, s) for a, s in zip(v6, strides)]
    vis = stats["vis"]
    avg = np.where(vis > 0, stats["grad_norm"] / np.where(vis > 0, vis, 1) * th["half"], 0)
    high = (vis > 0) & (avg > th["grad"])
    large = np.exp(P[1][:n]).max(1) > th["size"]
    split = high & (large | (stats["max2d"] > th["screen"]))
    dup = high & ~large
    rows = [p[:n].copy() for p in P]
    mrows = [a[:n].copy() for a in M]
    vrows = [a[:n].copy() for a in V]
    lsf = math.log(np.float32(1.6))
    new = [[] for _ in range(6)]
    for ord_, i in enumerate(np.flatnonzero(split)):
        q = P[2][i] / np.linalg.norm(P[2][i])
        w, x, y, z = q
        Rm = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                       [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                       [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])
        s = np.exp(P[1][i])
        for k in range(2):
            off = Rm @ (rs[2 * ord_ + k] * np.array([s[0], s[1], 0.0]))
            new[0].append(P[0][i] + off)
            new[1].append(P[1][i] - lsf)
            for gi in range(2, 6):
                new[gi].append(P[gi][i].copy())
        rows[1][i] = P[1][i] - lsf
    for i in np.flatnonzero(dup):
        for gi in range(6):
            new[gi].append(rows[gi][i].copy())
    nnew = len(new[0])
    allp = [np.concatenate([rows[gi], np.array(new[gi]).reshape(nnew, strides[gi])]) for gi in range(6)]
    allm = [np.concatenate([mrows[gi], np.zeros((nnew, strides[gi]))]) for gi in range(6)]
    allv = [np.concatenate([vrows[gi], np.zeros((nnew, strides[gi]))]) for gi in range(6)]
    N_new = n + nnew
    sig = 1 / (1 + np.exp(-allp[5][:, 0]))
    cull = sig < th["cull_alpha"]
    cull[:n] |= split
    cull |= np.exp(allp[1]).max(1) > th["cull_scale"]
    cull[:n] |= stats["max2d"] > th["cull_screen"]
    keep = ~cull
    return int(keep.sum()), [a[keep] for a in allp], [a[keep] for a in allm], [a[keep] for a in allv], N_new


def test_densify_matches_numpy_restatement(orc):
    from msplat import synthetic as S
    scene = S.make_scene(5, n=800, width=100, height=80, num_cameras=1)
    n = scene.n
    rng = S.SplitMix64(31)
    scene.scales[::4] += np.float32(2.5)
    scene.opacities[::9] = np.float32(-5.0)
    strides = [3, 2, 4, 3, 45, 1]
    cap = 3 * n
    src = scene.params()
    params = [np.zeros(cap * s, np.float32) for s in strides]
    for p, s, st in zip(params, src, strides):
        p[: n * st] = s.reshape(-1)
    m6 = [np.zeros(cap * s, np.float32) for s in strides]
    v6 = [np.zeros(cap * s, np.float32) for s in strides]
    for a, s in zip(m6 + v6, strides * 2):
        a[: n * s] = rng.uniform(n * s) * 1e-3
    stats = dict(grad_norm=(rng.uniform(n) * 0.02).astype(np.float32),
                 vis=np.floor(rng.uniform(n) * 4).astype(np.float32),
                 max2d=(rng.uniform(n) * 0.3).astype(np.float32))
    rs = rng.normal(2 * n * 3).reshape(2 * n, 3)
    th = dict(grad=0.0002, size=0.01, screen=0.05, cull_alpha=0.1, cull_scale=0.5, cull_screen=0.15, half=50.0)
    kept, P, M, V, N_new = _densify_numpy(n, params, m6, v6, strides, stats, rs.astype(np.float64), th)
    got = orc.densify(n, cap, [p.copy() for p in params] and params, m6, v6, 45, stats, rs, half_max_dim=50.0)
    assert got == kept and 0 < kept < N_new
    for gi, s in enumerate(strides):
        assert np.allclose(params[gi][: kept * s].reshape(kept, s), P[gi], atol=2e-6, rtol=2e-6), gi
        assert np.allclose(m6[gi][: kept * s].reshape(kept, s), M[gi], atol=1e-9), gi
        assert np.allclose(v6[gi][: kept * s].reshape(kept, s), V[gi], atol=1e-9), gi
