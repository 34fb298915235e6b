"""GPU parity: every stage of the HIP training step against the CPU golden
model on identical seeded inputs, through the C-ABI.

Bars (the oracle's arithmetic contract makes the non-atomic stages exact):
  projection, binning, per-tile order, rasterize forward, loss gradient,
  projection backward (given equal raster gradients), Adam, densify:
  bit-exact;
  rasterize backward (float atomics): per element |gpu - oracle| <=
  1e-3 |oracle| + 1e-4 A + 1e-7 max|oracle|, A the magnitude of its
  summands (tests/parity.py), and that bound carried through the projection
  backward and Adam for the post-Adam parameters;
  scalar loss: relative 1e-5 (fp64 reduction order differs).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from msplat import _engine as E  # noqa: E402
from msplat import device as D  # noqa: E402
from msplat import synthetic as S  # noqa: E402
from parity import grad_close, param_grad_noise, post_adam_close  # noqa: E402
from scenes import adversarial  # noqa: E402


def _cams(scene, idx, orc):
    c = scene.cameras[idx]
    return orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)


def _params(scene):
    return dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                features_dc=scene.features_dc, features_rest=scene.features_rest)


def _assert_bitexact(a, b, what):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype.kind == "f":
        bad = ~((a == b) | (np.isnan(a) & np.isnan(b)))
    else:
        bad = a != b
    nbad = int(bad.sum())
    if nbad:
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {nbad} of {a.size} entries differ, first at {idx.tolist()}: "
                             f"gpu={a[tuple(idx[0])]!r} oracle={b[tuple(idx[0])]!r}")


def _forward_both(scene, cam_idx, orc, eng, dtu=None):
    dtu = scene.sh_degree if dtu is None else dtu
    ocam, proj, bins, fwd = orc.render(scene, cam_idx, dtu)
    ds = D.DeviceScene(scene)
    gcam = ds.camera(scene.cameras[cam_idx], dtu)
    out = D.render(ds, gcam, outputs=("out_img", "final_Ts", "final_idx", "out_depth", "out_normal", "out_alpha",
                                      "out_median_depth", "out_distortion"))
    return ocam, proj, bins, fwd, ds, gcam, out


SCENES = {
    "fwd16k": lambda: S.make_scene(1),
    "blob40k_sh3": lambda: S.make_scene(2, n=40_000, width=320, height=208, num_cameras=4),
    # edge-on, needle-thin, huge, near-camera and off-screen splats
    "adversarial": lambda: adversarial(3000, 21, width=200, height=136),
}


@pytest.mark.parametrize("name", list(SCENES))
def test_camera_setup_bitexact(name, orc, eng):
    scene = SCENES[name]()
    for idx in range(len(scene.cameras)):
        c = scene.cameras[idx]
        o = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
        g = E.prepare_camera(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height, scene.sh_degree,
                             scene.sh_degree)
        _assert_bitexact(np.array(g.viewmat), np.array(o.viewmat), "viewmat")
        _assert_bitexact(np.array(g.projmat), np.array(o.projmat), "projmat")
        _assert_bitexact(np.array(g.cam_pos), np.array(o.cam_pos), "cam_pos")


@pytest.mark.parametrize("name", list(SCENES))
def test_project_and_binning_bitexact(name, orc, eng):
    scene = SCENES[name]()
    print(f"[project/binning] scene={name} n={scene.n}", flush=True)
    ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    n = scene.n
    _assert_bitexact(E.last("radii"), proj["radii"], "radii")
    _assert_bitexact(E.last("depths"), proj["depths"], "depths")
    _assert_bitexact(E.last("xys", (n, 2)), proj["xys"], "xys")
    _assert_bitexact(E.last("transmats", (n, 9)), proj["transmats"], "transmats")
    _assert_bitexact(E.last("normals", (n, 3)), proj["normal_opac"][:, :3], "normals")
    vis = proj["radii"] > 0
    sig = np.zeros(n, np.float32)
    for i in np.flatnonzero(vis):
        sig[i] = np.float32(1.0) / (np.float32(1.0) + np.float32(orc.expf(-proj["normal_opac"][i, 3])))
    _assert_bitexact(E.last("opacity_sigmoid"), sig, "opacity sigmoid")
    used = np.where(vis[:, None], np.maximum(proj["colors"] + np.float32(0.5), np.float32(0.0)), 0).astype(np.float32)
    _assert_bitexact(E.last("colors_used", (n, 3)), used, "colors (clamped)")
    _assert_bitexact(E.last("num_tiles_hit"), proj["tiles_hit"], "tiles hit")
    assert out["num_intersections"] == bins["num_intersections"]
    _assert_bitexact(E.last("tile_offsets"), bins["tile_offsets"], "tile offsets")
    _assert_bitexact(E.last("gaussian_ids"), bins["ids"], "per-tile sorted ids")


@pytest.mark.parametrize("name", list(SCENES))
def test_raster_forward_bitexact(name, orc, eng):
    scene = SCENES[name]()
    print(f"[raster fwd] scene={name}", flush=True)
    ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    for k in ("out_img", "final_Ts", "final_idx", "out_depth", "out_normal", "out_alpha", "out_median_depth",
              "out_distortion"):
        _assert_bitexact(out[k], fwd[k], k)


def test_fast_reciprocal_is_the_division(eng):
    """The rasterizer's 1 / ray.z (hardware reciprocal + one Newton step)
    equals the correctly rounded division, the golden model's, for every
    normal float of magnitude below 2^126 (exponent fields 1..252, both
    signs, all 2^23 mantissas: 4.2e9 floats).  Above, 1 / x is subnormal and
    the rasterizer takes the division itself."""
    bad = C.c_int64(-1)
    E.check(E.lib().msplat_hip_check_fast_rcp(1, 252, C.byref(bad)))
    assert bad.value == 0


@pytest.mark.parametrize("wide", [False, True], ids=["packed-keys", "wide-keys"])
def test_overflow_tiles_merge_path(wide, orc, eng):
    """Tiles far above 2048 intersections: the chunked LDS sort + global
    merge must give the oracle's full (untruncated) per-tile order, with
    either key layout."""
    scene = S.make_scene(4, n=100_000, width=480, height=270, num_cameras=2)
    print(f"[overflow] n={scene.n} wide={wide}", flush=True)
    E.check(E.lib().msplat_hip_set_wide_keys(1 if wide else 0))
    try:
        ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    finally:
        E.check(E.lib().msplat_hip_set_wide_keys(0))
    assert bins["tile_counts"].max() > 8 * 2048, bins["tile_counts"].max()
    _assert_bitexact(E.last("tile_offsets"), bins["tile_offsets"], "tile offsets")
    _assert_bitexact(E.last("gaussian_ids"), bins["ids"], "per-tile sorted ids")
    _assert_bitexact(out["out_img"], fwd["out_img"], "out_img")
    _assert_bitexact(out["final_idx"], fwd["final_idx"], "final_idx")


@pytest.mark.parametrize("name", ["blob40k_sh3", "adversarial"])
def test_wide_binning_keys_bitexact(name, orc, eng):
    """The binning's wide key layout (depth bits << 32 | id, the rectangle
    gathered per key), which scenes of 2^24 gaussians and more use, forced
    on small scenes: the same tile offsets and per-tile order as the golden
    model (the default packed layout is checked by every other test)."""
    scene = SCENES[name]()
    print(f"[wide keys] scene={name}", flush=True)
    E.check(E.lib().msplat_hip_set_wide_keys(1))
    try:
        ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    finally:
        E.check(E.lib().msplat_hip_set_wide_keys(0))
    assert out["num_intersections"] == bins["num_intersections"]
    _assert_bitexact(E.last("tile_offsets"), bins["tile_offsets"], "tile offsets")
    _assert_bitexact(E.last("gaussian_ids"), bins["ids"], "per-tile sorted ids")
    _assert_bitexact(out["out_img"], fwd["out_img"], "out_img")


def test_empty_scene_renders_background(orc, eng):
    scene = S.make_scene(1, n=64, width=48, height=40)
    scene.means[:] = np.float32(-50.0)  # all behind the camera
    ds = D.DeviceScene(scene)
    out = D.render(ds, ds.camera(scene.cameras[0]))
    assert out["num_intersections"] == 0
    assert np.array_equal(out["out_img"], np.broadcast_to(scene.background, out["out_img"].shape))


def test_zero_splats_render_background(orc, eng):
    """No gaussians at all (the binning's count matrix has no rows): the
    frame is the background and no intersection is emitted."""
    import dataclasses
    scene = S.make_scene(1, n=64, width=48, height=40)
    empty = dataclasses.replace(scene, means=scene.means[:0], scales=scene.scales[:0], quats=scene.quats[:0],
                                opacities=scene.opacities[:0], features_dc=scene.features_dc[:0],
                                features_rest=scene.features_rest[:0])
    assert empty.n == 0
    ds = D.DeviceScene(empty)
    out = D.render(ds, ds.camera(empty.cameras[0]))
    assert out["num_intersections"] == 0
    assert np.array_equal(out["out_img"], np.broadcast_to(empty.background, out["out_img"].shape))


def _device(a):
    return E.DeviceArray.from_numpy(np.ascontiguousarray(a, np.float32))


@pytest.mark.parametrize("form", [1, 2], ids=["stream", "two_pass"])
@pytest.mark.parametrize("shape,ldist", [((208, 320), 0.0), ((37, 53), 0.0), ((1, 1), 0.0), ((11, 150), 0.0),
                                          ((300, 517), 0.0), ((97, 203), 0.05), ((1030, 1100), 0.0)])
def test_loss_fwd_bwd_bitexact(shape, ldist, form, orc, eng):
    # stream: one wave per (54-column strip, row segment, channel); (1030,
    # 1100) has 21 strips, the last one ragged, and 17 row segments.
    # two_pass: (300, 517) is mostly interior 32x32 tiles, whose staging
    # skips the bounds checks, with a ragged right and bottom edge.
    # (97, 203) adds the distortion term of the loss.
    H, W = shape
    E.check(E.lib().msplat_hip_set_loss_form(form))
    try:
        _check_loss(H, W, ldist, orc)
    finally:
        E.check(E.lib().msplat_hip_set_loss_form(0))


def _check_loss(H, W, ldist, orc):
    rng = S.SplitMix64(17 + H * W)
    img = rng.uniform(H * W * 3).reshape(H, W, 3).astype(np.float32)
    gt = rng.uniform(H * W * 3).reshape(H, W, 3).astype(np.float32)
    gt[: H // 2] = img[: H // 2]  # exact-equality pixels: sign(0) = 0
    dist = rng.uniform(H * W).reshape(H, W).astype(np.float32)
    loss_o, dL_o, _, ssim_o = orc.loss_fwd_bwd(img, gt, distortion=dist if ldist else None, lambda_dist=ldist)
    d_img, d_gt, d_dL = _device(img), _device(gt), E.DeviceArray((H, W, 3))
    d_dist = _device(dist)
    loss = C.c_double()
    ssim = C.c_double()
    E.check(E.lib().msplat_hip_loss_fwd_bwd(W, H, d_img.ptr, d_gt.ptr, d_dist.ptr if ldist else None, 0.8, ldist,
                                           0.2, d_dL.ptr, C.byref(loss), C.byref(ssim)))
    _assert_bitexact(d_dL.numpy(), dL_o, "dL/dimg")
    assert abs(loss.value - loss_o) <= 1e-5 * abs(loss_o) + 1e-9
    assert abs(ssim.value - ssim_o) <= 1e-6 * abs(ssim_o) + 1e-6


@pytest.mark.parametrize("name", list(SCENES))
def test_raster_backward_close(name, orc, eng):
    scene = SCENES[name]()
    print(f"[raster bwd] scene={name}", flush=True)
    ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    target = scene.jittered(0.01, 99)
    gt = orc.render(target, 0)[3]["out_img"]
    _, dL, _, _ = orc.loss_fwd_bwd(fwd["out_img"], gt)
    g_o, a_o = orc.raster_bwd(proj, bins, fwd, ocam, scene.background, dL, with_abs=True)
    d_dL = _device(dL)
    g16 = E.DeviceArray.zeros((scene.n, 16))
    E.check(E.lib().msplat_hip_raster_bwd(d_dL.ptr, None, None, None, None, None, g16.ptr))
    g = g16.numpy()
    assert np.abs(g_o).max() > 0
    grad_close(g, g_o, a_o, "grads16 [dT(9), dn(3), dopacity, dcolor(3)]")
    # culled splats receive nothing
    assert np.all(g[proj["radii"] <= 0] == 0)


def test_raster_backward_all_upstream_gradients(orc, eng):
    """The general backward (depth, alpha, normal, median-depth and
    distortion gradients besides the image's) against the oracle."""
    scene = S.make_scene(2, n=20_000, width=256, height=160, num_cameras=2)
    ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    H, W = gcam.height, gcam.width
    rng = S.SplitMix64(12)
    up = dict(img=rng.normal(H * W * 3, 0, 1e-3).reshape(H, W, 3), depth=rng.normal(H * W, 0, 1e-3).reshape(H, W),
              alpha=rng.normal(H * W, 0, 1e-3).reshape(H, W), normal=rng.normal(H * W * 3, 0, 1e-3).reshape(H, W, 3),
              median=rng.normal(H * W, 0, 1e-3).reshape(H, W), dist=rng.normal(H * W, 0, 1e-2).reshape(H, W))
    g_o, a_o = orc.raster_bwd(proj, bins, fwd, ocam, scene.background, up["img"], up["depth"], up["alpha"],
                              up["normal"], up["median"], up["dist"], with_abs=True)
    dev = {k: _device(v) for k, v in up.items()}
    g16 = E.DeviceArray.zeros((scene.n, 16))
    E.check(E.lib().msplat_hip_raster_bwd(dev["img"].ptr, dev["depth"].ptr, dev["alpha"].ptr, dev["normal"].ptr,
                                          dev["median"].ptr, dev["dist"].ptr, g16.ptr))
    grad_close(g16.numpy(), g_o, a_o, "grads16 with all upstream gradients")


@pytest.mark.parametrize("name", list(SCENES))
def test_project_backward_bitexact(name, orc, eng):
    scene = SCENES[name]()
    ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    n = scene.n
    rng = S.SplitMix64(5)
    g16 = (rng.normal(n * 16, 0.0, 1e-3).reshape(n, 16)).astype(np.float32)
    g16[proj["radii"] <= 0] = 0
    stats0 = dict(grad_norm=rng.uniform(n).astype(np.float32), vis=np.floor(rng.uniform(n) * 3).astype(np.float32),
                  max2d=(rng.uniform(n) * 0.05).astype(np.float32))
    o = orc.project_bwd(_params(scene), ocam, scene.sh_degree, scene.sh_degree, proj["radii"], g16,
                        {k: v.copy() for k, v in stats0.items()})
    K3 = ((scene.sh_degree + 1) ** 2 - 1) * 3
    outs = {k: E.DeviceArray.zeros(s) for k, s in dict(dmeans=(n, 3), dscales=(n, 2), dquats=(n, 4),
                                                         dmean2d=(n, 2), dfdc=(n, 3), dfrest=(n, max(K3, 1))).items()}
    st = {k: _device(v) for k, v in stats0.items()}
    radii = E.DeviceArray.from_numpy(proj["radii"])
    d16 = _device(g16)
    E.check(E.lib().msplat_hip_project_bwd(C.byref(gcam), C.byref(ds.gaussians), radii.ptr, d16.ptr,
                                           outs["dmeans"].ptr, outs["dscales"].ptr, outs["dquats"].ptr,
                                           outs["dmean2d"].ptr, outs["dfdc"].ptr, outs["dfrest"].ptr,
                                           st["grad_norm"].ptr, st["vis"].ptr, st["max2d"].ptr,
                                           float(np.float32(1) / np.float32(max(gcam.width, gcam.height)))))
    for k in ("dmeans", "dscales", "dquats", "dmean2d", "dfdc"):
        _assert_bitexact(outs[k].numpy(), o[k], k)
    if K3:
        _assert_bitexact(outs["dfrest"].numpy().reshape(o["dfrest"].shape), o["dfrest"], "dfrest")
    for k in ("grad_norm", "vis", "max2d"):
        _assert_bitexact(st[k].numpy(), o[k], k)


def test_adam_bitexact(orc, eng):
    rng = S.SplitMix64(23)
    n = 100_003
    p = rng.normal(n).astype(np.float32)
    g = (rng.normal(n) * 1e-3).astype(np.float32)
    g[::7] = 0
    m = (rng.normal(n) * 1e-4).astype(np.float32)
    v = (rng.uniform(n) * 1e-6).astype(np.float32)
    dp, dg, dm, dv = (_device(a) for a in (p, g, m, v))
    step, bc2 = np.float32(0.005 / 0.271), np.float32(np.sqrt(np.float32(0.003)))
    E.check(E.lib().msplat_hip_fused_adam(dp.ptr, dg.ptr, dm.ptr, dv.ptr, n, step, 0.9, 0.999, bc2, 1e-8))
    orc.adam(p, g, m, v, step, 0.9, 0.999, bc2, 1e-8)
    _assert_bitexact(dp.numpy(), p, "params")
    _assert_bitexact(dm.numpy(), m, "exp_avg")
    _assert_bitexact(dv.numpy(), v, "exp_avg_sq")


def test_fused_adam_step_equals_unfused(orc, eng):
    """Projection backward with the six Adam groups fused in must equal the
    reference flow (gradients to memory, then msplat_fused_adam per group)
    bit for bit, given the same raster gradients."""
    scene = S.make_scene(2, n=30_000, width=256, height=160, num_cameras=2)
    dsA, dsB = D.DeviceScene(scene), D.DeviceScene(scene)
    gcam = dsA.camera(scene.cameras[0])
    D.render(dsA, gcam)
    radii = E.DeviceArray.from_numpy(E.last("radii"))
    n = scene.n
    rng = S.SplitMix64(8)
    K3 = 45
    inv_max_dim = float(np.float32(1) / np.float32(max(gcam.width, gcam.height)))
    for step in range(3):
        g16 = _device((rng.normal(n * 16, 0.0, 1e-3).reshape(n, 16)).astype(np.float32))
        adamA = dsA.adam_struct()
        E.check(E.lib().msplat_hip_project_bwd_adam(C.byref(gcam), C.byref(dsA.gaussians), radii.ptr, g16.ptr,
                                                    dsA.grad_norm.ptr, dsA.vis.ptr, dsA.max2d.ptr, inv_max_dim,
                                                    C.byref(adamA)))
        outs = [E.DeviceArray.zeros(s) for s in ((n, 3), (n, 2), (n, 4), (n, 2), (n, 3), (n, K3))]
        E.check(E.lib().msplat_hip_project_bwd(C.byref(gcam), C.byref(dsB.gaussians), radii.ptr, g16.ptr,
                                               *[o.ptr for o in outs], dsB.grad_norm.ptr, dsB.vis.ptr, dsB.max2d.ptr,
                                               inv_max_dim))
        adamB = dsB.adam_struct()
        ga = E.DeviceArray.from_numpy(g16.numpy()[:, 12].copy())
        grads = [outs[0], outs[1], outs[2], outs[4], outs[5], ga]
        for gi in range(6):
            p = dsB.params[gi]
            E.check(E.lib().msplat_hip_fused_adam(p.ptr, grads[gi].ptr, dsB.exp_avg[gi].ptr, dsB.exp_avg_sq[gi].ptr,
                                                  int(np.prod(p.shape)), adamB.step_size[gi], adamB.beta1,
                                                  adamB.beta2, adamB.bc2_sqrt, adamB.eps))
        E.sync()
    pa, pb = dsA.host_params(), dsB.host_params()
    for k in pa:
        _assert_bitexact(pa[k], pb[k], k)
    for a, b in zip(dsA.exp_avg + dsA.exp_avg_sq, dsB.exp_avg + dsB.exp_avg_sq):
        _assert_bitexact(a.numpy(), b.numpy(), "adam moment")


def test_train_step_matches_oracle(orc, eng):
    scene = S.make_scene(2, n=30_000, width=256, height=160, num_cameras=2)
    target = scene.jittered(0.01, 4)
    ocam, _, _, tf = orc.render(target, 0)
    gt = tf["out_img"]
    # oracle step
    params = [p.copy() for p in scene.params()]
    m6 = [np.zeros_like(p) for p in params]
    v6 = [np.zeros_like(p) for p in params]
    stats = dict(grad_norm=np.zeros(scene.n, np.float32), vis=np.zeros(scene.n, np.float32),
                 max2d=np.zeros(scene.n, np.float32))
    loss_o, img_o, _, nis_o = orc.train_step(params, m6, v6, ocam, scene.background, gt, 3, 3, D.LR_INIT, 1, stats)
    # gpu step
    ds = D.DeviceScene(scene)
    gcam = ds.camera(scene.cameras[0])
    d_gt = _device(gt)
    loss, nis = D.train_step(ds, gcam, d_gt)
    assert nis == nis_o
    assert abs(loss - loss_o) <= 1e-5 * abs(loss_o)
    _assert_bitexact(E.last("out_img", img_o.shape), img_o, "rendered image")
    # the outputs the image-only training forward skips are produced on
    # demand, bit-identical to a full forward of the same (pre-step) splats
    _, proj_o, bins_o, full_o = orc.render(scene, 0)
    for k in ("final_Ts", "final_idx", "out_depth", "out_normal", "out_alpha", "out_median_depth",
              "out_distortion"):
        _assert_bitexact(E.last(k, full_o[k].shape), full_o[k], k)
    # the step's cached raster gradients (ray moments inside the step,
    # dL/dtransMat through the accessor) against the golden model's raster
    # backward of the same forward and loss gradient
    _, dL_o, _, _ = orc.loss_fwd_bwd(full_o["out_img"], gt)
    g_o, a_o = orc.raster_bwd(proj_o, bins_o, full_o, ocam, scene.background, dL_o, with_abs=True)
    grad_close(E.last("grads16", (scene.n, 16)), g_o, a_o, "train step grads16")
    got = ds.host_params()
    names = list(got)
    noise = param_grad_noise(orc, _params(scene), ocam, 3, 3, proj_o["radii"], g_o, a_o)
    post_adam_close(names, [got[k] for k in names], params, [m.numpy() for m in ds.exp_avg], m6, noise, D.LR_INIT)
    for k in stats:
        got_s = {"grad_norm": ds.grad_norm, "vis": ds.vis, "max2d": ds.max2d}[k].numpy()
        if k == "vis" or k == "max2d":
            _assert_bitexact(got_s, stats[k], k)


def _densify_inputs(scene, n, cap, seed):
    rng = S.SplitMix64(seed)
    K3 = ((scene.sh_degree + 1) ** 2 - 1) * 3
    strides = [3, 2, 4, 3, K3, 1]
    params = [np.zeros(cap * s, np.float32) for s in strides]
    src = [scene.means, scene.scales, scene.quats, scene.features_dc, scene.features_rest, scene.opacities]
    for p, s, st in zip(params, src, strides):
        p[: n * st] = s.reshape(-1)[: n * st]
    m6 = [np.zeros(cap * s, np.float32) for s in strides]
    v6 = [np.zeros(cap * s, np.float32) for s in strides]
    for a in m6 + v6:
        a[: a.size // cap * n] = (rng.uniform(a.size // cap * n) * 1e-3).astype(np.float32)
    stats = dict(grad_norm=(rng.uniform(n) * 0.02).astype(np.float32),
                 vis=np.floor(rng.uniform(n) * 4).astype(np.float32),
                 max2d=(rng.uniform(n) * 0.3).astype(np.float32))
    rs = rng.normal(2 * n * 3).reshape(2 * n, 3).astype(np.float32)
    return params, m6, v6, strides, stats, rs


def test_densify_bitexact(orc, eng):
    scene = S.make_scene(5, n=20_000, width=320, height=208, num_cameras=1)
    scene.scales[::3] += np.float32(2.0)  # large splats: split candidates
    scene.opacities[::11] = np.float32(-6.0)  # transparent splats: culled
    n = scene.n
    cap = 3 * n + 17
    params, m6, v6, strides, stats, rs = _densify_inputs(scene, n, cap, 77)
    dev = [_device(a) for a in params + m6 + v6]
    dstats = {k: _device(v) for k, v in stats.items()}
    d_rs = _device(rs)
    P6 = C.c_void_p * 6
    newc = C.c_int()
    E.check(E.lib().msplat_hip_densify(n, cap, 0.0002, 0.01, 0.05, 1, 0.1, 0.5, 0.15, 1, dstats["grad_norm"].ptr,
                                       dstats["vis"].ptr, dstats["max2d"].ptr, 648.5,
                                       P6(*[d.ptr for d in dev[0:6]]), strides[4], P6(*[d.ptr for d in dev[6:12]]),
                                       P6(*[d.ptr for d in dev[12:18]]), d_rs.ptr, C.byref(newc)))
    new_o = orc.densify(n, cap, params, m6, v6, strides[4], stats, rs, half_max_dim=648.5)
    assert newc.value == new_o
    assert new_o != n
    for i, (d, o) in enumerate(zip(dev, params + m6 + v6)):
        s = strides[i % 6]
        _assert_bitexact(d.numpy()[: new_o * s], o[: new_o * s], f"buffer {i}")


def test_densify_split_and_dup_beyond_3n(orc, eng):
    """Splats small in the world but wide on screen with a high gradient are
    classified both split and dup (msplat_metal.metal:3250-3262), so the
    appended count exceeds 3N.  At capacity 3N the call must leave every
    buffer untouched and report the rows it needs; at that capacity it must
    match the golden model bit for bit."""
    scene = S.make_scene(5, n=5000, width=320, height=208, num_cameras=1)
    n = scene.n
    rng = S.SplitMix64(91)
    scene.scales[:] = np.float32(-6.0)  # max scale 2.5e-3 < size threshold: not large
    params, m6, v6, strides, stats, rs = _densify_inputs(scene, n, 4 * n, 92)
    stats["grad_norm"][:] = np.float32(0.01)  # high gradient everywhere
    stats["vis"][:] = np.float32(1.0)
    stats["max2d"][:] = (0.04 + rng.uniform(n) * 0.04).astype(np.float32)  # about 3/4 above 0.05
    P6 = C.c_void_p * 6
    args = (0.0002, 0.01, 0.05, 1, 0.005, 0.5, 0.15, 0)
    dstats = {k: _device(v) for k, v in stats.items()}
    d_rs = _device(rs)
    dev = [_device(a) for a in params + m6 + v6]

    def call(cap):
        newc = C.c_int()
        rc = E.lib().msplat_hip_densify(n, cap, *args, dstats["grad_norm"].ptr, dstats["vis"].ptr,
                                        dstats["max2d"].ptr, 160.0, P6(*[d.ptr for d in dev[0:6]]), strides[4],
                                        P6(*[d.ptr for d in dev[6:12]]), P6(*[d.ptr for d in dev[12:18]]), d_rs.ptr,
                                        C.byref(newc))
        return rc, newc.value

    rc, need = call(3 * n)
    assert rc == E.MSPLAT_E_CAPACITY and need > 3 * n, (rc, need)
    for i, (d, o) in enumerate(zip(dev, params + m6 + v6)):
        _assert_bitexact(d.numpy(), o, f"buffer {i} after the refused call")
    assert orc.densify(n, 3 * n, params, m6, v6, strides[4], stats, rs, *args, half_max_dim=160.0) == -need
    rc, newc = call(need)
    assert rc == 0
    new_o = orc.densify(n, need, params, m6, v6, strides[4], stats, rs, *args, half_max_dim=160.0)
    assert newc == new_o and new_o > n
    for i, (d, o) in enumerate(zip(dev, params + m6 + v6)):
        st = strides[i % 6]
        _assert_bitexact(d.numpy()[: new_o * st], o[: new_o * st], f"buffer {i}")
