"""The 3DGS mode on the GPU against the golden model: projection records,
tile lists and images bit for bit (also for needle-thin, near-opaque and
off-screen Gaussians, which stress the quadrant masks), raster gradients
within the float-atomic bound, the projection backward bit for bit from
the GPU's own raster gradients, the fused Adam step, and training."""
import ctypes as C
import os

import numpy as np
import pytest

from parity import literal_rel, raster_bound, record, trainer_post_adam_close

pytestmark = pytest.mark.gpu

GROUPS = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")


def _scene(seed, n, W, H, needles=False):
    rng = np.random.default_rng(seed)
    p = dict(means=np.column_stack([rng.uniform(-0.9, 0.9, n), rng.uniform(-0.7, 0.7, n), rng.uniform(-0.8, 0.8, n)]),
             scales=rng.uniform(-3.6, -2.4, (n, 3)),
             quats=rng.normal(0, 1, (n, 4)),
             opacities=rng.uniform(-1.5, 2.0, (n, 1)),
             features_dc=rng.uniform(-1.2, 1.2, (n, 3)),
             features_rest=rng.normal(0, 0.2, (n, 15, 3)))
    if needles:
        k = n // 3
        p["scales"][:k, 0] = rng.uniform(-1.6, -1.0, k)  # long axis
        p["scales"][:k, 1:] = rng.uniform(-6.5, -5.5, (k, 2))  # thin
        p["opacities"][:k] = rng.uniform(4.0, 9.0, (k, 1))  # near-opaque
        p["means"][k:2 * k, :2] *= 1.6  # partly off screen
    p["quats"] /= np.linalg.norm(p["quats"], axis=1, keepdims=True)
    p = {k: v.astype(np.float32) for k, v in p.items()}
    c2w = np.eye(4, dtype=np.float32)
    c2w[2, 3] = 3.2
    cam = dict(c2w=c2w, fx=1.05 * W, fy=1.1 * W, cx=W / 2 + 0.3, cy=H / 2 - 0.6, W=W, H=H)
    return p, cam


def _cams(orc, eng, c):
    ocam = orc.prepare_cam(c["c2w"], c["fx"], c["fy"], c["cx"], c["cy"], c["W"], c["H"])
    gcam = eng.prepare_camera(c["c2w"], c["fx"], c["fy"], c["cx"], c["cy"], c["W"], c["H"], 3, 3)
    return ocam, gcam


def _oracle_render(orc, p, ocam, bg):
    proj = orc.project3d_fwd(p, ocam, 3, 3)
    bins = orc.bin_sort(proj, ocam)
    fwd = orc.raster3d_fwd(proj, bins, ocam, p["opacities"], bg)
    return proj, bins, fwd


@pytest.mark.parametrize("needles", [False, True])
def test_render3d_matches_oracle(orc, eng, needles):
    from msplat import device as D
    p, c = _scene(1 + needles, 3000, 200, 136, needles)
    bg = np.float32([0.2, 0.4, 0.7])
    ocam, gcam = _cams(orc, eng, c)
    proj, bins, fwd = _oracle_render(orc, p, ocam, bg)
    ds = D.DeviceScene3D(p, bg)
    out = D.render3d(ds, gcam)
    assert out["num_intersections"] == bins["num_intersections"] > 3000
    n = p["means"].shape[0]
    assert np.array_equal(eng.last("radii", (n,)), proj["radii"])
    vis = proj["radii"] > 0
    assert np.array_equal(eng.last("xys", (n, 2))[vis], proj["xys"][vis])
    assert np.array_equal(eng.last("depths", (n,))[vis], proj["depths"][vis])
    rec = eng.last("records", (n, 12))
    assert np.array_equal(rec[vis][:, 2:5], proj["conics"][vis])
    sig = np.float32(1.0) / (np.float32(1.0) + orc.expf_array(-p["opacities"][:, 0]))
    assert np.array_equal(rec[vis][:, 5], sig[vis])
    cols = np.maximum(proj["colors"] + np.float32(0.5), np.float32(0.0))
    assert np.array_equal(eng.last("colors_used", (n, 3))[vis], cols[vis])
    assert np.array_equal(eng.last("tile_offsets", (ocam.tiles_x * ocam.tiles_y + 1,)), bins["tile_offsets"])
    assert np.array_equal(eng.last("gaussian_ids", (bins["num_intersections"],)), bins["ids"])
    assert np.array_equal(out["out_img"], fwd["out_img"])
    assert np.array_equal(out["final_T"], fwd["final_T"])


def test_render3d_ill_conditioned_needles(orc, eng):
    """Long near-opaque needles at 1297x840 (2D covariances with condition
    numbers up to ~6e4), where a box without the rounding allowance for the
    conic's conditioning drops boundary pixels: images bit-exact."""
    from msplat import device as D
    from test_quadrant_masks import _scene3d
    p, c = _scene3d(4, 1500, 1297, 840, "needles")
    bg = np.float32([0.1, 0.2, 0.3])
    ocam = orc.prepare_cam(*c)
    gcam = eng.prepare_camera(*c, 3, 3)
    proj, bins, fwd = _oracle_render(orc, p, ocam, bg)
    out = D.render3d(D.DeviceScene3D(p, bg), gcam)
    assert out["num_intersections"] == bins["num_intersections"]
    assert np.array_equal(out["out_img"], fwd["out_img"])
    assert np.array_equal(out["final_T"], fwd["final_T"])


def _setup_step(orc, eng, seed, n=2500, W=160, H=120):
    from msplat import _engine as E
    from msplat import device as D
    p, c = _scene(seed, n, W, H)
    bg = np.float32([0.5, 0.3, 0.2])
    ocam, gcam = _cams(orc, eng, c)
    # the target: a render of jittered means
    pj = dict(p)
    pj["means"] = p["means"] + np.random.default_rng(seed + 7).normal(0, 0.02, p["means"].shape).astype(np.float32)
    gt = _oracle_render(orc, pj, ocam, bg)[2]["out_img"]
    return p, c, bg, ocam, gcam, gt, E.DeviceArray.from_numpy(gt), D


def test_train_step3d_gradients_match_oracle(orc, eng):
    p, c, bg, ocam, gcam, gt, gt_dev, D = _setup_step(orc, eng, 11)
    n = p["means"].shape[0]
    ds = D.DeviceScene3D(p, bg)
    loss, _ = D.train_step3d(ds, gcam, gt_dev, 0.2, fused_adam=False)
    proj, bins, fwd = _oracle_render(orc, p, ocam, bg)
    oloss, dL, _, _ = orc.loss_fwd_bwd(fwd["out_img"], gt, lambda_l1=0.8, lambda_dssim=0.2)
    assert loss == pytest.approx(oloss, rel=1e-6)
    assert np.array_equal(eng.last("dL_dout_img", (c["H"], c["W"], 3)), dL)
    g_o, a_o = orc.raster3d_bwd(proj, bins, fwd, ocam, p["opacities"], bg, dL, with_abs=True)
    g16 = eng.last("grads16", (n, 16))
    g9 = np.ascontiguousarray(g16[:, :9])
    err = np.abs(g9.astype(np.float64) - g_o)
    bound = raster_bound(g_o, a_o)
    assert (err <= bound).all(), f"worst err/bound {float((err / bound).max())}"
    # the projection backward from the GPU's own raster gradients
    ref = orc.project3d_bwd(p, ocam, 3, 3, proj["radii"], g9)
    for name, key, shape in (("dL_dmean3D", "dmeans", (n, 3)), ("dL_dscale", "dscales", (n, 3)),
                             ("dL_dquat", "dquats", (n, 4)), ("dL_dfeatures_dc", "dfdc", (n, 3)),
                             ("dL_dmean2D", "dmean2d", (n, 2))):
        got = eng.last(name, shape)
        assert np.array_equal(got, ref[key]), name
    assert np.array_equal(eng.last("dL_dfeatures_rest", (n, 15, 3)), ref["dfrest"])
    assert np.array_equal(ds.grad_norm.numpy(), ref["grad_norm"])
    assert np.array_equal(ds.vis.numpy(), ref["vis"])
    assert np.array_equal(ds.max2d.numpy(), ref["max2d"])


def test_train_step3d_fused_adam_matches_oracle(orc, eng):
    """The fused step's parameters and moments equal the golden model's
    projection backward and Adam applied to the same step's raster
    gradients, bit for bit (the raster backward's float atomics make two
    runs differ, so both sides take this run's)."""
    p, c, bg, ocam, gcam, gt, gt_dev, D = _setup_step(orc, eng, 12)
    n = p["means"].shape[0]
    ds = D.DeviceScene3D(p, bg)
    D.train_step3d(ds, gcam, gt_dev, 0.2, fused_adam=True)
    g9 = np.ascontiguousarray(eng.last("grads16", (n, 16))[:, :9])
    proj = orc.project3d_fwd(p, ocam, 3, 3)
    ref = orc.project3d_bwd(p, ocam, 3, 3, proj["radii"], g9)
    grads = [ref["dmeans"], ref["dscales"], ref["dquats"], ref["dfdc"], ref["dfrest"],
             np.ascontiguousarray(g9[:, 5:6])]
    adam = D.DeviceScene3D(p, bg).adam_struct()  # step 1's constants
    for g, name in enumerate(GROUPS):
        par = np.ascontiguousarray(p[name], np.float32).copy()
        m = np.zeros_like(par)
        v = np.zeros_like(par)
        orc.adam(par, np.ascontiguousarray(grads[g], np.float32).reshape(par.shape), m, v, adam.step_size[g],
                 adam.beta1, adam.beta2, adam.bc2_sqrt, adam.eps)
        assert np.array_equal(ds.params[g].numpy(), par), name
        assert np.array_equal(ds.exp_avg[g].numpy(), m), name
        assert np.array_equal(ds.exp_avg_sq[g].numpy(), v), name
    for k, d in (("grad_norm", ds.grad_norm), ("vis", ds.vis), ("max2d", ds.max2d)):
        assert np.array_equal(d.numpy(), ref[k]), k


def test_training3d_reduces_the_loss(orc, eng):
    p, c, bg, ocam, gcam, gt, gt_dev, D = _setup_step(orc, eng, 13)
    ds = D.DeviceScene3D(p, bg)
    losses = [D.train_step3d(ds, gcam, gt_dev, 0.2)[0] for _ in range(40)]
    assert np.isfinite(losses).all()
    assert losses[-1] < 0.7 * losses[0]


def test_densify3d_bitexact(orc, eng):
    """msplat_hip_densify_3dgs against the golden model's 3-scale densify:
    classification on the largest of three scales, children along three
    axes, splats both split and duplicated, culling and compaction."""
    from test_oracle3d import STRIDES3, _dens_inputs
    E = eng
    n, cap, params, m6, v6, stats, rs = _dens_inputs(n=20_000, seed=21)
    stats["grad_norm"][::7] = 0.0
    params[5][: n][::13] = -6.0  # transparent: culled
    dev = [E.DeviceArray.from_numpy(a) for a in params + m6 + v6]
    dstats = {k: E.DeviceArray.from_numpy(v) for k, v in stats.items()}
    d_rs = E.DeviceArray.from_numpy(rs)
    P6 = C.c_void_p * 6
    newc = C.c_int()
    E.check(E.lib().msplat_hip_densify_3dgs(n, cap, 0.0002, 0.05, 0.05, 1, 0.1, 0.5, 0.15, 1,
                                            dstats["grad_norm"].ptr, dstats["vis"].ptr, dstats["max2d"].ptr, 100.0,
                                            P6(*[d.ptr for d in dev[0:6]]), 45, P6(*[d.ptr for d in dev[6:12]]),
                                            P6(*[d.ptr for d in dev[12:18]]), d_rs.ptr, C.byref(newc)))
    new_o = orc.densify(n, cap, params, m6, v6, 45, stats, rs, size_thresh=0.05, half_max_dim=100.0, scale_dim=3)
    assert newc.value == new_o and new_o != n
    for i, (d, o) in enumerate(zip(dev, params + m6 + v6)):
        s = STRIDES3[i % 6]
        assert np.array_equal(d.numpy()[: new_o * s], o[: new_o * s]), f"buffer {i}"


def test_trainer3d_step_matches_golden_model(tmp_path):
    """GaussianTrainer(primitive='3dgs'): model init (three scales) ->
    export -> one step -> export, against the golden model's 3DGS step from
    the exported initial parameters through the trainer's own camera, bias
    corrections and learning rates."""
    import msplat
    from oracle import oracle as O
    from test_gpu_trainer import _dataset_inputs, _read_gaussian_ply

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=1)
    ds = msplat.Dataset.from_arrays(images, c2w, intr, xyz, rgb)
    bg = [float(v) for v in scene.background]
    cfg = msplat.TrainingConfig(iterations=100, num_downscales=0, bg_color=bg)
    tr = msplat.GaussianTrainer(ds, cfg, primitive="3dgs")
    assert tr.primitive == "3dgs"
    tr.export_ply(str(tmp_path / "p0.ply"))
    p0 = _read_gaussian_ply(tmp_path / "p0.ply")
    assert p0["scales"].shape == (len(xyz), 3)
    stats = tr.step()
    tr.export_ply(str(tmp_path / "p1.ply"))
    p1 = _read_gaussian_ply(tmp_path / "p1.ply")
    assert stats.iteration == 1 and stats.splat_count == len(xyz)

    c = scene.cameras[0]
    ocam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = {k: np.ascontiguousarray(p0[k], np.float32) for k in GROUPS}
    m = {k: np.zeros_like(v) for k, v in params.items()}
    v = {k: np.zeros_like(x) for k, x in params.items()}
    st = dict(grad_norm=np.zeros(len(xyz), np.float32), vis=np.zeros(len(xyz), np.float32),
              max2d=np.zeros(len(xyz), np.float32))
    lrs = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)
    loss_o, _, _ = O.train_step3d(params, m, v, ocam, np.float32(bg), images[0], 3, 0, lrs, 1, st)
    assert abs(stats.loss - loss_o) <= 1e-5 * abs(loss_o)
    for k, lr in zip(GROUPS, lrs):
        trainer_post_adam_close(k, p1[k], params[k], m[k], lr)
    assert np.abs(p1["means"] - p0["means"]).max() > 0


def test_trainer3d_training_densify_and_formats(tmp_path):
    """The 3DGS trainer end to end: training with densification (three-scale
    compaction), PLY / .splat / checkpoint round trips, and the depth-based
    exports refused."""
    import math

    import msplat
    from test_gpu_trainer import _dataset_inputs, _read_gaussian_ply

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=4)
    ds = msplat.Dataset.from_arrays(images, c2w, intr, xyz, rgb)
    cfg = msplat.TrainingConfig(iterations=2000, num_downscales=0, refine_every=10, warmup_length=10,
                                reset_alpha_every=3, densify_grad_thresh=1e-6)
    tr = msplat.GaussianTrainer(ds, cfg, primitive="3dgs")
    steps = [tr.step() for _ in range(55)]
    counts = [s.splat_count for s in steps]
    losses = [s.loss for s in steps]
    assert all(math.isfinite(x) for x in losses)
    assert counts[18] == len(xyz) and counts[19] != counts[18]  # densified at step 20
    assert counts[49] != counts[48]  # and at step 50
    assert np.mean(losses[-5:]) < np.mean(losses[:5])

    tr.export_ply(str(tmp_path / "g.ply"))
    g = _read_gaussian_ply(tmp_path / "g.ply")
    assert g["scales"].shape == (tr.splat_count, 3)
    assert [k for k in g["names"] if k.startswith("scale_")] == ["scale_0", "scale_1", "scale_2"]
    tr.export_splat(str(tmp_path / "g.splat"))
    assert (tmp_path / "g.splat").stat().st_size == 32 * tr.splat_count
    img = tr.render(0)
    tr.save_checkpoint(str(tmp_path / "g.msplat"))
    for _ in range(3):
        tr.step()
    assert not np.array_equal(tr.render(0), img)
    tr.load_checkpoint(str(tmp_path / "g.msplat"))
    assert tr.iteration == 55
    assert np.array_equal(tr.render(0), img)
    # the 3-scale PLY resumes into a 3DGS trainer with the same render
    tr2 = msplat.GaussianTrainer(ds, cfg, primitive="3dgs")
    assert tr2.load_ply(str(tmp_path / "g.ply")) == 55
    assert np.array_equal(tr2.render(0), img)
    with pytest.raises(RuntimeError):
        tr.extract_mesh(str(tmp_path / "m.ply"))
    with pytest.raises(RuntimeError):
        tr.export_point_cloud(str(tmp_path / "pc.ply"))
    # a surfel trainer refuses the 3-scale checkpoint
    tr_2d = msplat.GaussianTrainer(ds, cfg)
    with pytest.raises(RuntimeError):
        tr_2d.load_checkpoint(str(tmp_path / "g.msplat"))
    with pytest.raises(Exception):
        msplat.GaussianTrainer(ds, cfg, primitive="4dgs")


def test_c_abi_trainer_3dgs(tmp_path):
    """msplat_trainer_create_3dgs through the C ABI binding (msplat.capi):
    training steps, a 3-scale PLY, and extract_mesh refused with a message."""
    from msplat import capi
    from test_gpu_trainer import _dataset_inputs, _read_gaussian_ply

    L = capi.lib()
    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=3)
    imgs = [np.ascontiguousarray(i, np.float32) for i in images]
    cams = (capi.CameraImage * 3)()
    for i in range(3):
        cams[i].width, cams[i].height = imgs[i].shape[1], imgs[i].shape[0]
        cams[i].fx, cams[i].fy, cams[i].cx, cams[i].cy = (float(v) for v in intr[i])
        cams[i].camToWorld[:] = [float(v) for v in c2w[i].reshape(-1)]
        cams[i].rgb = imgs[i].ctypes.data
    pts = np.ascontiguousarray(xyz, np.float32)
    cols = np.ascontiguousarray(rgb, np.uint8)
    ds = L.msplat_dataset_create_from_memory(cams, 3, pts.ctypes.data, cols.ctypes.data, len(pts), False, 8)
    assert ds, capi.last_error()
    cfg = capi.default_config()
    cfg.numDownscales = 0
    tr = L.msplat_trainer_create_3dgs(ds, cfg)
    assert tr, capi.last_error()
    try:
        losses = [L.msplat_trainer_step(tr).loss for _ in range(20)]
        assert np.isfinite(losses).all() and np.mean(losses[-3:]) < np.mean(losses[:3])
        assert L.msplat_trainer_iteration(tr) == 20
        L.msplat_trainer_export_ply(tr, str(tmp_path / "c3.ply").encode())
        assert _read_gaussian_ply(tmp_path / "c3.ply")["scales"].shape == (len(pts), 3)
        assert L.msplat_trainer_extract_mesh(tr, str(tmp_path / "m.ply").encode(), 0.02, 1.0, 0.5, 4.0) == -1
        assert "depth" in capi.last_error()
    finally:
        L.msplat_trainer_destroy(tr)
        L.msplat_dataset_destroy(ds)


@pytest.mark.parametrize("workload", [2, 3], ids=["500k-1297x840", "3M-5187x3361"])
def test_full_step3d_matches_oracle_full_size(workload, orc, eng):
    """One fused 3DGS train step of a benchmark workload's splats as 3D
    Gaussians at full size against the golden model: intersections, tile
    lists and image bit-exact, the loss to 1e-5, the raster gradients per
    element within their summation bound, and the post-Adam parameters and
    moments bit-exact against the golden model's projection backward and
    Adam applied to the step's own raster gradients."""
    from msplat import synthetic as S
    from msplat import device as D

    scene = S.make_scene(workload, num_cameras=2).as_3dgs()
    print(f"[full step 3dgs] {scene.name}", flush=True)
    c = scene.cameras[0]
    tgt = D.DeviceScene3D.from_scene(scene.jittered(0.01, 4))
    d_gt = D.render3d_to_device(tgt, tgt.camera(c))
    del tgt
    gt = d_gt.numpy().reshape(c.height, c.width, 3)
    ds = D.DeviceScene3D.from_scene(scene)
    loss, nis = D.train_step3d(ds, ds.camera(c), d_gt)
    n = scene.n
    g_off = eng.last("tile_offsets")
    g_ids = eng.last("gaussian_ids")
    g_img = eng.last("out_img", (c.height, c.width, 3))
    g9 = np.ascontiguousarray(eng.last("grads16", (n, 16))[:, :9])
    got = [p.numpy() for p in ds.params]
    got_m = [m.numpy() for m in ds.exp_avg]
    got_s = {k: a.numpy() for k, a in (("grad_norm", ds.grad_norm), ("vis", ds.vis), ("max2d", ds.max2d))}
    del ds
    print(f"[full step 3dgs] gpu loss {loss:.6f}, {nis} intersections; running the golden model", flush=True)
    ocam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    pre = {k: np.ascontiguousarray(v, np.float32) for k, v in zip(GROUPS, scene.params())}
    proj, bins, fwd = _oracle_render(orc, pre, ocam, scene.background)
    assert nis == bins["num_intersections"]
    assert np.array_equal(g_off, bins["tile_offsets"]), "tile offsets differ"
    assert np.array_equal(g_ids, bins["ids"]), "per-tile sorted ids differ"
    assert np.array_equal(g_img, fwd["out_img"]), f"image differs in {int((g_img != fwd['out_img']).sum())} entries"
    loss_o, dL, _, _ = orc.loss_fwd_bwd(fwd["out_img"], gt, lambda_l1=0.8, lambda_dssim=0.2)
    assert abs(loss - loss_o) <= 1e-5 * abs(loss_o)
    g_o, a_o = orc.raster3d_bwd(proj, bins, fwd, ocam, pre["opacities"], scene.background, dL, with_abs=True)
    del fwd, bins
    err = np.abs(g9.astype(np.float64) - g_o)
    bound = raster_bound(g_o, a_o)
    print(f"[full step 3dgs] raster gradients: worst err/bound {float((err / bound).max()):.3g}", flush=True)
    assert (err <= bound).all()
    record("raster_grads", f"{scene.name} grads9", worst_err_over_bound=float((err / bound).max()),
           **literal_rel(g9, g_o))
    del a_o, err, bound
    ref = orc.project3d_bwd(pre, ocam, scene.sh_degree, scene.sh_degree, proj["radii"], g9)
    if os.environ.get("MSPLAT_PARITY_LOG"):
        # the literal bars against the golden model's own step (its raster
        # gradients through its projection backward and Adam)
        own = orc.project3d_bwd(pre, ocam, scene.sh_degree, scene.sh_degree, proj["radii"],
                                np.ascontiguousarray(g_o, np.float32))
        own_g = [own["dmeans"], own["dscales"], own["dquats"], own["dfdc"], own["dfrest"],
                 np.ascontiguousarray(g_o[:, 5:6], np.float32)]
        adam0 = D.DeviceScene3D(dict(zip(GROUPS, [p[:1] for p in scene.params()])), scene.background).adam_struct()
        for gi, name in enumerate(GROUPS):
            gg = [ref["dmeans"], ref["dscales"], ref["dquats"], ref["dfdc"], ref["dfrest"], g9[:, 5:6]][gi]
            record("param_grads", f"{scene.name} {name}", **literal_rel(np.asarray(gg).reshape(-1),
                                                                        np.asarray(own_g[gi]).reshape(-1)))
            par = pre[name].copy()
            mm = np.zeros_like(par)
            vv = np.zeros_like(par)
            orc.adam(par, np.ascontiguousarray(own_g[gi], np.float32).reshape(par.shape), mm, vv,
                     adam0.step_size[gi], adam0.beta1, adam0.beta2, adam0.bc2_sqrt, adam0.eps)
            diff = np.abs(got[gi].astype(np.float64).reshape(-1) - par.reshape(-1))
            record("post_adam", f"{scene.name} {name}", elements=int(diff.size), beyond_1e5=int((diff > 1e-5).sum()),
                   max_abs_diff=float(diff.max()))
        del own, own_g
    del g_o
    grads = [ref["dmeans"], ref["dscales"], ref["dquats"], ref["dfdc"], ref["dfrest"], np.ascontiguousarray(g9[:, 5:6])]
    adam = D.DeviceScene3D(dict(zip(GROUPS, [p[:1] for p in scene.params()])), scene.background).adam_struct()
    for g, name in enumerate(GROUPS):
        par = pre[name].copy()
        m = np.zeros_like(par)
        v = np.zeros_like(par)
        orc.adam(par, np.ascontiguousarray(grads[g], np.float32).reshape(par.shape), m, v, adam.step_size[g],
                 adam.beta1, adam.beta2, adam.bc2_sqrt, adam.eps)
        assert np.array_equal(got[g], par), name
        assert np.array_equal(got_m[g], m), name
    for k in got_s:
        assert np.array_equal(got_s[k], ref[k]), k


def test_empty_and_culled_scenes_3dgs(orc, eng):
    """No Gaussians, and Gaussians all behind the camera: the frame is the
    background, no intersection is emitted, and a training step gives a
    finite loss, zero raster gradients and unchanged parameters."""
    from msplat import _engine as E
    from msplat import device as D
    p, c = _scene(5, 300, 64, 48)
    bg = np.float32([0.3, 0.6, 0.9])
    ocam, gcam = _cams(orc, eng, c)
    gt = E.DeviceArray.from_numpy(np.full((48, 64, 3), 0.5, np.float32))
    empty = {k: v[:0] for k, v in p.items()}
    behind = dict(p)
    behind["means"] = p["means"] + np.float32([0.0, 0.0, 5.0])  # the camera sits at z = 3.2 looking down -z
    for name, params in (("empty", empty), ("behind", behind)):
        ds = D.DeviceScene3D(params, bg)
        out = D.render3d(ds, gcam)
        assert out["num_intersections"] == 0, name
        assert np.array_equal(out["out_img"], np.broadcast_to(bg, out["out_img"].shape)), name
        loss, nis = D.train_step3d(ds, gcam, gt)
        assert nis == 0 and np.isfinite(loss), name
        if params["means"].shape[0]:
            assert np.array_equal(eng.last("radii", (300,)), np.zeros(300, np.int32))
            assert not eng.last("grads16", (300, 16))[:, :9].any()
            for g, k in enumerate(GROUPS):
                assert np.array_equal(ds.params[g].numpy(), params[k]), k
