"""The 3DGS mode on the GPU against the golden model: projection records,
tile lists and images bit for bit (also for needle-thin, near-opaque and
off-screen Gaussians, which stress the quadrant masks), raster gradients
within the float-atomic bound, the projection backward bit for bit from
the GPU's own raster gradients, the fused Adam step, and training."""
import numpy as np
import pytest

from parity import raster_bound

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
