"""Training dynamics on the GPU against the golden model: thirty steps over
two cameras from the same start, the GPU's fused step against the golden
model's step, for surfels (2DGS) and 3D Gaussians.  Float-atomic gradient
sums make the two runs differ in the last bits from the first step on;
the check is that this noise stays noise: every step's loss within 1e-4
(relative) of the golden model's (measured: about 1e-6), the loss falling the same way, and the final
parameters close."""
import numpy as np
import pytest

from msplat import device as D
from msplat import synthetic as S

pytestmark = pytest.mark.gpu

STEPS = 30


def _gt(orc, scene, cam_index, three_d):
    tgt = scene.jittered(0.02, 99)
    c = tgt.cameras[cam_index]
    ocam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(zip(D.GROUPS, tgt.params()))
    if three_d:
        proj = orc.project3d_fwd(params, ocam, 3, 3)
        bins = orc.bin_sort(proj, ocam)
        return orc.raster3d_fwd(proj, bins, ocam, params["opacities"], tgt.background)["out_img"]
    return orc.render(tgt, cam_index)[3]["out_img"]


@pytest.mark.parametrize("three_d", [False, True], ids=["2dgs", "3dgs"])
def test_thirty_steps_track_the_golden_model(orc, eng, three_d):
    scene = S.make_scene(2, n=12_000, width=192, height=128, num_cameras=2, seed=41)
    if three_d:
        scene = scene.as_3dgs()
    gts = [_gt(orc, scene, k, three_d) for k in range(2)]
    # GPU run
    ds = D.DeviceScene3D.from_scene(scene) if three_d else D.DeviceScene(scene)
    cams = [ds.camera(c) for c in scene.cameras]
    d_gts = [eng.DeviceArray.from_numpy(g) for g in gts]
    step = D.train_step3d if three_d else D.train_step
    gpu = [step(ds, cams[k % 2], d_gts[k % 2])[0] for k in range(STEPS)]
    got = [p.numpy() for p in ds.params]
    # golden-model run
    ocams = [orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height) for c in scene.cameras]
    params = {k: np.ascontiguousarray(v, np.float32).copy() for k, v in zip(D.GROUPS, scene.params())}
    m = {k: np.zeros_like(v) for k, v in params.items()}
    v = {k: np.zeros_like(x) for k, x in params.items()}
    stats = dict(grad_norm=np.zeros(scene.n, np.float32), vis=np.zeros(scene.n, np.float32),
                 max2d=np.zeros(scene.n, np.float32))
    ref = []
    for k in range(STEPS):
        if three_d:
            loss, _, _ = orc.train_step3d(params, m, v, ocams[k % 2], scene.background, gts[k % 2], 3, 3,
                                          D.LR_INIT, k + 1, stats)
        else:
            p6 = [params[g] for g in D.GROUPS]
            loss, _, _, _ = orc.train_step(p6, [m[g] for g in D.GROUPS], [v[g] for g in D.GROUPS], ocams[k % 2],
                                           scene.background, gts[k % 2], 3, 3, D.LR_INIT, k + 1, stats)
        ref.append(loss)
    gpu, ref = np.asarray(gpu), np.asarray(ref)
    rel = np.abs(gpu - ref) / ref
    print(f"[dynamics] {'3dgs' if three_d else '2dgs'}: loss {ref[0]:.5f} -> {ref[-1]:.5f}, "
          f"worst relative gap {rel.max():.2e}", flush=True)
    assert rel.max() < 1e-4
    assert ref[-2:].mean() < 0.8 * ref[:2].mean() and gpu[-2:].mean() < 0.8 * gpu[:2].mean()
    for g, name in enumerate(D.GROUPS):
        o = params[name].reshape(got[g].shape)
        scale = max(1.0, float(np.abs(o).max()))
        diff = np.abs(got[g] - o)
        # parameters stay within a few Adam steps of each other (lr 0.05 for
        # opacities, 1.6e-4 for means): no drift beyond 30 steps' worth
        assert np.quantile(diff, 0.999) <= STEPS * D.LR_INIT[g] * scale, name
