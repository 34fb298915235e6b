"""The benchmark workloads at their full sizes on the GPU.

Each workload's full train step is compared with the golden model on the
same inputs (the headline 3M-splat step takes the golden model about 20 s
on the box's host cores), stage by stage: tile offsets and ids, the image,
the loss, the raster gradients and the post-Adam parameters (the bars of
tests/parity.py).  Besides, at 1M splats / 1920x1080 (the overflow
workload, tiles far above 2048 entries) and 3M splats / 5187x3361 the
binning is checked against properties that do not depend on the oracle:
  * every tile's entry count equals the number of visible splats whose tile
    rectangle covers it (a 2D difference array over the rectangles),
  * every entry's tile lies in its splat's rectangle,
  * every tile list is strictly ascending in (depth bits << 32 | id), so it
    holds no duplicate and is the reference's sort order,
  * pixels with no contributor are exactly the background, the final
    transmittance lies in (0, 1] and the image is finite,
  * a training step on the full workload gives a finite loss and finite,
    updated parameters.
The densification workload (growth from 200k blob splats through
repeated clone / split / cull over 1500 steps) runs at its size with every
compaction compared bit for bit with the golden model's on the same inputs;
a reduced cycle with a lower threshold checks three compactions quickly.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from msplat import _engine as E  # noqa: E402
from msplat import device as D  # noqa: E402
from msplat import synthetic as S  # noqa: E402


def _device(a):
    return E.DeviceArray.from_numpy(np.ascontiguousarray(a, np.float32))


def _host_rects(xys, radii, tiles_x, tiles_y):
    """get_tile_bbox (msplat_metal.metal:62-92) in float32, as the projection
    computes it: [x0, x1) x [y0, y1) in tiles."""
    r = radii.astype(np.float32) / np.float32(16.0)
    tcx = xys[:, 0] / np.float32(16.0)
    tcy = xys[:, 1] / np.float32(16.0)

    def trunc(v, hi):
        v = np.clip(np.trunc(v.astype(np.float64)), -2.0 ** 31, 2.0 ** 31 - 128)
        return np.clip(v.astype(np.int64), 0, hi)

    x0 = trunc(tcx - r, tiles_x)
    x1 = trunc((tcx + r) + np.float32(1.0), tiles_x)
    y0 = trunc(tcy - r, tiles_y)
    y1 = trunc((tcy + r) + np.float32(1.0), tiles_y)
    return x0, x1, y0, y1


def _check_binning_and_image(ds, cam, scene):
    out = D.render(ds, cam, outputs=("out_img", "final_Ts", "final_idx"))
    tx, ty = cam.tiles_x, cam.tiles_y
    T = tx * ty
    n = scene.n
    radii = E.last("radii")
    xys = E.last("xys", (n, 2))
    depths = E.last("depths")
    offsets = E.last("tile_offsets").astype(np.int64)
    ids = E.last("gaussian_ids")
    I = int(offsets[-1])
    assert I == out["num_intersections"] and ids.size == I
    vis = np.nonzero(radii > 0)[0]
    x0, x1, y0, y1 = _host_rects(xys[vis], radii[vis], tx, ty)
    assert np.all((x1 > x0) & (y1 > y0))
    # per-tile counts from the rectangles
    diff = np.zeros((ty + 1, tx + 1), np.int64)
    np.add.at(diff, (y0, x0), 1)
    np.add.at(diff, (y0, x1), -1)
    np.add.at(diff, (y1, x0), -1)
    np.add.at(diff, (y1, x1), 1)
    counts = np.cumsum(np.cumsum(diff, 0), 1)[:ty, :tx].reshape(-1)
    assert np.array_equal(np.diff(offsets), counts), "tile counts differ from the rectangle enumeration"
    # every entry's tile lies in its splat's rectangle
    rx0 = np.zeros(n, np.int64)
    rx1 = np.zeros(n, np.int64)
    ry0 = np.zeros(n, np.int64)
    ry1 = np.zeros(n, np.int64)
    rx0[vis], rx1[vis], ry0[vis], ry1[vis] = x0, x1, y0, y1
    tile = np.repeat(np.arange(T, dtype=np.int64), counts)
    etx, ety = tile % tx, tile // tx
    assert np.all((rx0[ids] <= etx) & (etx < rx1[ids]) & (ry0[ids] <= ety) & (ety < ry1[ids])), \
        "an entry lies outside its splat's rectangle"
    # strictly ascending (depth bits, id) inside every tile list
    key = (depths.view(np.uint32)[ids].astype(np.uint64) << np.uint64(32)) | ids.astype(np.uint64)
    inside = tile[1:] == tile[:-1]
    assert np.all(key[1:][inside] > key[:-1][inside]), "a tile list is not in (depth, id) order"
    # image
    img, fT, fidx = out["out_img"], out["final_Ts"][..., 0], out["final_idx"][..., 0]
    assert np.isfinite(img).all()
    assert np.all((fT > 0.0) & (fT <= 1.0))
    empty = fidx == 0
    assert np.array_equal(img[empty], np.broadcast_to(scene.background, img[empty].shape))
    return I, counts.max()


def _full_step_finite(ds, scene, cam):
    tgt = D.DeviceScene(scene.jittered(0.01, 3))
    gt = D.render_to_device(tgt, cam)
    before = ds.params[0].numpy()
    loss, nis = D.train_step(ds, cam, gt)
    assert np.isfinite(loss) and loss > 0.0 and nis > 0
    for p in ds.params:
        assert np.isfinite(p.numpy()).all()
    assert np.abs(ds.params[0].numpy() - before).max() > 0.0


def test_overflow_workload_full_size(orc, eng):
    """1M splats at 1920x1080, 40% in a 0.1-unit ball on the optical axis."""
    scene = S.make_scene(4, num_cameras=2)
    print(f"[workload] {scene.name}", flush=True)
    ds = D.DeviceScene(scene)
    cam = ds.camera(scene.cameras[0])
    I, largest = _check_binning_and_image(ds, cam, scene)
    print(f"[workload] {scene.name}: {I} intersections, largest tile {largest}", flush=True)
    assert largest > 2048  # exercises the multi-run sort and merge
    _full_step_finite(ds, scene, cam)


def test_headline_workload_full_size(orc, eng):
    """3M splats, SH degree 3, 5187x3361."""
    scene = S.make_scene(3, num_cameras=2)
    print(f"[workload] {scene.name}", flush=True)
    ds = D.DeviceScene(scene)
    cam = ds.camera(scene.cameras[0])
    I, largest = _check_binning_and_image(ds, cam, scene)
    print(f"[workload] {scene.name}: {I} intersections, largest tile {largest}", flush=True)
    _full_step_finite(ds, scene, cam)


@pytest.mark.parametrize("workload", [2, 3, 4], ids=["500k-1297x840", "3M-5187x3361", "1M-overflow-1920x1080"])
def test_full_step_matches_oracle_full_size(workload, orc, eng):
    """One full train step of a benchmark workload at its full size against
    the golden model on the same inputs: intersection count, tile offsets and
    per-tile ids bit-exact, the image bit-exact, the loss to 1e-5 relative,
    the raster gradients per element within their summation bound, and the
    post-Adam parameters within the range that bound permits (1e-5 wherever
    the gradient is resolved)."""
    from parity import grad_close, param_grad_noise, post_adam_close

    scene = S.make_scene(workload, num_cameras=2)
    print(f"[full step] {scene.name}", flush=True)
    c = scene.cameras[0]
    # the target: the GPU render of the jittered scene (the forward is
    # bit-identical to the golden model's, checked above and in the parity suite)
    tgt = D.DeviceScene(scene.jittered(0.01, 4))
    d_gt = D.render_to_device(tgt, tgt.camera(c))
    del tgt
    gt = d_gt.numpy().reshape(c.height, c.width, 3)
    ds = D.DeviceScene(scene)
    loss, nis = D.train_step(ds, ds.camera(c), d_gt)
    g_off = E.last("tile_offsets")
    g_ids = E.last("gaussian_ids")
    g_img = E.last("out_img", (c.height, c.width, 3))
    g_16 = E.last("grads16", (scene.n, 16))
    got = ds.host_params()
    got_m = [m.numpy() for m in ds.exp_avg]
    del ds
    print(f"[full step] gpu loss {loss:.6f}, {nis} intersections; running the golden model", flush=True)
    ocam = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = [p.copy() for p in scene.params()]
    m6 = [np.zeros_like(p) for p in params]
    v6 = [np.zeros_like(p) for p in params]
    stats = dict(grad_norm=np.zeros(scene.n, np.float32), vis=np.zeros(scene.n, np.float32),
                 max2d=np.zeros(scene.n, np.float32))
    loss_o, img_o, stage_ms, nis_o = orc.train_step(params, m6, v6, ocam, scene.background, gt, scene.sh_degree,
                                                    scene.sh_degree, D.LR_INIT, 1, stats, detail="grads")
    det = stats.pop("detail")
    print(f"[full step] oracle loss {loss_o:.6f}, {nis_o} intersections, {sum(stage_ms) / 1e3:.1f} s", flush=True)
    assert nis == nis_o
    assert np.array_equal(g_off, det["tile_offsets"]), "tile offsets differ"
    assert np.array_equal(g_ids, det["ids"]), "per-tile sorted ids differ"
    assert np.array_equal(g_img, img_o), f"image differs in {int((g_img != img_o).sum())} entries"
    assert abs(loss - loss_o) <= 1e-5 * abs(loss_o)
    grad_close(g_16, det["grads16"], det["grads16_abs"], f"{scene.name} grads16")
    pre = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
               features_dc=scene.features_dc, features_rest=scene.features_rest)
    radii = orc.project_fwd(pre, ocam, scene.sh_degree, scene.sh_degree)["radii"]
    noise = param_grad_noise(orc, pre, ocam, scene.sh_degree, scene.sh_degree, radii, det["grads16"],
                             det["grads16_abs"])
    post_adam_close(D.GROUPS, [got[k] for k in D.GROUPS], params, got_m, m6, noise, D.LR_INIT, label=scene.name)


def test_densify_cycle_bitexact(orc, eng):
    """Clone / split / cull cycles on statistics accumulated by real training
    steps (the densification workload's mechanism at reduced size): three
    rounds of 10 steps + densify, the GPU compaction of all 18 buffers
    compared bit for bit with the golden model's on the same inputs."""
    scene = S.make_scene(5, n=6000, width=320, height=208, num_cameras=4)
    target = D.DeviceScene(scene.jittered(0.02, 5))
    gts = [D.render_to_device(target, target.camera(c)) for c in scene.cameras]
    del target
    strides = [3, 2, 4, 3, 45, 1]
    cap = 120_000
    n = scene.n
    src = [scene.means, scene.scales, scene.quats, scene.features_dc, scene.features_rest, scene.opacities]
    host = [np.zeros(cap * s, np.float32) for s in strides]
    for h, a, s in zip(host, src, strides):
        h[: n * s] = a.reshape(-1)
    ds = D.DeviceScene(scene)
    ds.params = [_device(h) for h in host]
    ds.exp_avg = [E.DeviceArray.zeros(cap * s) for s in strides]
    ds.exp_avg_sq = [E.DeviceArray.zeros(cap * s) for s in strides]
    ds.grad_norm, ds.vis, ds.max2d = (E.DeviceArray.zeros(cap) for _ in range(3))
    rng = S.SplitMix64(1234)
    P6 = C.c_void_p * 6
    counts = [n]
    for cycle in range(3):
        for k in range(10):
            ci = k % len(scene.cameras)
            loss, _ = D.train_step(ds, ds.camera(scene.cameras[ci]), gts[ci])
            assert np.isfinite(loss)
        n = ds.n
        assert 3 * n <= cap
        params = [p.numpy() for p in ds.params]
        m6 = [p.numpy() for p in ds.exp_avg]
        v6 = [p.numpy() for p in ds.exp_avg_sq]
        stats = dict(grad_norm=ds.grad_norm.numpy()[:n].copy(), vis=ds.vis.numpy()[:n].copy(),
                     max2d=ds.max2d.numpy()[:n].copy())
        rs = rng.normal(2 * n * 3).reshape(2 * n, 3).astype(np.float32)
        d_rs = _device(rs)
        newc = C.c_int()
        half = 0.5 * max(scene.cameras[0].width, scene.cameras[0].height)
        args = (2e-5, 0.01, 0.05, 1, 0.005, 0.5, 0.15, 1)
        E.check(E.lib().msplat_hip_densify(n, cap, *args, ds.grad_norm.ptr, ds.vis.ptr, ds.max2d.ptr, half,
                                           P6(*[p.ptr for p in ds.params]), strides[4],
                                           P6(*[p.ptr for p in ds.exp_avg]), P6(*[p.ptr for p in ds.exp_avg_sq]),
                                           d_rs.ptr, C.byref(newc)))
        new_o = orc.densify(n, cap, params, m6, v6, strides[4], stats, rs, grad_thresh=args[0], size_thresh=args[1],
                            screen_thresh=args[2], check_screen=args[3], cull_alpha=args[4], cull_scale=args[5],
                            cull_screen=args[6], check_huge=args[7], half_max_dim=half)
        print(f"[densify] cycle {cycle}: {n} -> gpu {newc.value}, oracle {new_o}", flush=True)
        assert newc.value == new_o
        for i, (d, o) in enumerate(zip(ds.params + ds.exp_avg + ds.exp_avg_sq, params + m6 + v6)):
            s = strides[i % 6]
            got = d.numpy()[: new_o * s]
            bad = got != o[: new_o * s]
            assert not bad.any(), f"cycle {cycle}, buffer {i}: {int(bad.sum())} entries differ"
        ds.n = new_o
        for a in (ds.grad_norm, ds.vis, ds.max2d):
            E.check(E.lib().msplat_hip_memset(a.ptr, 0, cap * 4))
        counts.append(new_o)
    assert counts[-1] != counts[0]
    assert max(counts) > counts[0]  # the scene grew at least once


def test_densify_workload_full_size(orc, eng):
    """The densification workload at its size: 200k blob splats at 1297x840
    trained for 1500 steps under Model::afterTrain's schedule (densify every
    100 steps from step 200, opacity reset at step 100) with grad threshold
    2e-4, cull opacity 0.005 and the capacity rule at 2M splats; every
    compaction compared bit for bit with the golden model's on the GPU's own
    pre-densify state."""
    scene = S.make_scene(5)
    print(f"[densify] {scene.name}", flush=True)
    ds = D.CapacityScene(scene, 4_000_000)
    tgt = D.DeviceScene(scene.jittered(0.01, 0xC0FFEE + 105))
    gts = [D.render_to_device(tgt, tgt.camera(c)) for c in scene.cameras]
    del tgt
    cams = [ds.camera(c) for c in scene.cameras]
    rng = S.SplitMix64(0xC0FFEE + 5)
    half = 0.5 * max(scene.cameras[0].width, scene.cameras[0].height)
    counts = [ds.n]
    for step in range(1, 1501):
        ci = (step - 1) % len(cams)
        loss, _ = D.train_step(ds, cams[ci], gts[ci])
        assert np.isfinite(loss), step
        dens, reset = D.densify_schedule(step, ds.n, 2_000_000, num_cameras=len(cams))
        if dens:
            n = ds.n
            params, m6, v6, stats = ds.state(3 * n)
            rs = rng.normal(2 * n * 3).reshape(2 * n, 3).astype(np.float32)
            new_o = orc.densify(n, 3 * n, params, m6, v6, 45, stats, rs, grad_thresh=0.0002, size_thresh=0.01,
                                screen_thresh=0.05, check_screen=1, cull_alpha=0.005, cull_scale=0.5,
                                cull_screen=0.15, check_huge=0, half_max_dim=half)
            new_g = ds.densify(rs, half, grad_thresh=0.0002, cull_alpha=0.005)
            print(f"[densify] step {step}: {n} -> gpu {new_g}, oracle {new_o}", flush=True)
            assert new_g == new_o
            gp, gm, gv, _ = ds.state()
            for i, (g, o) in enumerate(zip(gp + gm + gv, params + m6 + v6)):
                k = new_o * D.STRIDES[i % 6]
                bad = g[:k] != o[:k]
                assert not bad.any(), f"step {step}, buffer {i}: {int(bad.sum())} of {k} entries differ"
            counts.append(new_g)
        if reset:
            ds.reset_opacity()
        if step % 100 == 0:
            ds.reset_stats()
    print(f"[densify] splat counts per cycle: {counts}", flush=True)
    assert len(counts) >= 4 and counts[-1] >= 2_000_000
    assert all(b > a for a, b in zip(counts, counts[1:]))


def test_loss_forms_agree_full_size(eng):
    """The SSIM + L1 loss at the headline frame size (5187x3361: the
    streaming form's size) against the two-pass form on the same images:
    dL/dimage bit-identical, the loss and the SSIM sum equal up to the fp64
    summation order.  Pins the streaming form at its real shape (97 strips,
    7 row segments per strip) without the golden model's minutes."""
    W, H = 5187, 3361
    print(f"[loss forms] {W}x{H}", flush=True)
    rng = np.random.default_rng(31)
    gt = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    img = np.clip(gt + rng.normal(0.0, 0.05, gt.shape).astype(np.float32), 0.0, 1.0)
    eq = rng.random((H, W)) < 0.1  # exact-equality pixels: sign(0) = 0 in the L1 gradient
    img[eq] = gt[eq]
    d_img, d_gt = _device(img), _device(gt)
    out = {}
    for form in (1, 2):
        E.check(E.lib().msplat_hip_set_loss_form(form))
        try:
            d_dL = E.DeviceArray((H, W, 3))
            loss, ssim = C.c_double(), C.c_double()
            E.check(E.lib().msplat_hip_loss_fwd_bwd(W, H, d_img.ptr, d_gt.ptr, None, 0.8, 0.0, 0.2, d_dL.ptr,
                                                   C.byref(loss), C.byref(ssim)))
            out[form] = (d_dL.numpy(), loss.value, ssim.value)
        finally:
            E.check(E.lib().msplat_hip_set_loss_form(0))
    (dl1, l1, s1), (dl2, l2, s2) = out[1], out[2]
    assert np.isfinite(dl1).all()
    nbad = int((dl1 != dl2).sum())
    assert nbad == 0, f"{nbad} dL/dimage entries differ between the loss forms"
    assert abs(l1 - l2) <= 1e-9 * abs(l2), (l1, l2)
    assert abs(s1 - s2) <= 1e-9 * abs(s2), (s1, s2)
