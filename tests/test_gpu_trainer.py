"""The trainer surface on the GPU: msplat.GaussianTrainer / Dataset (the
reference's Python API), the C ABI of msplat_c_api.h, checkpoints, PLY and
.splat export, densification through the trainer, and one trainer step
checked end to end against the golden model."""
from __future__ import annotations

import ctypes as C
import ctypes.util
import math

import numpy as np
import pytest

from msplat import synthetic as S
from parity import trainer_post_adam_close

pytestmark = pytest.mark.gpu


def _read_gaussian_ply(path):
    """Parses the Gaussian PLY layout written by export_ply."""
    with open(path, "rb") as f:
        names, n = [], 0
        assert f.readline().strip() == b"ply"
        while True:
            line = f.readline().strip().decode()
            if line == "end_header":
                break
            if line.startswith("element vertex"):
                n = int(line.split()[-1])
            if line.startswith("property float"):
                names.append(line.split()[-1])
        rows = np.frombuffer(f.read(), np.float32).reshape(n, len(names))
    col = {k: i for i, k in enumerate(names)}
    nfr = sum(k.startswith("f_rest_") for k in names) // 3
    fr = np.stack([rows[:, col[f"f_rest_{ch * nfr + b}"]] for b in range(nfr) for ch in range(3)], 1)
    ns = sum(k.startswith("scale_") for k in names)
    return dict(means=rows[:, [col["x"], col["y"], col["z"]]], scales=rows[:, [col[f"scale_{i}"] for i in range(ns)]],
                quats=rows[:, [col[f"rot_{i}"] for i in range(4)]],
                features_dc=rows[:, [col[f"f_dc_{i}"] for i in range(3)]],
                features_rest=fr.reshape(n, nfr, 3), opacities=rows[:, [col["opacity"]]], names=names)


def _dataset_inputs(n_cams=4, width=160, height=112, n=4000, seed=3):
    """Synthetic cameras + target images (golden-model renders of a blob
    scene with jittered means) + an initial point cloud."""
    from oracle import oracle as O

    scene = S.make_scene(2, n=n, width=width, height=height, num_cameras=n_cams, seed=seed)
    target = scene.jittered(0.01, 11)
    images = [O.render(target, i)[3]["out_img"] for i in range(n_cams)]
    c2w = np.stack([c.cam_to_world for c in scene.cameras]).astype(np.float32)
    intr = np.array([[c.fx, c.fy, c.cx, c.cy] for c in scene.cameras], np.float32)
    rgb = np.clip((scene.features_dc * 0.28209479 + 0.5) * 255, 0, 255).astype(np.uint8)
    return scene, images, c2w, intr, scene.means.astype(np.float32), rgb


def test_trainer_step_matches_golden_model(tmp_path):
    """Model init -> export -> one GaussianTrainer step -> export, against
    the golden model's train step from the exported initial parameters:
    camera, Adam bias correction and learning rates all go through the
    trainer's own host code."""
    import msplat
    from oracle import oracle as O

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=1)
    ds = msplat.Dataset.from_arrays(images, c2w, intr, xyz, rgb)
    bg = [float(v) for v in scene.background]
    cfg = msplat.TrainingConfig(iterations=100, num_downscales=0, bg_color=bg)
    tr = msplat.GaussianTrainer(ds, cfg)
    tr.export_ply(str(tmp_path / "p0.ply"))
    p0 = _read_gaussian_ply(tmp_path / "p0.ply")
    stats = tr.step()
    tr.export_ply(str(tmp_path / "p1.ply"))
    p1 = _read_gaussian_ply(tmp_path / "p1.ply")
    assert stats.iteration == 1 and stats.splat_count == xyz.shape[0]

    c = scene.cameras[0]
    ocam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    keys = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")
    params = [np.ascontiguousarray(p0[k], np.float32) for k in keys]
    m6 = [np.zeros_like(p) for p in params]
    v6 = [np.zeros_like(p) for p in params]
    st = dict(grad_norm=np.zeros(len(xyz), np.float32), vis=np.zeros(len(xyz), np.float32),
              max2d=np.zeros(len(xyz), np.float32))
    lrs = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)
    loss_o, _, _, _ = O.train_step(params, m6, v6, ocam, np.float32(bg), images[0], 3, 0, lrs, 1, st)
    assert abs(stats.loss - loss_o) <= 1e-5 * abs(loss_o)
    for k, p, m, lr in zip(keys, params, m6, lrs):
        trainer_post_adam_close(k, p1[k], p, m, lr)
    moved = np.abs(p1["means"] - p0["means"]).max()
    assert moved > 0


def test_trainer_training_render_checkpoint(tmp_path):
    import msplat

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=4)
    ds = msplat.Dataset.from_arrays(images, c2w, intr, xyz, rgb, eval_mode=True, test_every=4)
    assert (ds.num_train, ds.num_test) == (3, 1)
    cfg = msplat.TrainingConfig(iterations=1000, num_downscales=1, resolution_schedule=20)
    tr = msplat.GaussianTrainer(ds, cfg)
    losses = [tr.step().loss for _ in range(60)]
    assert all(math.isfinite(x) for x in losses)
    assert np.mean(losses[-5:]) < np.mean(losses[:5])
    assert tr.iteration == 60

    img = tr.render(0)
    assert img.shape == (112, 160, 3) and img.dtype == np.float32
    same = tr.render_from_pose(ds.camera_pose(0), 0)
    assert np.array_equal(img, same)
    with pytest.raises(RuntimeError):
        tr.render(7)
    ev = tr.evaluate()
    assert set(ev) >= {"psnr", "ssim", "l1", "num_test", "num_gaussians"} and ev["num_test"] == 1
    assert math.isfinite(ev["psnr"]) and 0 < ev["ssim"] <= 1

    tr.save_checkpoint(str(tmp_path / "a.msplat"))
    for _ in range(3):
        tr.step()
    assert not np.array_equal(tr.render(0), img)
    tr.load_checkpoint(str(tmp_path / "a.msplat"))
    assert tr.iteration == 60
    assert np.array_equal(tr.render(0), img)

    tr.export_splat(str(tmp_path / "a.splat"))
    assert (tmp_path / "a.splat").stat().st_size == 32 * tr.splat_count


def test_trainer_densify_and_opacity_reset():
    """refine_every 10 after a 10-step warmup, reset interval 30: densify at
    steps 20 and 50, opacity reset at step 40 (model.cpp:240-306)."""
    import msplat

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=4)
    ds = msplat.Dataset.from_arrays(images, c2w, intr, xyz, rgb)
    cfg = msplat.TrainingConfig(iterations=2000, num_downscales=0, refine_every=10, warmup_length=10,
                                reset_alpha_every=3, densify_grad_thresh=1e-6)
    tr = msplat.GaussianTrainer(ds, cfg)
    counts = [tr.step().splat_count for _ in range(55)]
    assert counts[18] == xyz.shape[0]
    assert counts[19] != counts[18]      # densified at step 20
    assert counts[48] == counts[40]      # nothing at steps 30 and 40
    assert counts[49] != counts[48]      # densified at step 50
    assert math.isfinite(tr.step().loss)


class _Cfg(C.Structure):
    _fields_ = [("iterations", C.c_int), ("shDegree", C.c_int), ("shDegreeInterval", C.c_int),
                ("ssimWeight", C.c_float), ("numDownscales", C.c_int), ("resolutionSchedule", C.c_int),
                ("refineEvery", C.c_int), ("warmupLength", C.c_int), ("resetAlphaEvery", C.c_int),
                ("densifyGradThresh", C.c_float), ("densifySizeThresh", C.c_float), ("stopScreenSizeAt", C.c_int),
                ("splitScreenSize", C.c_float), ("keepCrs", C.c_bool), ("downscaleFactor", C.c_float),
                ("bgColor", C.c_float * 3)]


class _CamImg(C.Structure):
    _fields_ = [("width", C.c_int), ("height", C.c_int), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float),
                ("cy", C.c_float), ("camToWorld", C.c_float * 16), ("rgb", C.c_void_p)]


class _Stats(C.Structure):
    _fields_ = [("iteration", C.c_int), ("splatCount", C.c_int), ("msPerStep", C.c_float), ("loss", C.c_float)]


class _Px(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("width", C.c_int), ("height", C.c_int)]


class _Eval(C.Structure):
    _fields_ = [("psnr", C.c_float), ("ssim", C.c_float), ("l1", C.c_float), ("numTest", C.c_int),
                ("numGaussians", C.c_int)]


def test_c_abi_trainer(tmp_path):
    """The reference's C ABI driven through ctypes, as a Swift or C caller
    would (msplat_c_api.h)."""
    from msplat import _engine as E

    lib = E.lib()
    libc = C.CDLL(ctypes.util.find_library("c"))
    lib.msplat_dataset_create_from_memory.restype = C.c_void_p
    lib.msplat_dataset_create_from_memory.argtypes = [C.POINTER(_CamImg), C.c_int, C.c_void_p, C.c_void_p,
                                                      C.c_int64, C.c_bool, C.c_int]
    lib.msplat_trainer_create.restype = C.c_void_p
    lib.msplat_trainer_create.argtypes = [C.c_void_p, _Cfg]
    lib.msplat_trainer_step.restype = _Stats
    lib.msplat_trainer_step.argtypes = [C.c_void_p]
    lib.msplat_trainer_render.restype = _Px
    lib.msplat_trainer_render.argtypes = [C.c_void_p, C.c_int, C.c_bool]
    lib.msplat_trainer_evaluate.restype = _Eval
    lib.msplat_trainer_evaluate.argtypes = [C.c_void_p]
    lib.msplat_trainer_render_pose_to_buffer.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.c_int, C.c_void_p,
                                                         C.POINTER(C.c_int), C.POINTER(C.c_int)]
    lib.msplat_trainer_extract_mesh.restype = C.c_int64
    lib.msplat_trainer_extract_mesh.argtypes = [C.c_void_p, C.c_char_p, C.c_float, C.c_float, C.c_float,
                                                C.c_float]
    for fn in ("msplat_trainer_splat_count", "msplat_trainer_iteration", "msplat_dataset_num_train",
               "msplat_dataset_num_test"):
        getattr(lib, fn).argtypes = [C.c_void_p]
    for fn in ("msplat_trainer_export_ply", "msplat_trainer_export_splat", "msplat_trainer_save_checkpoint",
               "msplat_trainer_load_checkpoint"):
        getattr(lib, fn).argtypes = [C.c_void_p, C.c_char_p]
    lib.msplat_trainer_destroy.argtypes = [C.c_void_p]
    lib.msplat_dataset_destroy.argtypes = [C.c_void_p]
    lib.msplat_last_error.restype = C.c_char_p
    libc.free.argtypes = [C.c_void_p]

    scene, images, c2w, intr, xyz, rgb = _dataset_inputs(n_cams=3)
    imgs = [np.ascontiguousarray(i, np.float32) for i in images]
    cams = (_CamImg * 3)()
    for i in range(3):
        cams[i].width, cams[i].height = imgs[i].shape[1], imgs[i].shape[0]
        cams[i].fx, cams[i].fy, cams[i].cx, cams[i].cy = (float(v) for v in intr[i])
        cams[i].camToWorld[:] = [float(v) for v in c2w[i].reshape(-1)]
        cams[i].rgb = imgs[i].ctypes.data
    ds = lib.msplat_dataset_create_from_memory(cams, 3, xyz.ctypes.data, rgb.ctypes.data, len(xyz), True, 3)
    assert ds, lib.msplat_last_error()
    assert (lib.msplat_dataset_num_train(ds), lib.msplat_dataset_num_test(ds)) == (2, 1)

    cfg = _Cfg(iterations=100, shDegree=3, shDegreeInterval=1000, ssimWeight=0.2, numDownscales=0,
               resolutionSchedule=3000, refineEvery=100, warmupLength=500, resetAlphaEvery=30,
               densifyGradThresh=0.0002, densifySizeThresh=0.01, stopScreenSizeAt=4000, splitScreenSize=0.05,
               keepCrs=False, downscaleFactor=1.0)
    cfg.bgColor[:] = [0.613, 0.0101, 0.3984]
    tr = lib.msplat_trainer_create(ds, cfg)
    assert tr, lib.msplat_last_error()
    for k in range(5):
        s = lib.msplat_trainer_step(tr)
        assert s.iteration == k + 1 and s.splatCount == len(xyz) and math.isfinite(s.loss) and s.msPerStep > 0
    assert lib.msplat_trainer_iteration(tr) == 5

    px = lib.msplat_trainer_render(tr, 0, False)
    assert (px.width, px.height) == (imgs[0].shape[1], imgs[0].shape[0])
    img = np.ctypeslib.as_array(px.data, (px.height, px.width, 3)).copy()
    libc.free(C.cast(px.data, C.c_void_p))
    bad = lib.msplat_trainer_render(tr, 9, False)
    assert not bad.data and bad.width == 0

    pose = (C.c_float * 16)(*[float(v) for v in c2w[cams_train_index(0)].reshape(-1)])
    w, h = C.c_int(), C.c_int()
    lib.msplat_trainer_render_pose_to_buffer(tr, pose, 0, None, C.byref(w), C.byref(h))
    assert (w.value, h.value) == (px.width, px.height)
    buf = np.zeros((h.value, w.value, 4), np.uint8)
    lib.msplat_trainer_render_pose_to_buffer(tr, pose, 0, buf.ctypes.data, C.byref(w), C.byref(h))
    expect = (np.clip(img, 0, 1) * np.float32(255)).astype(np.uint8)
    assert np.array_equal(buf[..., :3], expect) and np.all(buf[..., 3] == 255)

    ev = lib.msplat_trainer_evaluate(tr)
    assert ev.numTest == 1 and math.isfinite(ev.psnr)
    lib.msplat_trainer_export_ply(tr, str(tmp_path / "c.ply").encode())
    lib.msplat_trainer_export_splat(tr, str(tmp_path / "c.splat").encode())
    assert (tmp_path / "c.splat").stat().st_size == 32 * len(xyz)
    assert _read_gaussian_ply(tmp_path / "c.ply")["means"].shape == (len(xyz), 3)
    lib.msplat_trainer_save_checkpoint(tr, str(tmp_path / "c.msplat").encode())
    assert lib.msplat_trainer_load_checkpoint(tr, str(tmp_path / "c.msplat").encode()) == 5
    assert lib.msplat_trainer_load_checkpoint(tr, str(tmp_path / "missing.msplat").encode()) == -1
    assert b"Cannot open checkpoint" in lib.msplat_last_error()
    ntri = lib.msplat_trainer_extract_mesh(tr, str(tmp_path / "m.ply").encode(), 0.02, 1.0, 0.5, 4.0)
    assert ntri > 0
    head = (tmp_path / "m.ply").read_bytes()[:400]
    assert f"element face {ntri}".encode() in head
    assert lib.msplat_trainer_extract_mesh(tr, b"/nonexistent-dir/m.ply", 0.02, 1.0, 0.5, 4.0) == -1
    assert lib.msplat_last_error()
    lib.msplat_trainer_destroy(tr)
    lib.msplat_dataset_destroy(ds)


def cams_train_index(k: int) -> int:
    """Index into the 3 in-memory cameras of training camera k when camera 0
    is held out (test_every = 3)."""
    return [1, 2][k]
