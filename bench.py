"""Benchmark: the 2DGS training step (projection + SH, binning, per-tile
sort, rasterize, SSIM + L1, backward, fused Adam on six groups) on one
MI355X, for every synthetic workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-configs] [--no-cpu-baseline]

The headline line (`value`) is the train-step throughput of the 3M-splat,
5187x3361, SH-degree-3 workload; `configs` adds the other workloads:
  C1 forward-16k-256        render FPS
  C2 train-500k-1297x840    train steps/s, render FPS
  C3 train-3M-5187x3361     (the headline) + render FPS through the C ABI
  C4 overflow-1M-1920x1080  train steps/s, render FPS
  C5 densify-200k-1297x840  1500 steps with densification every 100
  C3_shard8                 C3 camera 0 in 8 bands of tile rows, each trained as
                            its own camera: one GPU's share of image-space
                            sharding at its real shape
  C3_3dgs                   the C3 splats as 3D Gaussians in the 3DGS mode
  mesh                      TSDF fusion of 32 depth views + marching cubes, 300^3
each next to the golden model (scalar C++, OpenMP) timed on this host.
Inputs are synthetic (seeded; targets are renders of the scene with
jittered means) and resident in HBM before every timed region.  Prints ONE
JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import gc
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "msplat-ios_amd"))

METRIC = "train steps/s @3M splats 5187x3361; render FPS; % HBM peak per kernel"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
# The vector ALUs' ceiling: MI355X's published FP32 vector peak, 157.3
# TFLOP/s = 256 CUs x 4 SIMDs x 32 FMA lanes x 2 flops x 2.4 GHz, is 32
# lanes per cycle per SIMD, so no wave64 VALU instruction issues in fewer
# than 2 cycles: at most 1024 SIMDs x 2.4 GHz / 2 = 1228.8 G wave-instructions
# per second.  (A plain v_fma_f32 measured 1.3 ns per SIMD with 8 waves, 0.64
# of this ceiling.)
VALU_PEAK_GIPS = 1024 * 2.4 / 2.0
LR = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)
BOUND = {"project_fwd": "hbm", "tile_scan": "latency", "scatter_sort": "hbm", "raster_fwd": "valu",
         "ssim_l1": "valu", "raster_bwd": "valu", "project_bwd_adam": "hbm"}


def algorithmic_bytes(stage: str, N: int, I: int, P: int, T: int) -> float:
    """Compulsory HBM bytes of one launch of each stage (fp32, 2DGS, SH
    degree 3, fused dataflow; N splats, I tile intersections, P pixels, T
    tiles): projection 232 B in + 80 B out per splat; binning 32 B per splat
    + 8 B per intersection + 12 B per tile (count + scan + scatter), the
    per-tile sort 12 B per intersection + 8 B per tile; raster forward 76 B
    per intersection (id + record) + 60 B per pixel (the reference's eight
    per-pixel outputs); SSIM + L1 36 B per pixel; raster backward 140 B per
    intersection + 60 B per pixel + 64 B per splat (zero fill); projection
    backward fused with Adam 1716 B per splat."""
    return {
        "project_fwd": 312.0 * N,
        "tile_scan": 12.0 * T,
        "scatter_sort": 32.0 * N + 20.0 * I + 8.0 * T,
        "raster_fwd": 76.0 * I + 60.0 * P,
        "ssim_l1": 36.0 * P,
        "raster_bwd": 140.0 * I + 60.0 * P + 64.0 * N,
        "project_bwd_adam": 1716.0 * N,
    }.get(stage, 0.0)


def profile_record(kind: str, stage: str, workload: str):
    """The `bench-<kind>:` records for (stage, workload) from the committed
    rocprofv3 summaries under profiles/, merged over the stage's kernels
    (instruction counts and bytes summed, kernel names joined); None when
    none covers it."""
    recs = []
    for f in sorted((REPO / "profiles").glob("*.md")):
        for line in f.read_text().splitlines():
            if line.startswith(f"bench-{kind}:"):
                rec = json.loads(line.split(":", 1)[1])
                if rec.get("stage") == stage and rec.get("workload") == workload:
                    recs.append(rec)
    if not recs:
        return None
    out = dict(recs[0])
    out["kernel"] = " + ".join(r["kernel"] for r in recs)
    for key in ("valu_insts", "salu_insts", "waves", "bytes"):
        if key in out:
            out[key] = sum(r[key] for r in recs)
    return out


def copy_calibration(mib: int) -> int:
    """A plain device-to-device copy of `mib` MiB through the engine, three
    times: the kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the
    HBM traffic figures (each launch reads and writes exactly mib MiB)."""
    from msplat import _engine as E

    E.init()
    n = mib * (1 << 20)
    src = E.DeviceArray((n,), np.uint8)
    dst = E.DeviceArray((n,), np.uint8)
    E.check(E.lib().msplat_hip_memset(src.ptr, 1, n))
    for _ in range(3):
        E.check(E.lib().msplat_hip_copy(dst.ptr, src.ptr, n))
    E.sync()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 3}))
    return 0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ GPU --
def _timed_steps(E, step, first: int, steps: int, ncams: int):
    """Exactly `steps` train steps (cameras first, first + 1, ... cyclic)
    between two device synchronisations, with the engine's stage timing
    off.  Returns (ms per step, losses, intersection counts)."""
    losses, isect = [], []
    E.enable_timing(False)
    E.sync()
    t0 = time.perf_counter()
    for k in range(steps):
        loss, nis = step((first + k) % ncams)
        losses.append(loss)
        isect.append(nis)
    E.sync()
    return (time.perf_counter() - t0) * 1e3 / steps, losses, isect


def _stage_breakdown(E, step, first: int, steps: int, ncams: int) -> dict[str, float]:
    """Per-stage milliseconds (HIP events on the engine stream around every
    stage) over `steps` further train steps, outside the timed run.  Each
    stage's mean drops its highest and lowest sample when there are five or
    more: the binning stage ends in a host synchronisation, so one step in
    which the host thread stalls there would otherwise move that stage's
    mean many times over."""
    samples: dict[str, list[float]] = {}
    E.enable_timing(True)
    for k in range(steps):
        step((first + k) % ncams)
        for name, ms in E.stage_times().items():
            samples.setdefault(name, []).append(ms)
    E.enable_timing(False)
    out = {}
    for name, v in samples.items():
        v = sorted(v)
        if len(v) >= 5:
            v = v[1:-1]
        out[name] = sum(v) / len(v)
    return out



def gpu_train(workload: int, steps: int, warmup: int, render_frames: int, counters: bool):
    """Train steps (timed between synchronisations, HIP events per stage)
    and device-resident render frames of one workload."""
    from msplat import _engine as E
    from msplat import device as D
    from msplat import synthetic as S

    scene = S.make_scene(workload)
    ds = D.DeviceScene(scene)
    tgt = D.DeviceScene(scene.jittered(0.01, 0xC0FFEE + 100 + workload))
    cams = [ds.camera(c) for c in scene.cameras]
    gts = [D.render_to_device(tgt, c) for c in cams]
    del tgt
    E.sync()
    for k in range(warmup):
        D.train_step(ds, cams[k % len(cams)], gts[k % len(cams)])
    redos = E.log_pool_stats()["redos"]
    ms_per_step, losses, isect = _timed_steps(E, lambda ci: D.train_step(ds, cams[ci], gts[ci]), warmup, steps,
                                              len(cams))
    pool = log_pool(E, redos)
    stage_ms = _stage_breakdown(E, lambda ci: D.train_step(ds, cams[ci], gts[ci]), warmup + steps,
                                min(steps, 10), len(cams))
    out = dict(scene=scene, ds=ds, cams=cams, ms_per_step=ms_per_step, losses=losses,
               isect=float(np.mean(isect)), stage_ms=stage_ms, log_pool=pool)
    if counters:
        # two untimed steps with the raster work counters on
        E.enable_timing(False, pairs=True)
        pairs = []
        for k in range(2):
            ci = (warmup + steps + k) % len(cams)
            D.train_step(ds, cams[ci], gts[ci])
            pairs.append(E.raster_counts())
        E.enable_timing(False)
        out["raster_counts"] = {key: int(np.mean([p[key] for p in pairs])) for key in pairs[0]}
    del gts
    out["render_ms"] = gpu_render_ms(ds, cams, render_frames)
    return out


def log_pool(E, redos_before: int) -> dict:
    """The blend-log pool after the timed steps: the device memory its
    buffers hold in MiB (chunks of 64 16-byte entries and 64 checkpoint
    floats, chunk tables, counts), the last frame's pool and the chunks its
    step claimed, the worst case, and the overflowed (redone) steps among
    the timed ones."""
    st = E.log_pool_stats()
    return {"device_mb": round(st["bytes"] / 2**20, 1), "chunks": st["chunks"], "claimed_last_step": st["taken"],
            "worst_case_chunks": st["worst"], "redone_steps": st["redos"] - redos_before}


def gpu_shard(scene, ds, bands: int, steps: int, warmup: int) -> dict:
    """One GPU's share of image-space sharding at its real shape: camera 0
    of the workload split into `bands` bands of tile rows (as even as the
    tile rows allow), each trained as its own camera (the same intrinsics
    with the principal point moved up by the band's first row, so it
    renders exactly those rows of the full image, against those rows of the
    full target).  Every band projects all splats and runs the projection
    backward with Adam on all of them, as each GPU would after the gradient
    all-reduce; the all-reduce itself and the SSIM halo exchange at band
    edges (zero padding here) are not part of the measured step."""
    from msplat import _engine as E
    from msplat import device as D

    c = scene.cameras[0]
    tgt = D.DeviceScene(scene.jittered(0.01, 0xC0FFEE + 100 + 3))
    full_gt = D.render_to_device(tgt, ds.camera(c))
    del tgt
    tiles_y = (c.height + 15) // 16
    out = []
    for b in range(bands):
        r0, r1 = b * tiles_y // bands, (b + 1) * tiles_y // bands
        y0, hb = 16 * r0, min(16 * (r1 - r0), c.height - 16 * r0)
        cam = E.prepare_camera(c.cam_to_world, c.fx, c.fy, c.cx, c.cy - y0, c.width, hb, ds.sh_degree,
                               ds.sh_degree)
        gt = E.DeviceArray((hb, c.width, 3), ptr=full_gt.ptr + y0 * c.width * 12, owned=False)
        for _ in range(warmup):
            D.train_step(ds, cam, gt)
        ms, losses, isect = _timed_steps(E, lambda ci: D.train_step(ds, cam, gt), 0, steps, 1)
        out.append({"rows": [y0, y0 + hb], "ms_per_step": round(ms, 3), "intersections": int(np.mean(isect))})
    del full_gt
    return {"workload": f"{scene.name}, camera 0 in {bands} bands of tile rows (one band per GPU)",
            "bands": out, "steps_per_band": steps,
            "max_ms_per_step": max(r["ms_per_step"] for r in out),
            "sum_ms_per_step": round(sum(r["ms_per_step"] for r in out), 3),
            "excluded": "the all-reduce of the per-splat raster gradients (16 floats x N) before the projection "
                        "backward, and the SSIM halo exchange at band edges"}


def gpu_train3d(workload: int, steps: int, warmup: int, render_frames: int):
    """The 3DGS mode on a workload's splats as 3D Gaussians (Scene.as_3dgs):
    train steps (msplat_hip_train_step_3dgs, fused Adam) and render frames."""
    from msplat import _engine as E
    from msplat import device as D
    from msplat import synthetic as S

    scene = S.make_scene(workload).as_3dgs()
    ds = D.DeviceScene3D.from_scene(scene)
    tgt = D.DeviceScene3D.from_scene(scene.jittered(0.01, 0xC0FFEE + 100 + workload))
    cams = [ds.camera(c) for c in scene.cameras]
    gts = [D.render3d_to_device(tgt, c) for c in cams]
    del tgt
    E.sync()
    for k in range(warmup):
        D.train_step3d(ds, cams[k % len(cams)], gts[k % len(cams)])
    redos = E.log_pool_stats()["redos"]
    ms_per_step, losses, isect = _timed_steps(E, lambda ci: D.train_step3d(ds, cams[ci], gts[ci]), warmup, steps,
                                              len(cams))
    pool = log_pool(E, redos)
    stage_ms = _stage_breakdown(E, lambda ci: D.train_step3d(ds, cams[ci], gts[ci]), warmup + steps,
                                min(steps, 10), len(cams))
    del gts
    n = E.C.c_int64()
    for k in range(3):
        E.check(E.lib().msplat_hip_render_3dgs(E.C.byref(cams[k % len(cams)]), E.C.byref(ds.gaussians),
                                               ds.background.ptr, E.C.byref(n)))
    E.sync()
    t0 = time.perf_counter()
    for k in range(render_frames):
        E.check(E.lib().msplat_hip_render_3dgs(E.C.byref(cams[k % len(cams)]), E.C.byref(ds.gaussians),
                                               ds.background.ptr, E.C.byref(n)))
    E.sync()
    render_ms = (time.perf_counter() - t0) * 1e3 / max(render_frames, 1)
    return dict(scene=scene, ms_per_step=ms_per_step, losses=losses, isect=float(np.mean(isect)),
                stage_ms=stage_ms, render_ms=render_ms, log_pool=pool)


def gpu_render_ms(ds, cams, frames: int) -> float:
    """Device-resident render-only frames (the image stays in HBM)."""
    from msplat import _engine as E
    from msplat import device as D

    for k in range(3):
        D.render(ds, cams[k % len(cams)], outputs=())
    E.sync()
    n = E.C.c_int64()
    t0 = time.perf_counter()
    for k in range(frames):
        E.check(E.lib().msplat_hip_render(E.C.byref(cams[k % len(cams)]), E.C.byref(ds.gaussians),
                                          ds.background.ptr, E.C.byref(n)))
    E.sync()
    return (time.perf_counter() - t0) * 1e3 / max(frames, 1)


class _StdoutToStderr:
    """Sends what the C++ library prints on stdout (e.g. Model::load's
    message) to stderr for the duration, so this script's stdout stays its
    one JSON line."""

    def __enter__(self):
        sys.stdout.flush()
        self.saved = os.dup(1)
        os.dup2(2, 1)

    def __exit__(self, *exc):
        sys.stdout.flush()
        os.dup2(self.saved, 1)
        os.close(self.saved)


def gpu_c_abi(scene, frames: int, steps: int, warmup: int, ncams: int = 4) -> dict:
    """The reference's public path through the C ABI: a Trainer on a
    dataset of `ncams` of the scene's cameras with host target images
    (renders of the jittered scene), holding the scene's splats (loaded
    from a .msplat checkpoint written at step 30000: SH degree 3 active,
    full resolution, past densification).  Times `steps` msplat_trainer_step
    calls (Trainer::step, msplat_api.mm:106-128: camera choice, prepareCam,
    the fused step, the loss readback, schedulers, afterTrain) after
    `warmup` untimed ones plus one per camera (each camera's target image
    is uploaded to HBM on its first step and cached, as the reference
    caches its Metal buffers), and `frames`
    msplat_trainer_render_pose_to_buffer calls (render + RGBA8 conversion +
    the copy to host memory)."""
    from msplat import _engine as E
    from msplat import capi
    from msplat import device as D
    from msplat import formats

    import shutil

    L = capi.lib()
    cams = scene.cameras[:ncams]
    need = scene.n * 58 * 4 * 3 + (1 << 28)  # parameters and both moments
    dirs = [d for d in ("/dev/shm", tempfile.gettempdir(), str(REPO / "_build")) if os.path.isdir(d)]
    dirs = [d for d in dirs if shutil.disk_usage(d).free > need]
    if not dirs:
        raise RuntimeError(f"no directory with {need >> 20} MiB free for the checkpoint")
    tgt = D.DeviceScene(scene.jittered(0.01, 0xC0FFEE + 103))
    imgs = []
    for c in cams:
        g = D.render_to_device(tgt, tgt.camera(c))
        imgs.append(np.ascontiguousarray(g.numpy().reshape(c.height, c.width, 3), np.float32))
        del g
    del tgt
    gc.collect()
    with tempfile.TemporaryDirectory(dir=dirs[0]) as td:
        ckpt = os.path.join(td, "scene.msplat")
        params = dict(zip(formats.GROUPS, scene.params()))
        formats.write_checkpoint(ckpt, params, scene.sh_degree, step=30000)
        recs = (capi.CameraImage * len(cams))()
        for r, c, img in zip(recs, cams, imgs):
            r.width, r.height, r.fx, r.fy, r.cx, r.cy = c.width, c.height, c.fx, c.fy, c.cx, c.cy
            r.camToWorld[:] = [float(v) for v in c.cam_to_world.reshape(-1)]
            r.rgb = img.ctypes.data
        pts = np.ascontiguousarray(scene.means[:1000], np.float32)
        rgb = np.full((len(pts), 3), 128, np.uint8)
        dset = L.msplat_dataset_create_from_memory(recs, len(cams), pts.ctypes.data, rgb.ctypes.data, len(pts),
                                                   False, 8)
        if not dset:
            raise RuntimeError(capi.last_error())
        cfg = capi.default_config()
        cfg.numDownscales = 0
        tr = L.msplat_trainer_create(dset, cfg)
        if not tr:
            raise RuntimeError(capi.last_error())
        try:
            with _StdoutToStderr():
                if L.msplat_trainer_load_checkpoint(tr, ckpt.encode()) < 0:
                    raise RuntimeError(capi.last_error())
            assert L.msplat_trainer_splat_count(tr) == scene.n
            for _ in range(warmup + len(cams)):
                L.msplat_trainer_step(tr)
            E.sync()
            losses = []
            t0 = time.perf_counter()
            for _ in range(steps):
                st = L.msplat_trainer_step(tr)
                losses.append(st.loss)
            step_ms = (time.perf_counter() - t0) * 1e3 / max(steps, 1)
            assert L.msplat_trainer_splat_count(tr) == scene.n  # no densification on the way
            c0 = cams[0]
            buf = np.zeros((c0.height, c0.width, 4), np.uint8)
            w, h = C.c_int(), C.c_int()
            poses = [np.ascontiguousarray(c.cam_to_world, np.float32).reshape(-1) for c in scene.cameras]
            fp = C.POINTER(C.c_float)
            for k in range(2):
                L.msplat_trainer_render_pose_to_buffer(tr, poses[k].ctypes.data_as(fp), 0, buf.ctypes.data,
                                                       C.byref(w), C.byref(h))
            t0 = time.perf_counter()
            for k in range(frames):
                L.msplat_trainer_render_pose_to_buffer(tr, poses[k % len(poses)].ctypes.data_as(fp), 0,
                                                       buf.ctypes.data, C.byref(w), C.byref(h))
            ms = (time.perf_counter() - t0) * 1e3 / max(frames, 1)
            assert (w.value, h.value) == (c0.width, c0.height)
        finally:
            L.msplat_trainer_destroy(tr)
            L.msplat_dataset_destroy(dset)
    return dict(render_ms=ms, step_ms=step_ms, losses=losses, cameras=len(cams))


def gpu_densify(total_steps: int = 1500, refine_every: int = 100, max_splats: int = 2_000_000,
                cap: int = 4_000_000):
    """The densification workload: training from 200k blob splats at
    1297x840 with Model::afterTrain's schedule (densify every 100 steps from
    step 200, the opacity reset at step 100), grad threshold 2e-4 and cull
    opacity 0.005, and its capacity rule with the 250k cap raised to 2M (no
    densification once N reaches it).  Returns per-cycle timings."""
    from msplat import _engine as E
    from msplat import device as D
    from msplat import synthetic as S

    scene = S.make_scene(5)
    ds = D.CapacityScene(scene, cap)
    tgt = D.DeviceScene(scene.jittered(0.01, 0xC0FFEE + 105))
    gts = [D.render_to_device(tgt, tgt.camera(c)) for c in scene.cameras]
    del tgt
    cams = [ds.camera(c) for c in scene.cameras]
    rng = S.SplitMix64(0xC0FFEE + 5)
    half = 0.5 * max(scene.cameras[0].width, scene.cameras[0].height)
    E.sync()
    cycles = []
    t_cycle = time.perf_counter()
    t_all = t_cycle
    for step in range(1, total_steps + 1):
        ci = (step - 1) % len(cams)
        D.train_step(ds, cams[ci], gts[ci])
        dens, reset = D.densify_schedule(step, ds.n, max_splats, refine_every, num_cameras=len(cams))
        if dens:
            E.sync()
            n0 = ds.n
            rs = rng.normal(2 * n0 * 3).reshape(2 * n0, 3)
            ds.stage_samples(rs)  # the split samples are an input: resident before the timed call
            E.sync()
            td = time.perf_counter()
            ds.densify(None, half, grad_thresh=0.0002, cull_alpha=0.005)
            dms = (time.perf_counter() - td) * 1e3
            now = time.perf_counter()
            cycles.append(dict(step=step, n_before=n0, n_after=ds.n, densify_ms=round(dms, 3),
                               grow_ms=round(ds.last_grow_ms, 3), cycle_ms=round((now - t_cycle) * 1e3, 2)))
            log(f"densify at step {step}: {n0} -> {ds.n} ({cycles[-1]['cycle_ms']:.0f} ms cycle)")
            t_cycle = now
        if reset:
            ds.reset_opacity()
        if step % refine_every == 0:
            ds.reset_stats()
    E.sync()
    total_ms = (time.perf_counter() - t_all) * 1e3
    return dict(scene=scene, cycles=cycles, total_ms=total_ms, n_final=ds.n)


# ------------------------------------------------------------------ CPU --
def mesh_views(n_views: int, W: int, H: int, radius: float, dist: float):
    """Synthetic depth views of a sphere: cameras on a Fibonacci sphere of
    radius `dist` looking at the origin (OpenCV viewmats), each with the
    exact z-depth of its first sphere hit per pixel centre and alpha 1
    there (0 elsewhere) -- the median depth and alpha a render of an opaque
    sphere gives."""
    fx = fy = 1.35 * W
    cx, cy = W / 2, H / 2
    u = (np.arange(W) + 0.5 - cx) / fx
    v = (np.arange(H) + 0.5 - cy) / fy
    d = np.stack(np.broadcast_arrays(u[None, :], v[:, None], np.ones((H, W))), -1)  # camera-frame rays, z = 1
    views = []
    for k in range(n_views):
        z = 1 - 2 * (k + 0.5) / n_views
        phi = k * np.pi * (3 - np.sqrt(5))
        eye = dist * np.array([np.sqrt(1 - z * z) * np.cos(phi), np.sqrt(1 - z * z) * np.sin(phi), z])
        fwd = -eye / np.linalg.norm(eye)
        up0 = np.array([0.0, 0.0, 1.0]) if abs(fwd[2]) < 0.9 else np.array([1.0, 0.0, 0.0])
        right = np.cross(fwd, up0)
        right /= np.linalg.norm(right)
        down = np.cross(fwd, right)
        R = np.stack([right, down, fwd])  # world -> camera rows
        w = d @ R  # world ray directions (z-depth parametrisation)
        a = np.einsum("hwc,hwc->hw", w, w)
        b = 2 * w @ eye
        c = eye @ eye - radius * radius
        disc = b * b - 4 * a * c
        hit = disc >= 0
        t = np.where(hit, (-b - np.sqrt(np.where(hit, disc, 0))) / (2 * a), 0.0)
        vm = np.eye(4)
        vm[:3, :3] = R
        vm[:3, 3] = -R @ eye
        views.append((vm.astype(np.float32), fx, fy, cx, cy, t.astype(np.float32), hit.astype(np.float32)))
    return views


def gpu_mesh(reps: int = 5):
    """TSDF fusion + marching cubes at the reference's fine setting (2 mm
    voxels, 0.3 m bound: a 300^3 grid, model.cpp:641-650) from 32 views of
    1297x840 of a 0.2 m sphere seen from 1 m; entry points timed end to end
    (views uploaded and the triangle count read back, triangles left in
    HBM), median of `reps`."""
    from msplat import _engine as E
    dim, vs, bound, nviews, W, H = 300, 0.002, 0.3, 32, 1297, 840
    origin = [-bound] * 3
    views = mesh_views(nviews, W, H, 0.2, 1.0)
    dev_maps = [(E.DeviceArray.from_numpy(v[5]), E.DeviceArray.from_numpy(v[6])) for v in views]
    dviews = [v[:5] + m for v, m in zip(views, dev_maps)]
    grid = E.DeviceArray((dim, dim, dim, 2)).zero_()
    trunc, athr = 4 * vs, 0.5
    t_tsdf = []
    for r in range(reps + 1):
        grid.zero_()
        E.sync()
        t0 = time.perf_counter()
        E.tsdf_integrate(grid, origin, vs, dviews, trunc, athr)
        if r:
            t_tsdf.append((time.perf_counter() - t0) * 1e3)
    w = grid.numpy()[..., 1]
    updated = int((w > 0).sum())
    del w
    max_tris = 4_000_000
    out = E.DeviceArray((max_tris, 9))
    org = (C.c_float * 3)(*origin)
    n, tot = C.c_int64(), C.c_int64()
    t_mc = []
    for r in range(reps + 1):
        t0 = time.perf_counter()
        E.check(E.lib().msplat_hip_marching_cubes(grid.ptr, dim, dim, dim, org, vs, max_tris, out.ptr, C.byref(n),
                                                   C.byref(tot)))
        if r:
            t_mc.append((time.perf_counter() - t0) * 1e3)
    V, Cc, P = dim ** 3, (dim - 1) ** 3, W * H
    tsdf_ms, mc_ms = float(np.median(t_tsdf)), float(np.median(t_mc))
    # compulsory bytes: each updated voxel read + written once, each view's
    # depth + alpha read once; marching cubes reads the grid once, writes and
    # rereads one case byte per cell, writes 36 B per triangle
    tsdf_bytes = 16.0 * updated + 8.0 * P * nviews
    mc_bytes = 8.0 * V + 2.0 * Cc + 36.0 * n.value
    return {"workload": f"tsdf-mc-{dim}^3-2mm-{nviews}x{W}x{H}", "grid": [dim, dim, dim], "voxel_m": vs,
            "views": nviews, "voxels_updated": updated, "triangles": int(n.value),
            "tsdf_ms": round(tsdf_ms, 3), "tsdf_views_per_s": round(nviews * 1e3 / tsdf_ms, 1),
            "tsdf_gbs": round(tsdf_bytes / tsdf_ms / 1e6, 1),
            "tsdf_hbm_frac": round(tsdf_bytes / tsdf_ms / 1e6 / HBM_PEAK_GBS, 4),
            "mc_ms": round(mc_ms, 3), "mc_gbs": round(mc_bytes / mc_ms / 1e6, 1),
            "mc_hbm_frac": round(mc_bytes / mc_ms / 1e6 / HBM_PEAK_GBS, 4),
            "timing": "entry points end to end (host wall clock, synchronous calls), median of %d" % reps,
            "_views": views, "_origin": origin}


def cpu_mesh(O, m: dict) -> dict:
    """The golden model on the same workload: TSDF fusion of the 32 views
    (OpenMP over z-slices, one view at a time as the reference dispatches
    them) and marching cubes (one thread) over the fused grid."""
    from msplat import _engine as E
    dim = m["grid"][0]
    grid = np.zeros((dim, dim, dim, 2), np.float32)
    t0 = time.perf_counter()
    for vm, fx, fy, cx, cy, depth, alpha in m["_views"]:
        O.tsdf_integrate(grid, m["_origin"], m["voxel_m"], vm, fx, fy, cx, cy, depth, alpha, 4 * m["voxel_m"], 0.5)
    tsdf_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.marching_cubes(grid, m["_origin"], m["voxel_m"], E.mc_table())
    mc_s = time.perf_counter() - t0
    nv = len(m["_views"])
    return {"tsdf": {"value": round(nv / tsdf_s, 3), "unit": "views/s", "cores": O.num_threads(), "kind": "port",
                     "cpu": cpu_model(), "sample": f"the {nv} views over the {dim}^3 grid, once"},
            "mc": {"value": round(1.0 / mc_s, 4), "unit": "grids/s", "cores": 1, "kind": "port", "cpu": cpu_model(),
                   "sample": f"one pass over the fused {dim}^3 grid"}}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle():
    sys.path.insert(0, str(REPO))
    from oracle import oracle as O
    return O


def cpu_train_step_s(O, scene, target_img, reps: int, warm_scene=None, warm_img=None, fwd_s=None) -> list[float]:
    """Seconds per golden-model train step (camera 0), `reps` timed steps
    after one warm-up step (on warm_scene when given, e.g. a smaller one).
    fwd_s (a list) receives each timed step's forward seconds (projection,
    binning and sort, rasterize: a render)."""
    c = scene.cameras[0]
    cam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)

    def one(sc, img, cm):
        params = [p.copy() for p in sc.params()]
        m6 = [np.zeros_like(p) for p in params]
        v6 = [np.zeros_like(p) for p in params]
        stats = dict(grad_norm=np.zeros(sc.n, np.float32), vis=np.zeros(sc.n, np.float32),
                     max2d=np.zeros(sc.n, np.float32))
        t0 = time.perf_counter()
        _, _, stage_ms, _ = O.train_step(params, m6, v6, cm, sc.background, img, sc.sh_degree, sc.sh_degree, LR,
                                         1, stats)
        return time.perf_counter() - t0, float(sum(stage_ms[:3])) / 1e3

    if warm_scene is not None:
        wc = warm_scene.cameras[0]
        one(warm_scene, warm_img, O.prepare_cam(wc.cam_to_world, wc.fx, wc.fy, wc.cx, wc.cy, wc.width, wc.height))
    else:
        one(scene, target_img, cam)
    runs = [one(scene, target_img, cam) for _ in range(reps)]
    if fwd_s is not None:
        fwd_s.extend(r[1] for r in runs)
    return [r[0] for r in runs]


def cpu_train3d_step_s(O, scene, target_img, reps: int) -> list[float]:
    """Seconds per golden-model 3DGS train step (camera 0): projection,
    binning, compositing, SSIM + L1, both backwards and Adam on six groups."""
    c = scene.cameras[0]
    cam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    names = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")
    out = []
    for _ in range(reps):
        params = {k: np.ascontiguousarray(v, np.float32).copy() for k, v in zip(names, scene.params())}
        m = {k: np.zeros_like(v) for k, v in params.items()}
        v = {k: np.zeros_like(x) for k, x in params.items()}
        stats = dict(grad_norm=np.zeros(scene.n, np.float32), vis=np.zeros(scene.n, np.float32),
                     max2d=np.zeros(scene.n, np.float32))
        t0 = time.perf_counter()
        O.train_step3d(params, m, v, cam, scene.background, target_img, scene.sh_degree, scene.sh_degree, LR, 1,
                       stats)
        out.append(time.perf_counter() - t0)
    return out


def cpu_render_s(O, scene, reps: int) -> list[float]:
    O.render(scene, 0)
    out = []
    for _ in range(reps):
        t0 = time.perf_counter()
        O.render(scene, 0)
        out.append(time.perf_counter() - t0)
    return out


def _cpu_render3d_inputs(O, scene):
    c = scene.cameras[0]
    cam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    params = dict(zip(("means", "scales", "quats", "features_dc", "features_rest", "opacities"), scene.params()))
    proj = O.project3d_fwd(params, cam, scene.sh_degree, scene.sh_degree)
    return proj, O.bin_sort(proj, cam), cam, params["opacities"], scene.background


def cpu_cell(O, per_s: list[float], unit: str, sample: str) -> dict:
    med = float(np.median(per_s))
    return {"value": round(1.0 / med, 5), "unit": unit, "cores": O.num_threads(), "kind": "port",
            "cpu": cpu_model(), "median_s": round(med, 4), "runs_s": [round(x, 3) for x in per_s],
            "sample": sample}


# ----------------------------------------------------------------- main --
def headline_roofline(kernels: dict, workload: str) -> dict:
    """The dominant kernel against HBM: algorithmic bytes per launch over its
    HIP-event duration, against 8 TB/s, with the calibrated FETCH + WRITE
    bytes per launch (traffic) from the committed rocprofv3 summaries.  Its
    VALU issue rate sits beside it (`valu`): executed VALU instructions per
    launch (rocprofv3 SQ_INSTS_VALU, profiles/) over the same duration,
    against the VALU ceiling VALU_PEAK_GIPS."""
    dominant = max(kernels, key=lambda k: kernels[k]["ms"])
    dk = kernels[dominant]
    traffic = profile_record("traffic", dominant, workload)
    cnt = profile_record("counters", dominant, workload)
    out = {"kernel": dominant, "bound": "hbm", "achieved": dk["GB_per_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": dk["frac_hbm_peak"], "traffic": traffic["bytes"] if traffic else None,
           "algorithmic_bytes": round(dk["algorithmic_GB"] * 1e9)}
    if cnt is not None:
        gips = cnt["valu_insts"] / (dk["ms"] * 1e-3) / 1e9
        out["valu"] = {"achieved": round(gips, 1), "peak": round(VALU_PEAK_GIPS, 1),
                       "unit": "G VALU wave-instructions/s", "frac": round(gips / VALU_PEAK_GIPS, 4),
                       "basis": f"{cnt['kernel']}: {cnt['valu_insts']:.4g} VALU instructions per launch "
                                f"(rocprofv3 SQ_INSTS_VALU, profiles/); ceiling 1024 SIMDs x 2.4 GHz / 2 cycles"}
    return out


def kernel_table(stage_ms: dict, N: int, I: int, P: int, T: int, workload: str) -> dict:
    kernels = {}
    for name, ms in stage_ms.items():
        b = algorithmic_bytes(name, N, I, P, T)
        gbs = b / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        row = {"ms": round(ms, 4), "bound": BOUND.get(name, "hbm"), "algorithmic_GB": round(b / 1e9, 4),
               "GB_per_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        cnt = profile_record("counters", name, workload)
        if cnt is not None and ms > 0:
            row["frac_valu_peak"] = round(cnt["valu_insts"] / (ms * 1e-3) / 1e9 / VALU_PEAK_GIPS, 4)
        kernels[name] = row
    return kernels


def issue_table(stage_ms: dict, workload: str) -> dict:
    """Stage times with, where the committed profiles hold the stage's
    kernel counters, the VALU issue fraction and the measured HBM rate (the
    3DGS mode: its algorithmic bytes differ from the 2DGS table's)."""
    out = {}
    for name, ms in stage_ms.items():
        row = {"ms": round(ms, 4), "bound": BOUND.get(name, "hbm")}
        cnt = profile_record("counters", name, workload)
        if cnt is not None and ms > 0:
            row["kernel"] = cnt["kernel"]
            row["frac_valu_peak"] = round(cnt["valu_insts"] / (ms * 1e-3) / 1e9 / VALU_PEAK_GIPS, 4)
        tr = profile_record("traffic", name, workload)
        if tr is not None and ms > 0:
            row["hbm_GB_per_s_measured"] = round(tr["bytes"] / (ms * 1e-3) / 1e9, 1)
        out[name] = row
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run the copy kernel used to calibrate rocprofv3 byte counters")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--render-frames", type=int, default=20)
    ap.add_argument("--no-configs", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-buffer-render", action="store_true",
                    help="skip the render-to-host-buffer frames (e.g. under a profiler)")
    ap.add_argument("--profile-workload", type=int, default=0, metavar="N",
                    help="only run the train steps and render frames of workload N (for a profiler)")
    ap.add_argument("--mesh-only", action="store_true",
                    help="only the mesh workload (TSDF fusion + marching cubes; for a profiler)")
    ap.add_argument("--densify-only", action="store_true",
                    help="only the densification workload (200k -> ~2.8M splats over 1500 steps; for a profiler)")
    ap.add_argument("--3dgs-only", dest="gs3d_only", action="store_true",
                    help="only the 3DGS-mode workload (the C3 splats as 3D Gaussians; for a profiler)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the training step is single-GPU (one camera per step); "
              "multi-GPU runs are not supported.", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    os.environ.setdefault("OMP_NUM_THREADS", str(args.cpu_threads))

    from msplat import _engine as E
    from msplat import synthetic as S

    E.init()
    if args.mesh_only:
        mesh = gpu_mesh()
        print(json.dumps({k: v for k, v in mesh.items() if not k.startswith("_")}))
        return 0
    if args.densify_only:
        d5 = gpu_densify()
        print(json.dumps({"workload": d5["scene"].name, "splats_end": d5["n_final"],
                          "total_s": round(d5["total_ms"] / 1e3, 3), "cycles": d5["cycles"]}))
        return 0
    if args.gs3d_only:
        r = gpu_train3d(3, args.steps, args.warmup, args.render_frames)
        print(json.dumps({"workload": r["scene"].name, "ms_per_step": round(r["ms_per_step"], 3),
                          "render_ms": round(r["render_ms"], 3), "intersections_mean": int(r["isect"]),
                          "blend_log_pool": r["log_pool"],
                          "stage_ms": {k: round(v, 4) for k, v in r["stage_ms"].items()},
                          "loss_first_last": [round(r["losses"][0], 6), round(r["losses"][-1], 6)]}))
        return 0
    if args.profile_workload:
        r = gpu_train(args.profile_workload, args.steps, args.warmup, args.render_frames, counters=False)
        print(json.dumps({"workload": r["scene"].name, "ms_per_step": round(r["ms_per_step"], 3),
                          "render_ms": round(r["render_ms"], 3), "intersections_mean": int(r["isect"]),
                          "blend_log_pool": r["log_pool"],
                          "stage_ms": {k: round(v, 4) for k, v in r["stage_ms"].items()}}))
        return 0
    # ---- headline: C3 ----
    h = gpu_train(3, args.steps, args.warmup, args.render_frames, counters=True)
    scene = h["scene"]
    W, H = scene.cameras[0].width, scene.cameras[0].height
    P = W * H
    T = h["cams"][0].tiles_x * h["cams"][0].tiles_y
    N, I = scene.n, h["isect"]
    log(f"{scene.name}: {h['ms_per_step']:.3f} ms/step, render {h['render_ms']:.3f} ms")
    kernels = kernel_table(h["stage_ms"], N, int(I), P, T, scene.name)
    kernels["raster_fwd"].update(h["raster_counts"])
    shard = None
    if not args.no_configs:
        shard = gpu_shard(scene, h["ds"], 8, 10, 2)
        log(f"{scene.name} in 8 bands: slowest band {shard['max_ms_per_step']:.3f} ms/step, "
            f"all bands {shard['sum_ms_per_step']:.3f} ms")
    del h["ds"]
    gc.collect()
    capi_run = None if args.no_buffer_render else gpu_c_abi(scene, max(args.render_frames // 2, 5),
                                                            max(args.steps // 2, 5), 2)
    buf_ms = capi_run["render_ms"] if capi_run else None
    if capi_run:
        log(f"{scene.name}: render_pose_to_buffer {buf_ms:.3f} ms, msplat_trainer_step {capi_run['step_ms']:.3f} ms")
    result = {
        "metric": METRIC,
        "value": round(1000.0 / h["ms_per_step"], 4),
        "unit": "train steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": scene.name, "splats": N, "width": W, "height": H, "sh_degree": scene.sh_degree,
                   "tiles": T, "intersections_mean": int(I), "cameras": len(h["cams"]),
                   "device": E.device_name()},
        "blend_log_pool": h["log_pool"],
        "render_fps": round(1000.0 / h["render_ms"], 2),
        "render_ms": round(h["render_ms"], 3),
        "render_fps_to_buffer": round(1000.0 / buf_ms, 2) if buf_ms else None,
        "render_ms_to_buffer": round(buf_ms, 3) if buf_ms else None,
        "trainer_step": ({"train_steps_per_s": round(1000.0 / capi_run["step_ms"], 3),
                          "ms_per_step": round(capi_run["step_ms"], 3),
                          "cameras": capi_run["cameras"],
                          "path": "msplat_trainer_step (C ABI), checkpoint of the same splats, host target images"}
                         if capi_run else None),
        "kernels": kernels,
        "roofline": headline_roofline(kernels, scene.name),
        "loss_first_last": [round(h["losses"][0], 6), round(h["losses"][-1], 6)],
    }
    del h

    # ---- the other workloads ----
    configs = {}
    if shard is not None:
        configs["C3_shard8"] = shard
    if not args.no_configs:
        for wl, key in ((2, "C2"), (4, "C4")):
            r = gpu_train(wl, max(args.steps, 30), args.warmup, args.render_frames, counters=False)
            sc = r["scene"]
            Tn = r["cams"][0].tiles_x * r["cams"][0].tiles_y
            Pn = sc.cameras[0].width * sc.cameras[0].height
            configs[key] = {"workload": sc.name, "splats": sc.n, "intersections_mean": int(r["isect"]),
                            "train_steps_per_s": round(1000.0 / r["ms_per_step"], 3),
                            "ms_per_step": round(r["ms_per_step"], 3),
                            "render_fps": round(1000.0 / r["render_ms"], 2),
                            "blend_log_pool": r["log_pool"],
                            "kernels": kernel_table(r["stage_ms"], sc.n, int(r["isect"]), Pn, Tn, sc.name)}
            log(f"{sc.name}: {r['ms_per_step']:.3f} ms/step, render {r['render_ms']:.3f} ms")
            del r
            gc.collect()
        from msplat import device as D
        sc1 = S.make_scene(1)
        ds1 = D.DeviceScene(sc1)
        cams1 = [ds1.camera(c) for c in sc1.cameras]
        r1 = gpu_render_ms(ds1, cams1, 200)
        configs["C1"] = {"workload": sc1.name, "splats": sc1.n, "render_fps": round(1000.0 / r1, 1),
                         "render_ms": round(r1, 4)}
        log(f"{sc1.name}: render {r1:.4f} ms")
        del ds1
        d5 = gpu_densify()
        cyc = d5["cycles"]
        configs["C5"] = {"workload": d5["scene"].name, "steps": 1500, "max_splats": 2_000_000,
                         "densify_cycles": len(cyc),
                         "splats_start": d5["scene"].n, "splats_end": d5["n_final"],
                         "total_s": round(d5["total_ms"] / 1e3, 3),
                         "cycle_ms_mean": round(float(np.mean([c["cycle_ms"] for c in cyc])), 2),
                         "densify_ms_mean": round(float(np.mean([c["densify_ms"] for c in cyc])), 3),
                         "cycles": cyc}
        log(f"{d5['scene'].name}: {d5['scene'].n} -> {d5['n_final']} splats in {d5['total_ms'] / 1e3:.2f} s")
        gc.collect()
        r3 = gpu_train3d(3, max(args.steps // 2, 5), args.warmup, max(args.render_frames // 2, 5))
        sc3 = r3["scene"]
        configs["C3_3dgs"] = {"workload": sc3.name, "splats": sc3.n, "intersections_mean": int(r3["isect"]),
                              "train_steps_per_s": round(1000.0 / r3["ms_per_step"], 3),
                              "ms_per_step": round(r3["ms_per_step"], 3),
                              "render_fps": round(1000.0 / r3["render_ms"], 2),
                              "render_ms": round(r3["render_ms"], 3),
                              "blend_log_pool": r3["log_pool"],
                              "kernels": issue_table(r3["stage_ms"], sc3.name),
                              "loss_first_last": [round(r3["losses"][0], 6), round(r3["losses"][-1], 6)]}
        log(f"{sc3.name}: {r3['ms_per_step']:.3f} ms/step, render {r3['render_ms']:.3f} ms")
        del r3
        gc.collect()
        mesh = gpu_mesh()
        log(f"{mesh['workload']}: TSDF {mesh['tsdf_ms']:.3f} ms, marching cubes {mesh['mc_ms']:.3f} ms, "
            f"{mesh['triangles']} triangles")
        configs["mesh"] = {k: v for k, v in mesh.items() if not k.startswith("_")}
        gc.collect()
        result["configs"] = configs

    # ---- CPU baselines: the golden model on this host ----
    if not args.no_cpu_baseline:
        O = _oracle()
        from msplat import device as D
        warm = S.make_scene(2, n=200_000)
        warm_img = O.render(warm.jittered(0.01, 1), 0)[3]["out_img"]
        gt3 = O.render(scene.jittered(0.01, 0xC0FFEE + 103), 0)[3]["out_img"]
        fwd3 = []
        runs = cpu_train_step_s(O, scene, gt3, args.cpu_reps, warm, warm_img, fwd3)
        result["cpu_baseline"] = cpu_cell(O, runs, "train steps/s",
                                          f"median of {len(runs)} full golden-model steps of {scene.name} "
                                          f"(camera 0) after a warm-up step of 200k splats at 1297x840")
        result["cpu_render_fps"] = cpu_cell(O, fwd3, "render FPS",
                                            f"the forward stages (projection, binning + sort, rasterize) of the "
                                            f"{len(fwd3)} timed steps")
        log(f"cpu {scene.name}: {np.median(runs):.2f} s/step")
        if configs:
            for wl, key in ((2, "C2"), (4, "C4")):
                sc = S.make_scene(wl, num_cameras=1)
                gt = O.render(sc.jittered(0.01, 0xC0FFEE + 100 + wl), 0)[3]["out_img"]
                runs = cpu_train_step_s(O, sc, gt, args.cpu_reps)
                configs[key]["cpu_train"] = cpu_cell(O, runs, "train steps/s",
                                                     f"median of {len(runs)} steps (camera 0) after one warm-up")
                rr = cpu_render_s(O, sc, args.cpu_reps)
                configs[key]["cpu_render"] = cpu_cell(O, rr, "render FPS", f"median of {len(rr)} renders")
                log(f"cpu {sc.name}: {np.median(runs):.2f} s/step")
            sc1 = S.make_scene(1)
            rr = cpu_render_s(O, sc1, 10)
            configs["C1"]["cpu_render"] = cpu_cell(O, rr, "render FPS", f"median of {len(rr)} renders")
            # densify cycle: 100 golden-model steps + one compaction, from a
            # timed step and a timed compaction at the starting size
            sc5 = S.make_scene(5, num_cameras=1)
            gt5 = O.render(sc5.jittered(0.01, 7), 0)[3]["out_img"]
            step_s = float(np.median(cpu_train_step_s(O, sc5, gt5, 1)))
            n5 = sc5.n
            cap = 4 * n5  # the appended count reaches up to 4N
            strides = [3, 2, 4, 3, 45, 1]
            params = [np.zeros(cap * s, np.float32) for s in strides]
            for p, a, s in zip(params, sc5.params(), strides):
                p[: n5 * s] = a.reshape(-1)
            m6 = [np.zeros(cap * s, np.float32) for s in strides]
            v6 = [np.zeros(cap * s, np.float32) for s in strides]
            rng = np.random.default_rng(5)
            stats = dict(grad_norm=rng.uniform(0, 0.05, n5).astype(np.float32),
                         vis=np.ones(n5, np.float32), max2d=rng.uniform(0, 0.1, n5).astype(np.float32))
            rs = rng.normal(size=(2 * n5, 3)).astype(np.float32)
            td = time.perf_counter()
            O.densify(n5, cap, params, m6, v6, 45, stats, rs, grad_thresh=0.0002, cull_alpha=0.005,
                      half_max_dim=648.5)
            dens_s = time.perf_counter() - td
            cyc_s = 100 * step_s + dens_s
            configs["mesh"]["cpu"] = cpu_mesh(O, mesh)
            sc3 = scene.as_3dgs()
            gt3d = O.raster3d_fwd(*_cpu_render3d_inputs(O, sc3.jittered(0.01, 0xC0FFEE + 103)))["out_img"]
            runs = cpu_train3d_step_s(O, sc3, gt3d, 1)
            configs["C3_3dgs"]["cpu_train"] = cpu_cell(O, runs, "train steps/s",
                                                       f"{len(runs)} golden-model 3DGS step of {sc3.name} "
                                                       f"(camera 0) after the 2DGS runs")
            log(f"cpu {sc3.name}: {np.median(runs):.2f} s/step")
            configs["C5"]["cpu_cycle"] = {"value": round(1.0 / cyc_s, 6), "unit": "densify cycles/s",
                                          "cores": O.num_threads(), "kind": "port", "cpu": cpu_model(),
                                          "cycle_s": round(cyc_s, 2),
                                          "sample": f"1 golden-model step ({step_s:.2f} s) and 1 compaction "
                                                    f"({dens_s * 1e3:.0f} ms) at 200k splats, cycle = 100 steps "
                                                    f"+ 1 compaction"}
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
