"""Benchmark: the full 2DGS training step (projection + SH, binning, per-tile
sort, rasterize, SSIM + L1, backward, fused Adam on six groups) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload 3] [--gpus 1]

Default workload: 3M splats, SH degree 3, 5187x3361 (the train-step
configuration of the headline metric).  Inputs are synthetic (seeded blob
mixture, 32 orbit cameras; targets are renders of the scene with jittered
means) and resident in HBM before the timed region.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "msplat-ios_amd"))

METRIC = "train steps/s @3M splats 5187x3361; render FPS; % HBM peak per kernel"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E


def algorithmic_bytes(stage: str, N: int, I: int, P: int, T: int) -> float:
    """Compulsory HBM bytes of one launch of each stage of a fused fp32 2DGS
    step (N splats, I tile intersections, P pixels, T tiles): projection
    232 B in + 80 B out per splat; binning 32 B per splat + 8 B per
    intersection + 12 B per tile, sorting 12 B per intersection + 8 B per
    tile; raster forward 76 B per intersection + 20 B per pixel (the
    training forward produces the image, the final transmittance and the
    last contributor; the other per-pixel outputs are made on demand); SSIM + L1
    36 B per pixel; raster backward 140 B per intersection + 16 B per pixel
    (the final transmittance and dL/dimage) + 64 B per splat; projection
    backward fused with Adam 1716 B per splat."""
    return {
        "project_fwd": 312.0 * N,
        "tile_scan": 12.0 * T,
        "scatter_sort": 32.0 * N + 20.0 * I + 8.0 * T,
        "raster_fwd": 76.0 * I + 20.0 * P,
        "ssim_l1": 36.0 * P,
        "raster_bwd": 140.0 * I + 16.0 * P + 64.0 * N,
        "project_bwd_adam": 1716.0 * N,
    }.get(stage, 0.0)


def measured_traffic(stage: str, workload: str):
    """HBM bytes per launch of `stage` on `workload` from the committed
    rocprofv3 --pmc summaries (FETCH_SIZE + WRITE_SIZE, scaled by the
    copy-kernel calibration); None when no summary covers it."""
    for f in sorted((REPO / "profiles").glob("*.md")):
        for line in f.read_text().splitlines():
            if line.startswith("bench-traffic:"):
                rec = json.loads(line.split(":", 1)[1])
                if rec.get("stage") == stage and rec.get("workload") == workload:
                    return rec["bytes"]
    return None


def copy_calibration(mib: int) -> int:
    """A plain device-to-device copy of `mib` MiB, three times: the reference
    kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the HBM traffic
    figures (each launch reads and writes exactly mib MiB)."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 3}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run the copy kernel used to calibrate rocprofv3 byte counters")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=3)
    ap.add_argument("--render-frames", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=16)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the training step is single-GPU (one camera per step); "
              "multi-GPU runs are not supported.", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)

    from msplat import _engine as E
    from msplat import device as D
    from msplat import synthetic as S

    E.init()
    t0 = time.time()
    scene = S.make_scene(args.workload)
    target_scene = scene.jittered(0.01, 0xC0FFEE + 100 + args.workload)
    print(f"[bench] scene {scene.name}: n={scene.n} generated in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    ds = D.DeviceScene(scene)
    tgt = D.DeviceScene(target_scene)
    cams = [ds.camera(c) for c in scene.cameras]
    gts = [D.render_to_device(tgt, c) for c in cams]
    del tgt
    E.sync()
    W, H = scene.cameras[0].width, scene.cameras[0].height
    P = W * H
    T = cams[0].tiles_x * cams[0].tiles_y
    print(f"[bench] targets rendered; warmup {args.warmup}", file=sys.stderr, flush=True)

    for k in range(args.warmup):
        D.train_step(ds, cams[k % len(cams)], gts[k % len(cams)])
    # HIP events on the engine stream bracket every stage of every timed step
    E.enable_timing(True)
    E.sync()
    stage_sum: dict[str, float] = {}
    isect = []
    pairs = []
    losses = []
    t_start = time.perf_counter()
    for k in range(args.steps):
        ci = (args.warmup + k) % len(cams)
        loss, nis = D.train_step(ds, cams[ci], gts[ci])
        losses.append(loss)
        isect.append(nis)
        for name, ms in E.stage_times().items():
            stage_sum[name] = stage_sum.get(name, 0.0) + ms
    E.sync()
    t_end = time.perf_counter()
    ms_per_step = (t_end - t_start) * 1e3 / args.steps
    print(f"[bench] {args.steps} steps: {ms_per_step:.2f} ms/step, loss {losses[0]:.4f} -> {losses[-1]:.4f}",
          file=sys.stderr, flush=True)

    # two untimed steps with the raster pair counter on (work per kernel)
    E.enable_timing(False, pairs=True)
    for k in range(2):
        ci = (args.warmup + args.steps + k) % len(cams)
        D.train_step(ds, cams[ci], gts[ci])
        pairs.append(E.raster_counts())

    # render-only frames (the FPS half of the metric)
    E.enable_timing(False)
    for k in range(3):
        D.render(ds, cams[k % len(cams)], outputs=())
    E.sync()
    r0 = time.perf_counter()
    for k in range(args.render_frames):
        n = E.C.c_int64()
        E.check(E.lib().msplat_hip_render(E.C.byref(cams[k % len(cams)]), E.C.byref(ds.gaussians),
                                          ds.background.ptr, E.C.byref(n)))
    E.sync()
    render_ms = (time.perf_counter() - r0) * 1e3 / max(args.render_frames, 1)

    N = scene.n
    I = float(np.mean(isect))
    kernels = {}
    for name, tot in stage_sum.items():
        avg = tot / args.steps
        b = algorithmic_bytes(name, N, int(I), P, T)
        gbs = b / (avg * 1e-3) / 1e9 if avg > 0 else 0.0
        kernels[name] = {"ms": round(avg, 4), "algorithmic_GB": round(b / 1e9, 4), "GB_per_s": round(gbs, 1),
                         "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    dominant = max(kernels, key=lambda k: kernels[k]["ms"])
    dk = kernels[dominant]
    for key in ("pairs_evaluated", "pairs_blended", "log_entries", "visits", "visit_slots"):
        kernels["raster_fwd"][key] = int(np.mean([c[key] for c in pairs]))

    result = {
        "metric": METRIC,
        "value": round(1000.0 / ms_per_step, 4),
        "unit": "train steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": scene.name, "splats": N, "width": W, "height": H, "sh_degree": scene.sh_degree,
                   "tiles": T, "intersections_mean": int(I), "cameras": len(cams),
                   "device": E.device_name()},
        "render_fps": round(1000.0 / render_ms, 2) if args.render_frames else None,
        "render_ms": round(render_ms, 3),
        "kernels": kernels,
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": dk["GB_per_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": dk["frac_hbm_peak"], "traffic": measured_traffic(dominant, scene.name)},
        "loss_first_last": [round(losses[0], 6), round(losses[-1], 6)],
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(scene, target_scene, args.cpu_threads)
    print(json.dumps(result))
    return 0


def cpu_baseline(scene, target_scene, threads: int) -> dict:
    """The golden model (scalar C++ restatement, OpenMP) timed on this host:
    one full training step of the same workload on camera 0 (the target is
    rendered by the golden model first, untimed)."""
    os.environ["OMP_NUM_THREADS"] = str(threads)
    sys.path.insert(0, str(REPO))
    from oracle import oracle as O

    c = scene.cameras[0]
    cam = O.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    gt = O.render(target_scene, 0)[3]["out_img"]
    params = [p.copy() for p in scene.params()]
    m6 = [np.zeros_like(p) for p in params]
    v6 = [np.zeros_like(p) for p in params]
    stats = dict(grad_norm=np.zeros(scene.n, np.float32), vis=np.zeros(scene.n, np.float32),
                 max2d=np.zeros(scene.n, np.float32))
    t0 = time.perf_counter()
    loss, _, stage_ms, nis = O.train_step(params, m6, v6, cam, scene.background, gt, scene.sh_degree,
                                          scene.sh_degree, (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05), 1, stats)
    dt = time.perf_counter() - t0
    return {"value": round(1.0 / dt, 5), "unit": "train steps/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"1 full step of {scene.name} (camera 0, {nis} intersections) in {dt:.2f} s",
            "stage_ms": [round(x, 1) for x in stage_ms[:7]]}


if __name__ == "__main__":
    sys.exit(main())
