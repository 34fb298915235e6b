"""The deep-tile rasterizer path (k_raster_deep + k_deep_log): tiles whose
list holds at least the deep threshold of entries are rendered pixel by
pixel instead of by one workgroup, and their wave blend logs are rebuilt
from the pixels' blended lists.  The threshold is lowered so that ordinary
tiles of small scenes take that path; every output must stay bit-identical
to the golden model, the blend logs and checkpoints identical to the
per-tile kernel's, and the backward over them within the parity bounds.
The overflow workload's real deep tiles (lists of up to ~200k entries at
the default threshold) are covered by tests/test_gpu_workloads.py."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent))
sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "msplat-ios_amd"))

pytestmark = pytest.mark.gpu

from msplat import _engine as E  # noqa: E402
from msplat import device as D  # noqa: E402
from msplat import synthetic as S  # noqa: E402
from parity import grad_close  # noqa: E402
from scenes import adversarial  # noqa: E402
from test_gpu_parity import _assert_bitexact, _device, _forward_both  # noqa: E402

OUTPUTS = ("out_img", "final_Ts", "final_idx", "out_depth", "out_normal", "out_alpha", "out_median_depth",
           "out_distortion")

SCENES = {
    "blob40k_sh3": lambda: S.make_scene(2, n=40_000, width=320, height=208, num_cameras=4),
    "adversarial": lambda: adversarial(3000, 21, width=200, height=136),
    "overflow100k": lambda: S.make_scene(4, n=100_000, width=480, height=270, num_cameras=2),
}


class deep_len:
    """Context: tiles with at least `n` list entries take the deep path."""

    def __init__(self, n: int):
        self.n = n

    def __enter__(self):
        E.check(E.lib().msplat_hip_set_deep_tile_len(self.n))

    def __exit__(self, *exc):
        E.check(E.lib().msplat_hip_set_deep_tile_len(0))


def _logs(offsets):
    """Per (tile, wave) log entries [0, count) and checkpoints of the last
    forward that wrote a blend log (gathered from the pool chunks through
    each wave's chunk table)."""
    T = offsets.size - 1
    cnt = E.last("wave_counts").reshape(T, 4)
    log = E.last("blend_log").reshape(-1, 64, 4)
    ck = E.last("blend_ckpt").reshape(-1, 64)
    table = E.last("blend_chunks")
    ents, cks = [], []
    for t in range(T):
        s0, ln = int(offsets[t]), int(offsets[t + 1] - offsets[t])
        for w in range(4):
            tb = (4 * s0 + w * ln) // 64 + 4 * t + w
            c = int(cnt[t, w])
            chunks = table[tb:tb + (c + 63) // 64]
            if c:
                ents.append(log[chunks].reshape(-1, 4)[:c])
            for k in range(64, c + 1, 64):
                cks.append(ck[chunks[k // 64 - 1]])
    return cnt, np.concatenate(ents) if ents else np.zeros((0, 4), np.int32), \
        np.concatenate(cks) if cks else np.zeros(0, np.float32)


@pytest.mark.parametrize("name", list(SCENES))
def test_deep_path_forward_bitexact(name, orc, eng):
    """The longer half of the tile lists through the deep path: all eight
    forward outputs bit-identical to the golden model."""
    scene = SCENES[name]()
    counts = orc.render(scene, 0)[2]["tile_counts"]
    thr = int(np.median(counts[counts > 0])) + 1
    print(f"[deep fwd] scene={name} deep tiles: lists of {thr} entries or more", flush=True)
    assert (counts >= thr).sum() > 0 and ((counts > 0) & (counts < thr)).sum() > 0  # both paths run
    with deep_len(thr):
        ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
    for k in OUTPUTS:
        _assert_bitexact(out[k], fwd[k], k)


@pytest.mark.parametrize("name", list(SCENES))
def test_deep_path_blend_log_identical(name, orc, eng):
    """The blend logs, checkpoints and entry counts rebuilt for deep tiles
    equal those the per-tile kernel writes, entry for entry; the backward
    over them matches the golden model within the parity bounds."""
    scene = SCENES[name]()
    print(f"[deep log] scene={name}", flush=True)
    ocam, proj, bins, fwd = orc.render(scene, 0)
    target = scene.jittered(0.01, 99)
    gt = orc.render(target, 0)[3]["out_img"]
    _, dL, _, _ = orc.loss_fwd_bwd(fwd["out_img"], gt)
    g_o, a_o = orc.raster_bwd(proj, bins, fwd, ocam, scene.background, dL, with_abs=True)
    ds = D.DeviceScene(scene)
    gcam = ds.camera(scene.cameras[0])
    d_dL = _device(dL)
    offsets = bins["tile_offsets"]
    res = {}
    for thr in (1 << 30, 16):
        with deep_len(thr):
            D.render(ds, gcam, outputs=())
            g16 = E.DeviceArray.zeros((scene.n, 16))
            # the backward replays the forward with the blend log first
            E.check(E.lib().msplat_hip_raster_bwd(d_dL.ptr, None, None, None, None, None, g16.ptr))
            res[thr] = _logs(offsets) + (g16.numpy(),)
    (c0, e0, k0, g0), (c1, e1, k1, g1) = res[1 << 30], res[16]
    assert c0.sum() > 0
    _assert_bitexact(c1, c0, "entries per wave log")
    _assert_bitexact(e1, e0, "blend log entries")
    _assert_bitexact(k1, k0, "transmittance checkpoints")
    grad_close(g1, g_o, a_o, "grads16 over the deep-path logs")


def test_deep_path_all_upstream_gradients(orc, eng):
    """The general backward (depth, alpha, normal, median and distortion
    gradients besides the image's) after a full-output deep-path forward."""
    scene = S.make_scene(2, n=20_000, width=256, height=160, num_cameras=2)
    with deep_len(32):
        ocam, proj, bins, fwd, ds, gcam, out = _forward_both(scene, 0, orc, eng)
        H, W = gcam.height, gcam.width
        rng = S.SplitMix64(12)
        up = dict(img=rng.normal(H * W * 3, 0, 1e-3).reshape(H, W, 3),
                  depth=rng.normal(H * W, 0, 1e-3).reshape(H, W), alpha=rng.normal(H * W, 0, 1e-3).reshape(H, W),
                  normal=rng.normal(H * W * 3, 0, 1e-3).reshape(H, W, 3),
                  median=rng.normal(H * W, 0, 1e-3).reshape(H, W), dist=rng.normal(H * W, 0, 1e-2).reshape(H, W))
        g_o, a_o = orc.raster_bwd(proj, bins, fwd, ocam, scene.background, up["img"], up["depth"], up["alpha"],
                                  up["normal"], up["median"], up["dist"], with_abs=True)
        dev = {k: _device(v) for k, v in up.items()}
        g16 = E.DeviceArray.zeros((scene.n, 16))
        E.check(E.lib().msplat_hip_raster_bwd(dev["img"].ptr, dev["depth"].ptr, dev["alpha"].ptr,
                                              dev["normal"].ptr, dev["median"].ptr, dev["dist"].ptr, g16.ptr))
    for k in OUTPUTS:
        _assert_bitexact(out[k], fwd[k], k)
    grad_close(g16.numpy(), g_o, a_o, "grads16 with all upstream gradients (deep path)")


def test_deep_path_train_step(orc, eng):
    """A fused training step with the deep path on most tiles: image
    bit-exact, loss equal, post-Adam parameters within their bounds (the
    trainer-level check of tests/test_gpu_parity.py)."""
    import test_gpu_parity as T
    with deep_len(48):
        T.test_train_step_matches_oracle(orc, eng)
