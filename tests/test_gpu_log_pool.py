"""The blend-log pool under overflow.  The rasterizer's per-wave blend logs
are written into a pool of 64-entry chunks sized from the frame's
intersection count; a forward whose logs do not fit marks the pool
overflowed, the backward and the fused Adam of that step skip, and the step
is redone after the pool doubles.  With the pool forced down to a few
chunks every step here overflows at least once: the logs read back through
the chunk tables, the gradients and the post-Adam parameters must be those
of a pool that never overflows (and of the golden model)."""
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
from test_gpu_deep_tiles import _logs, deep_len  # noqa: E402
from test_gpu_parity import _assert_bitexact, _device  # noqa: E402


class pool_chunks:
    """Context: each frame's blend-log pool starts at `n` chunks."""

    def __init__(self, n: int):
        self.n = n

    def __enter__(self):
        E.check(E.lib().msplat_hip_set_log_pool_chunks(self.n))

    def __exit__(self, *exc):
        E.check(E.lib().msplat_hip_set_log_pool_chunks(0))


def _pool_chunks_used() -> int:
    return E.last_ptr("blend_ckpt")[1] // 64


@pytest.mark.parametrize("deep", [False, True], ids=["per-tile", "deep-tiles"])
def test_overflowed_pool_logs_identical(deep, orc, eng):
    """The backward's replay of the forward into a pool of 8 chunks
    overflows and is redone: the logs and checkpoints gathered through the
    chunk tables equal those of an ample pool, and the gradients over them
    match the golden model.  With `deep` the longer half of the lists take
    the deep-tile path, whose log rebuild claims many chunks at once."""
    scene = S.make_scene(2, n=40_000, width=320, height=208, num_cameras=2)
    ocam, proj, bins, fwd = orc.render(scene, 0)
    gt = orc.render(scene.jittered(0.01, 5), 0)[3]["out_img"]
    _, dL, _, _ = orc.loss_fwd_bwd(fwd["out_img"], gt)
    g_o, a_o = orc.raster_bwd(proj, bins, fwd, ocam, scene.background, dL, with_abs=True)
    counts = bins["tile_counts"]
    thr = int(np.median(counts[counts > 0])) + 1 if deep else 1 << 30
    ds = D.DeviceScene(scene)
    gcam = ds.camera(scene.cameras[0])
    d_dL = _device(dL)
    res = {}
    for chunks in (1 << 22, 8):
        print(f"[log pool] deep={deep} pool of {chunks} chunks", flush=True)
        with deep_len(thr), pool_chunks(chunks):
            D.render(ds, gcam, outputs=())
            g16 = E.DeviceArray.zeros((scene.n, 16))
            E.check(E.lib().msplat_hip_raster_bwd(d_dL.ptr, None, None, None, None, None, g16.ptr))
            res[chunks] = _logs(bins["tile_offsets"]) + (g16.numpy(), _pool_chunks_used())
    (c0, e0, k0, g0, u0), (c1, e1, k1, g1, u1) = res[1 << 22], res[8]
    need = int(((c0 + 63) // 64).sum())
    print(f"[log pool] {need} chunks taken; the small pool grew to {u1}", flush=True)
    assert need > 8 * 4 and u1 > 8  # it overflowed at least twice
    _assert_bitexact(c1, c0, "entries per wave log")
    _assert_bitexact(e1, e0, "blend log entries")
    _assert_bitexact(k1, k0, "transmittance checkpoints")
    grad_close(g1, g_o, a_o, "grads16 after pool overflows")


def test_overflowed_pool_train_step(orc, eng):
    """A fused training step (forward, loss, backward, Adam) whose log
    overflows a pool of 8 chunks: nothing of the overflowed attempts
    reaches the parameters, moments or statistics, the redone step matches
    the golden model's (the trainer-level check of tests/test_gpu_parity.py)."""
    import test_gpu_parity as T
    with pool_chunks(8):
        T.test_train_step_matches_oracle(orc, eng)
        assert _pool_chunks_used() > 8


def test_overflowed_pool_train_step_3dgs(orc, eng):
    """The same for the 3DGS training step and its fused Adam."""
    import test_gpu_3dgs as T3
    with pool_chunks(8):
        T3.test_train_step3d_fused_adam_matches_oracle(orc, eng)
        assert _pool_chunks_used() > 8


def test_pool_keeps_grown_size_across_frames(eng):
    """A pool grown by overflows keeps its size for later frames (whose own
    estimate may be smaller): after one pass over the cameras a training
    run does not overflow and redo again."""
    scene = S.make_scene(2, n=20_000, width=256, height=160, num_cameras=3)
    ds = D.DeviceScene(scene)
    cams = [ds.camera(c) for c in scene.cameras]
    gts = [D.render_to_device(ds, c) for c in cams]
    with pool_chunks(8):
        r0 = E.log_pool_stats()["redos"]
        for c, g in zip(cams, gts):
            D.train_step(ds, c, g)
        st = E.log_pool_stats()
        assert st["redos"] > r0 and st["chunks"] > 8
        assert 0 < st["taken"] <= st["chunks"] <= st["worst"] * 2
        for c, g in zip(cams + cams, gts + gts):
            D.train_step(ds, c, g)
            assert E.log_pool_stats()["redos"] == st["redos"]
