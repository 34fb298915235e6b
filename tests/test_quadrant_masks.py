"""The rasterizer's quadrant masks are conservative (CPU).

At load time k_raster_fwd gives each listed splat a 4-bit mask of the 8x8
pixel quadrants of the tile that it can reach (quad_mask on the splat's
MaskRec, the part the projection computes once per splat), and a wave
evaluates only the splats whose bit is set.  That must never drop a pair
the reference would blend: for every (tile, splat) pair the binning
produces, every pixel whose alpha reaches 1/255 in an fp64 evaluation of
the reference's pair test (with a 1e-4 relative margin, far above the fp32
rounding) must lie in a quadrant whose bit is set.  The helper
tests/native/libquadmask.so compiles the product's mask code for the host;
the golden model supplies the projected splats.  The scenes mix the
workload generators with adversarial splats: edge-on, needle-thin, huge,
near the camera, centred off screen, and nearly transparent.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from msplat import synthetic as S
from scenes import adversarial as _adversarial

LIB = Path(__file__).resolve().parent / "native" / "libquadmask.so"


def _lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is missing: build it with `make -C tests/native` (build() does)")
    L = C.CDLL(str(LIB))
    L.qm_check.restype = C.c_int64
    L.qm_check.argtypes = [C.c_int] + [C.c_void_p] * 5 + [C.c_int, C.c_int, C.c_float, C.c_void_p]
    return L


def _check(orc, scene, cam_index=0, tau_scale=1.0):
    cam, proj, _, _ = orc.render(scene, cam_index)
    out = np.zeros(5, np.int64)
    arrs = [np.ascontiguousarray(proj[k]) for k in ("transmats", "xys", "normal_opac", "radii", "rect")]
    misses = _lib().qm_check(scene.n, *[a.ctypes.data for a in arrs], cam.width, cam.height, tau_scale,
                             out.ctypes.data)
    return int(misses), out


CASES = {
    "forward-2k": lambda: S.make_scene(1, n=2000, width=128, height=96),
    "blobs-20k": lambda: S.make_scene(2, n=20_000, width=200, height=136, num_cameras=2),
    "dense-ball": lambda: S.make_scene(4, n=8000, width=160, height=96, num_cameras=2),
    "adversarial-a": lambda: _adversarial(3000, 11),
    "adversarial-b": lambda: _adversarial(3000, 12, width=97, height=61),
    # pixel coordinates in the thousands: the regime where the ray written
    # about the image origin cancels
    "adversarial-wide": lambda: _adversarial(1500, 13, width=1297, height=840),
    "adversarial-c": lambda: _adversarial(2500, 14, width=333, height=250),
}


@pytest.mark.parametrize("name", list(CASES))
def test_quadrant_masks_keep_every_blending_pixel(orc, name):
    misses, out = _check(orc, CASES[name]())
    checked, box_tiles, fine_tiles, box_bits, fine_bits = (int(x) for x in out)
    print(f"[masks] {name}: {checked} pairs checked, box bits {box_bits}, fine bits {fine_bits}")
    assert checked > 0
    assert misses == 0, f"{misses} blending (pixel, splat) pairs fall in masked-out quadrants"
    # the fine test is a refinement of the box test
    assert fine_bits <= box_bits and fine_tiles <= box_tiles


def test_quadrant_masks_prune(orc):
    """The refinement is not vacuous: on the blob workload it clears at
    least a tenth of the quadrant bits the box test sets (about half at the
    3M-splat 5187x3361 workload, where tiles are small against splats)."""
    _, out = _check(orc, CASES["blobs-20k"]())
    assert out[4] < 0.9 * out[3]


def test_planted_miss_is_caught(orc):
    """The checker itself: masks computed from a reach 20% short of the
    true one (a plausible slip in tau or its margin) must be reported."""
    misses, _ = _check(orc, CASES["blobs-20k"](), tau_scale=0.8)
    assert misses > 0


# ---- the 3DGS mode: the alpha >= 1/255 box of each Gaussian ---------------
def _scene3d(seed, n, W, H, kind):
    """3D Gaussians in front of a camera 3.2 units away: 'blobs' (random
    ellipsoids), 'needles' (long, thin, near-opaque, some off screen) or
    'near' (large Gaussians close to the camera)."""
    rng = np.random.default_rng(seed)
    p = dict(means=np.column_stack([rng.uniform(-0.9, 0.9, n), rng.uniform(-0.7, 0.7, n), rng.uniform(-0.8, 0.8, n)]),
             scales=rng.uniform(-3.6, -2.4, (n, 3)), quats=rng.normal(0, 1, (n, 4)),
             opacities=rng.uniform(-1.5, 2.0, (n, 1)), features_dc=rng.uniform(-1, 1, (n, 3)),
             features_rest=np.zeros((n, 15, 3)))
    if kind == "needles":
        p["scales"][:, 0] = rng.uniform(-1.8, -0.8, n)
        p["scales"][:, 1:] = rng.uniform(-7.0, -5.0, (n, 2))
        p["opacities"][:] = rng.uniform(3.0, 9.0, (n, 1))
        p["means"][: n // 3, :2] *= 1.7
    if kind == "near":
        p["means"][:, 2] = rng.uniform(2.2, 2.9, n)  # 0.3 - 1.0 from the camera
        p["scales"] = rng.uniform(-3.0, -1.5, (n, 3))
    p["quats"] /= np.linalg.norm(p["quats"], axis=1, keepdims=True)
    p = {k: np.ascontiguousarray(v, np.float32) for k, v in p.items()}
    c2w = np.eye(4, dtype=np.float32)
    c2w[2, 3] = 3.2
    return p, (c2w, 1.05 * W, 1.1 * W, W / 2 + 0.3, H / 2 - 0.6, W, H)


def _check3d(orc, p, c, tau_scale=1.0):
    cam = orc.prepare_cam(*c)
    proj = orc.project3d_fwd(p, cam, 3, 3)
    out = np.zeros(5, np.int64)
    lib = _lib()
    lib.qm3_check.restype = C.c_int64
    lib.qm3_check.argtypes = [C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_int, C.c_float, C.c_void_p]
    arrs = [np.ascontiguousarray(a) for a in (proj["xys"], proj["conics"], proj["cov2d"], p["opacities"][:, 0],
                                                proj["radii"], proj["rect"])]
    misses = lib.qm3_check(len(p["means"]), *[a.ctypes.data for a in arrs], c[5], c[6], tau_scale, out.ctypes.data)
    return int(misses), out


@pytest.mark.parametrize("kind,seed,n,W,H", [("blobs", 1, 3000, 200, 136), ("needles", 2, 2000, 200, 136),
                                             ("near", 3, 600, 160, 112), ("needles", 4, 1500, 1297, 840)])
def test_gauss3_boxes_keep_every_blending_pixel(orc, kind, seed, n, W, H):
    p, c = _scene3d(seed, n, W, H, kind)
    misses, out = _check3d(orc, p, c)
    print(f"[masks3d] {kind}: {int(out[0])} pairs checked, {int(out[3])} quadrant bits")
    assert out[0] > 0
    assert misses == 0, f"{misses} blending (pixel, Gaussian) pairs fall in masked-out quadrants"


def test_gauss3_box_planted_miss_is_caught(orc):
    """Boxes from a reach 20% short must be reported."""
    p, c = _scene3d(1, 3000, 200, 136, "blobs")
    misses, _ = _check3d(orc, p, c, tau_scale=0.8)
    assert misses > 0
