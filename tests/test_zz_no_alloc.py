"""The no-allocation loss entry point (msplat_hip_loss_fwd_bwd_noalloc)
against msplat_hip_loss_fwd_bwd, through the C ABI: dL/dimage, the loss and
the SSIM sum must be bit-identical on two calls in a row (the second on a
smaller image, over the scratch the first left behind), and sizes beyond the
scratch must be refused before any kernel runs."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _images(W, H, seed):
    rng = np.random.default_rng(seed)
    img = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    gt = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    eq = rng.random((H, W)) < 0.25  # exact-equality pixels: sign(0) = 0 in the L1 gradient
    gt[eq] = img[eq]
    return img, gt


def _run(E, fn, W, H, d_img, d_gt, d_dist, ldist):
    d_dL = E.DeviceArray((H, W, 3))
    loss, ssim = C.c_double(), C.c_double()
    rc = fn(W, H, d_img.ptr, d_gt.ptr, d_dist.ptr if d_dist is not None else None, 0.8, ldist, 0.2, d_dL.ptr,
            C.byref(loss), C.byref(ssim))
    E.check(rc)
    return d_dL.numpy(), loss.value, ssim.value


@pytest.mark.parametrize("form", [0, 1], ids=["by_size", "stream"])
def test_noalloc_loss_matches_allocating_entry(form, eng):
    E = eng
    L = E.lib()
    # form 0 picks the two-pass form at these sizes; form 1 forces the streaming one
    E.check(L.msplat_hip_set_loss_form(form))
    try:
        _match_entries(E, L)
    finally:
        E.check(L.msplat_hip_set_loss_form(0))


def _match_entries(E, L):
    # the largest accepted image, then a smaller, ragged one over the same scratch
    for (W, H), seed, ldist in [((2048, 1024), 1, 0.0), ((333, 217), 2, 0.05)]:
        print(f"[no_alloc] {W}x{H} seed {seed}", flush=True)
        img, gt = _images(W, H, seed)
        d_img, d_gt = E.DeviceArray.from_numpy(img), E.DeviceArray.from_numpy(gt)
        d_dist = E.DeviceArray.from_numpy(np.random.default_rng(seed + 10).uniform(0, 1, (H, W)).astype(np.float32))
        want = _run(E, L.msplat_hip_loss_fwd_bwd, W, H, d_img, d_gt, d_dist, ldist)
        got = _run(E, L.msplat_hip_loss_fwd_bwd_noalloc, W, H, d_img, d_gt, d_dist, ldist)
        assert np.array_equal(got[0], want[0]), (W, H)
        assert got[1] == want[1] and got[2] == want[2], (W, H, got[1:], want[1:])
        assert np.isfinite(got[1]) and got[2] > 0


def test_noalloc_loss_refuses_oversized_images(eng):
    E = eng
    L = E.lib()
    tiny = E.DeviceArray((16,))
    loss = C.c_double()
    # checked on the host before any kernel: the buffers are never touched
    for W, H in [(2049, 1024), (1 << 22, 1), (4096, 4096)]:
        rc = L.msplat_hip_loss_fwd_bwd_noalloc(W, H, tiny.ptr, tiny.ptr, None, 0.8, 0.0, 0.2, tiny.ptr,
                                                C.byref(loss), None)
        assert rc == -5, (W, H, rc)
        assert b"scratch" in L.msplat_hip_last_error() or b"tiles" in L.msplat_hip_last_error()
    # and the entry point still works afterwards
    img, gt = _images(64, 48, 3)
    d_img, d_gt = E.DeviceArray.from_numpy(img), E.DeviceArray.from_numpy(gt)
    want = _run(E, L.msplat_hip_loss_fwd_bwd, 64, 48, d_img, d_gt, None, 0.0)
    got = _run(E, L.msplat_hip_loss_fwd_bwd_noalloc, 64, 48, d_img, d_gt, None, 0.0)
    assert np.array_equal(got[0], want[0]) and got[1] == want[1]
