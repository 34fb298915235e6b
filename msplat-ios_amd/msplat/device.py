"""Device-resident scene state and one-call wrappers over the engine's render
and training-step entry points (Model::render / Model::fullIteration,
core/src/model.cpp:546-554 and 762-829, driven from Python)."""
from __future__ import annotations

import ctypes as C
import math
import struct

import time

import numpy as np

from . import _engine as E
from .synthetic import Camera, Scene

def _f32(x: float) -> float:
    """x rounded to float32."""
    return struct.unpack("f", struct.pack("f", x))[0]


# Model::setupOptimizers learning rates (core/src/model.cpp:142).
LR_INIT = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)
BETA1, BETA2, EPS = 0.9, 0.999, 1e-8
_F32_BETA1, _F32_BETA2 = _f32(BETA1), _f32(BETA2)
GROUPS = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")


class DeviceScene:
    """The six parameter groups on the device plus Adam state and the
    densify statistics (Model's tensors, model.hpp:81-133)."""

    def __init__(self, scene: Scene):
        self.sh_degree = scene.sh_degree
        self.n = scene.n
        self.params = [E.DeviceArray.from_numpy(p) for p in scene.params()]
        self.background = E.DeviceArray.from_numpy(np.asarray(scene.background, np.float32))
        self.exp_avg = [E.DeviceArray.zeros(p.shape) for p in self.params]
        self.exp_avg_sq = [E.DeviceArray.zeros(p.shape) for p in self.params]
        self.grad_norm = E.DeviceArray.zeros(self.n)
        self.vis = E.DeviceArray.zeros(self.n)
        self.max2d = E.DeviceArray.zeros(self.n)
        self.adam_step = 0
        self.lr = list(LR_INIT)

    @property
    def gaussians(self) -> E.MsplatGaussians:
        m, s, q, dc, fr, op = self.params
        return E.MsplatGaussians(self.n, m.ptr, s.ptr, q.ptr, op.ptr, dc.ptr, fr.ptr)

    def camera(self, cam: Camera, degrees_to_use: int | None = None) -> E.MsplatCamera:
        dtu = self.sh_degree if degrees_to_use is None else degrees_to_use
        return E.prepare_camera(cam.cam_to_world, cam.fx, cam.fy, cam.cx, cam.cy, cam.width, cam.height,
                                self.sh_degree, dtu)

    def host_params(self) -> dict[str, np.ndarray]:
        return {name: p.numpy() for name, p in zip(GROUPS, self.params)}

    def adam_struct(self) -> E.MsplatAdam:
        """Advances the Adam step and returns the fused-update arguments
        (bias corrections computed as Model::fullIteration does: the power
        in double, then float32)."""
        self.adam_step += 1
        bc1 = _f32(1.0 - _F32_BETA1 ** self.adam_step)
        bc2 = _f32(1.0 - _F32_BETA2 ** self.adam_step)
        a = getattr(self, "_adam", None)
        if a is None:
            a = self._adam = E.MsplatAdam()
            a.beta1, a.beta2, a.eps = BETA1, BETA2, EPS
        for g in range(6):
            a.exp_avg[g] = self.exp_avg[g].ptr
            a.exp_avg_sq[g] = self.exp_avg_sq[g].ptr
            # float32 lr / bc1 and sqrt(bc2), rounded once from double (exact
            # for a quotient or root of float32 operands)
            a.step_size[g] = _f32(_f32(self.lr[g]) / bc1)
        a.bc2_sqrt = _f32(math.sqrt(bc2))
        return a


def render(ds: DeviceScene, cam: E.MsplatCamera, outputs=("out_img",)) -> dict[str, np.ndarray]:
    n = C.c_int64()
    E.check(E.lib().msplat_hip_render(C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, C.byref(n)))
    H, W = cam.height, cam.width
    shapes = {"out_img": (H, W, 3), "final_Ts": (H, W, 3), "final_idx": (H, W, 2), "out_depth": (H, W),
              "out_normal": (H, W, 3), "out_alpha": (H, W), "out_median_depth": (H, W), "out_distortion": (H, W)}
    res = {k: E.last(k, shapes.get(k)) for k in outputs}
    res["num_intersections"] = int(n.value)
    return res


def render_to_device(ds: DeviceScene, cam: E.MsplatCamera) -> E.DeviceArray:
    """Renders and copies the image into a new device array (e.g. a target)."""
    n = C.c_int64()
    E.check(E.lib().msplat_hip_render(C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, C.byref(n)))
    ptr, numel = E.last_ptr("out_img")
    out = E.DeviceArray((cam.height, cam.width, 3))
    E.check(E.lib().msplat_hip_copy(out.ptr, ptr, numel * 4))
    return out


def train_step(ds: DeviceScene, cam: E.MsplatCamera, gt: E.DeviceArray, ssim_weight: float = 0.2,
               fused_adam: bool = True, lambda_dist: float = 0.0) -> tuple[float, int]:
    """Model::fullIteration: forward, SSIM+L1, backward, Adam on six groups.
    Returns (loss, number of tile intersections)."""
    loss = C.c_float()
    nis = C.c_int64()
    inv_max_dim = np.float32(1.0) / np.float32(max(cam.width, cam.height))
    if fused_adam:
        adam = ds.adam_struct()
        E.check(E.lib().msplat_hip_train_step(
            C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, gt.ptr, 1.0 - ssim_weight, lambda_dist,
            ssim_weight, ds.grad_norm.ptr, ds.vis.ptr, ds.max2d.ptr, float(inv_max_dim), C.byref(adam),
            C.byref(loss), C.byref(nis)))
    else:
        E.check(E.lib().msplat_hip_train_step(
            C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, gt.ptr, 1.0 - ssim_weight, lambda_dist,
            ssim_weight, ds.grad_norm.ptr, ds.vis.ptr, ds.max2d.ptr, float(inv_max_dim), None,
            C.byref(loss), C.byref(nis)))
        adam = ds.adam_struct()
        names = ["dL_dmean3D", "dL_dscale", "dL_dquat", "dL_dfeatures_dc", "dL_dfeatures_rest", "dL_dopacity"]
        for g, name in enumerate(names):
            gptr, _ = E.last_ptr(name)
            p = ds.params[g]
            n = int(np.prod(p.shape))
            E.check(E.lib().msplat_hip_fused_adam(p.ptr, gptr, ds.exp_avg[g].ptr, ds.exp_avg_sq[g].ptr, n,
                                                  adam.step_size[g], adam.beta1, adam.beta2, adam.bc2_sqrt,
                                                  adam.eps))
        E.sync()
    return float(loss.value), int(nis.value)


STRIDES = (3, 2, 4, 3, 45, 1)  # floats per splat of each group at SH degree 3


class CapacityScene(DeviceScene):
    """A DeviceScene whose six groups, Adam moments and densify statistics
    live in backing buffers of `cap` rows, the first `n` of them active
    (Model's *_buf tensors, core/src/model.cpp:201-233), so that
    msplat_hip_densify can append and compact in place."""

    def __init__(self, scene: Scene, cap: int):
        if scene.sh_degree != 3:
            raise ValueError("CapacityScene holds SH degree 3 scenes")
        self.sh_degree = 3
        self.n = scene.n
        self.cap = cap
        host = [np.zeros(cap * s, np.float32) for s in STRIDES]
        for h, a, s in zip(host, scene.params(), STRIDES):
            h[: self.n * s] = a.reshape(-1)
        self.params = [E.DeviceArray.from_numpy(h) for h in host]
        self.background = E.DeviceArray.from_numpy(np.asarray(scene.background, np.float32))
        self.exp_avg = [E.DeviceArray.zeros(cap * s) for s in STRIDES]
        self.exp_avg_sq = [E.DeviceArray.zeros(cap * s) for s in STRIDES]
        self.grad_norm, self.vis, self.max2d = (E.DeviceArray.zeros(cap) for _ in range(3))
        self.adam_step = 0
        self.lr = list(LR_INIT)

    def ensure_capacity(self, rows: int) -> None:
        """Grows the backing buffers to at least `rows` rows (doubling, as
        Model::ensureCapacity), keeping the first n rows of every buffer."""
        if rows <= self.cap:
            return
        cap = max(rows, 2 * self.cap)

        def grown(old: E.DeviceArray, stride: int) -> E.DeviceArray:
            new = E.DeviceArray.zeros(cap * stride)
            E.check(E.lib().msplat_hip_copy(new.ptr, old.ptr, self.n * stride * 4))
            return new

        self.params = [grown(p, s) for p, s in zip(self.params, STRIDES)]
        self.exp_avg = [grown(p, s) for p, s in zip(self.exp_avg, STRIDES)]
        self.exp_avg_sq = [grown(p, s) for p, s in zip(self.exp_avg_sq, STRIDES)]
        self.grad_norm, self.vis, self.max2d = (grown(a, 1) for a in (self.grad_norm, self.vis, self.max2d))
        E.sync()
        self.cap = cap

    def _rows(self, a: E.DeviceArray, stride: int, count: int, rows: int) -> np.ndarray:
        out = np.zeros(rows * stride, np.float32)
        if count:
            E.check(E.lib().msplat_hip_download(out.ctypes.data, a.ptr, count * stride * 4))
        return out

    def state(self, rows: int | None = None) -> tuple[list, list, list, dict]:
        """Host copies of the first n rows of every backing buffer, in host
        arrays of `rows` rows (default n, zero after n), and the first n
        statistics."""
        rows = self.n if rows is None else rows
        n = self.n
        stats = {k: self._rows(a, 1, n, n) for k, a in
                 (("grad_norm", self.grad_norm), ("vis", self.vis), ("max2d", self.max2d))}
        return ([self._rows(p, s, n, rows) for p, s in zip(self.params, STRIDES)],
                [self._rows(p, s, n, rows) for p, s in zip(self.exp_avg, STRIDES)],
                [self._rows(p, s, n, rows) for p, s in zip(self.exp_avg_sq, STRIDES)], stats)

    def stage_samples(self, random_normals: np.ndarray) -> None:
        """Uploads the [2n, 3] split samples into a device buffer kept across
        cycles (grown by doubling)."""
        rs = np.ascontiguousarray(random_normals, np.float32).reshape(-1)
        have = self._rs.shape[0] if getattr(self, "_rs", None) is not None else 0
        if have < rs.size:
            self._rs = E.DeviceArray((max(rs.size, 2 * have),))
        if rs.size:
            E.check(E.lib().msplat_hip_upload(self._rs.ptr, rs.ctypes.data, rs.nbytes))

    def densify(self, random_normals: np.ndarray | None, half_max_dim: float, grad_thresh=0.0002, size_thresh=0.01,
                screen_thresh=0.05, check_screen=1, cull_alpha=0.1, cull_scale=0.5, cull_screen=0.15,
                check_huge=0) -> int:
        """msplat_hip_densify with Model::afterTrain's arguments; random_normals
        is [2n, 3] (None: the samples last staged by stage_samples).  The
        backing buffers grow (doubling, as Model::ensureCapacity) only when
        the rows after appending exceed them: the call then reports the rows
        it needs and changes nothing, and runs again.  Returns the new count;
        the growth time of this call is kept in `last_grow_ms`."""
        if random_normals is not None:
            self.stage_samples(random_normals)
        P6 = C.c_void_p * 6
        newc = C.c_int()
        self.last_grow_ms = 0.0
        for _ in range(2):
            rc = E.lib().msplat_hip_densify(self.n, self.cap, grad_thresh, size_thresh, screen_thresh, check_screen,
                                            cull_alpha, cull_scale, cull_screen, check_huge, self.grad_norm.ptr,
                                            self.vis.ptr, self.max2d.ptr, half_max_dim,
                                            P6(*[p.ptr for p in self.params]), STRIDES[4],
                                            P6(*[m.ptr for m in self.exp_avg]),
                                            P6(*[v.ptr for v in self.exp_avg_sq]), self._rs.ptr, C.byref(newc))
            if rc != E.MSPLAT_E_CAPACITY:
                break
            # more rows after appending than the buffers hold: nothing was modified
            t0 = time.perf_counter()
            self.ensure_capacity(int(newc.value))
            self.last_grow_ms = (time.perf_counter() - t0) * 1e3
        E.check(rc)
        self.n = int(newc.value)
        return self.n

    def reset_stats(self) -> None:
        for a in (self.grad_norm, self.vis, self.max2d):
            a.zero_()

    def reset_opacity(self, logit: float = -1.3862943611198906) -> None:
        """Model::afterTrain's opacity reset: clamp to logit(0.2) and zero
        the opacity group's Adam moments."""
        E.check(E.lib().msplat_hip_clamp_max(self.params[5].ptr, self.n, logit))
        self.exp_avg[5].zero_()
        self.exp_avg_sq[5].zero_()


def densify_schedule(step: int, n: int, max_splats: int = 250_000, refine_every: int = 100, warmup: int = 0,
                     reset_every: int = 30, num_cameras: int = 32, stop_split_at: int = 29500) -> tuple[bool, bool]:
    """(densify, reset opacity) after `step` with n splats under
    Model::afterTrain's schedule and capacity rule (core/src/model.cpp:
    240-306: no densification once n reaches max_splats)."""
    if not (step % refine_every == 0 and step > warmup):
        return False, False
    interval = reset_every * refine_every
    dens = step < stop_split_at and step % interval > num_cameras + refine_every and n < max_splats
    reset = step < stop_split_at and step % interval == refine_every
    return dens, reset


# ---- 3DGS mode ------------------------------------------------------------
class DeviceScene3D(DeviceScene):
    """DeviceScene of 3D Gaussians (scales [N,3]) for the 3DGS mode;
    params in GROUPS order, as numpy arrays."""

    @classmethod
    def from_scene(cls, scene: Scene) -> "DeviceScene3D":
        """From a Scene whose scales are [N, 3] (Scene.as_3dgs)."""
        return cls(dict(zip(GROUPS, scene.params())), scene.background, scene.sh_degree)

    def __init__(self, params: dict, background, sh_degree: int = 3):
        self.sh_degree = sh_degree
        self.n = int(params["means"].shape[0])
        if params["scales"].shape != (self.n, 3):
            raise ValueError("the 3DGS mode needs scales of shape [N, 3]")
        self.params = [E.DeviceArray.from_numpy(np.ascontiguousarray(params[g], np.float32)) for g in GROUPS]
        self.background = E.DeviceArray.from_numpy(np.asarray(background, np.float32))
        self.exp_avg = [E.DeviceArray.zeros(p.shape) for p in self.params]
        self.exp_avg_sq = [E.DeviceArray.zeros(p.shape) for p in self.params]
        self.grad_norm = E.DeviceArray.zeros(self.n)
        self.vis = E.DeviceArray.zeros(self.n)
        self.max2d = E.DeviceArray.zeros(self.n)
        self.adam_step = 0
        self.lr = list(LR_INIT)


def render3d(ds: DeviceScene3D, cam: E.MsplatCamera) -> dict[str, np.ndarray]:
    n = C.c_int64()
    E.check(E.lib().msplat_hip_render_3dgs(C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, C.byref(n)))
    H, W = cam.height, cam.width
    return dict(out_img=E.last("out_img", (H, W, 3)), final_T=E.last("final_Ts", (H, W, 3))[..., 0],
                num_intersections=int(n.value))


def render3d_to_device(ds: DeviceScene3D, cam: E.MsplatCamera) -> E.DeviceArray:
    """Renders (3DGS mode) and copies the image into a new device array."""
    n = C.c_int64()
    E.check(E.lib().msplat_hip_render_3dgs(C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, C.byref(n)))
    ptr, numel = E.last_ptr("out_img")
    out = E.DeviceArray((cam.height, cam.width, 3))
    E.check(E.lib().msplat_hip_copy(out.ptr, ptr, numel * 4))
    return out


def train_step3d(ds: DeviceScene3D, cam: E.MsplatCamera, gt: E.DeviceArray, ssim_weight: float = 0.2,
                 fused_adam: bool = True) -> tuple[float, int]:
    """One 3DGS training step (msplat_hip_train_step_3dgs): with fused_adam
    the six Adam updates run inside the projection backward; without, the
    parameter gradients stay in the engine cache (MSPLAT_LAST_DL_*)."""
    loss = C.c_float()
    nis = C.c_int64()
    inv_max_dim = np.float32(1.0) / np.float32(max(cam.width, cam.height))
    adam = ds.adam_struct() if fused_adam else None
    E.check(E.lib().msplat_hip_train_step_3dgs(
        C.byref(cam), C.byref(ds.gaussians), ds.background.ptr, gt.ptr, 1.0 - ssim_weight, ssim_weight,
        ds.grad_norm.ptr, ds.vis.ptr, ds.max2d.ptr, float(inv_max_dim), C.byref(adam) if adam else None,
        C.byref(loss), C.byref(nis)))
    return float(loss.value), int(nis.value)
