"""Device-resident scene state and one-call wrappers over the engine's render
and training-step entry points (Model::render / Model::fullIteration,
core/src/model.cpp:546-554 and 762-829, driven from Python)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _engine as E
from .synthetic import Camera, Scene

# Model::setupOptimizers learning rates (core/src/model.cpp:142).
LR_INIT = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)
BETA1, BETA2, EPS = 0.9, 0.999, 1e-8
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
        (bias corrections computed as Model::fullIteration does)."""
        self.adam_step += 1
        bc1 = np.float32(1.0 - np.power(np.float64(np.float32(BETA1)), self.adam_step))
        bc2 = np.float32(1.0 - np.power(np.float64(np.float32(BETA2)), self.adam_step))
        a = E.MsplatAdam()
        for g in range(6):
            a.exp_avg[g] = self.exp_avg[g].ptr
            a.exp_avg_sq[g] = self.exp_avg_sq[g].ptr
            a.step_size[g] = float(np.float32(np.float32(self.lr[g]) / bc1))
        a.beta1, a.beta2, a.eps = BETA1, BETA2, EPS
        a.bc2_sqrt = float(np.sqrt(bc2, dtype=np.float32))
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
