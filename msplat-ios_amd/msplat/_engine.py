"""ctypes binding of the C-ABI engine (include/msplat_engine.h) plus a small
device-array helper.  This is the Python side of the drop-in boundary: it
loads the in-tree libmsplat_hip.so and raises if it is missing -- there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "libmsplat_hip.so"
_lib = None

c_float_p = C.POINTER(C.c_float)


MSPLAT_E_CAPACITY = -5


class MsplatError(RuntimeError):
    pass


class MsplatCamera(C.Structure):
    _fields_ = [
        ("viewmat", C.c_float * 16), ("projmat", C.c_float * 16), ("cam_pos", C.c_float * 3),
        ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float),
        ("width", C.c_int32), ("height", C.c_int32), ("tiles_x", C.c_int32), ("tiles_y", C.c_int32),
        ("glob_scale", C.c_float), ("clip_thresh", C.c_float),
        ("degree", C.c_int32), ("degrees_to_use", C.c_int32),
    ]


class MsplatGaussians(C.Structure):
    _fields_ = [
        ("num_points", C.c_int32), ("means", C.c_void_p), ("scales", C.c_void_p), ("quats", C.c_void_p),
        ("opacities", C.c_void_p), ("features_dc", C.c_void_p), ("features_rest", C.c_void_p),
    ]


class MsplatAdam(C.Structure):
    _fields_ = [
        ("exp_avg", C.c_void_p * 6), ("exp_avg_sq", C.c_void_p * 6), ("step_size", C.c_float * 6),
        ("beta1", C.c_float), ("beta2", C.c_float), ("bc2_sqrt", C.c_float), ("eps", C.c_float),
    ]


class MsplatTsdfView(C.Structure):
    _fields_ = [
        ("viewmat", C.c_float * 16), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float),
        ("width", C.c_int32), ("height", C.c_int32), ("depth_dev", C.c_void_p), ("alpha_dev", C.c_void_p),
    ]


LAST = {name: i for i, name in enumerate([
    "xys", "depths", "radii", "num_tiles_hit", "transmats", "colors_used", "opacity_sigmoid", "normals",
    "records", "tile_offsets", "gaussian_ids", "out_img", "final_Ts", "final_idx", "out_depth", "out_normal",
    "out_alpha", "out_median_depth", "out_distortion", "dL_dout_img", "grads16", "dL_dtransMat",
    "dL_dnormal3D", "dL_dopacity", "dL_dcolors", "dL_dmean3D", "dL_dscale", "dL_dquat", "dL_dmean2D",
    "dL_dfeatures_dc", "dL_dfeatures_rest", "blend_log", "blend_ckpt", "wave_counts", "blend_chunks",
])}
_INT_BUFS = {"radii", "num_tiles_hit", "tile_offsets", "gaussian_ids", "final_idx", "blend_log", "wave_counts", "blend_chunks"}

# Every entry point declared in include/msplat_engine.h.
EXPORTS = [
    "msplat_hip_prepare_camera", "msplat_hip_init", "msplat_hip_cleanup", "msplat_hip_last_error",
    "msplat_hip_device_name", "msplat_hip_alloc", "msplat_hip_free", "msplat_hip_memset", "msplat_hip_upload",
    "msplat_hip_download", "msplat_hip_copy", "msplat_hip_commit", "msplat_hip_sync", "msplat_hip_train_step",
    "msplat_hip_render", "msplat_hip_image_to_rgba8", "msplat_hip_fused_adam", "msplat_hip_densify", "msplat_hip_clamp_max", "msplat_hip_loss_fwd_bwd",
    "msplat_hip_loss_fwd_bwd_noalloc",
    "msplat_hip_raster_bwd", "msplat_hip_project_bwd", "msplat_hip_project_bwd_adam", "msplat_hip_last", "msplat_hip_enable_timing",
    "msplat_hip_stage_times", "msplat_hip_last_pairs_evaluated", "msplat_hip_last_raster_counts",
    "msplat_hip_check_fast_rcp", "msplat_hip_set_wide_keys", "msplat_hip_set_deep_tile_len",
    "msplat_hip_set_loss_form",
    "msplat_hip_set_log_pool_chunks", "msplat_hip_log_pool_stats",
    "msplat_hip_tsdf_integrate",
    "msplat_hip_marching_cubes", "msplat_hip_mc_table", "msplat_hip_unproject_depth", "msplat_hip_render_3dgs",
    "msplat_hip_train_step_3dgs", "msplat_hip_densify_3dgs",
]
SYNTH_EXPORTS = ["msplat_synth_uniform", "msplat_synth_normal"]


def lib() -> C.CDLL:
    """Loads libmsplat_hip.so (built by msplat-ios_amd/build.py)."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("MSPLAT_HIP_LIB", _LIB_PATH))
    if not path.exists():
        raise MsplatError(f"{path} is missing: build it with `python msplat-ios_amd/build.py` "
                          "(the HIP engine has no CPU fallback)")
    L = C.CDLL(str(path))
    P, I, F, I64, SZ = C.c_void_p, C.c_int, C.c_float, C.c_int64, C.c_size_t
    sig = {
        "msplat_hip_prepare_camera": (I, [c_float_p, F, F, F, F, I, I, I, I, C.POINTER(MsplatCamera)]),
        "msplat_hip_init": (I, []),
        "msplat_hip_cleanup": (None, []),
        "msplat_hip_last_error": (C.c_char_p, []),
        "msplat_hip_device_name": (I, [C.c_char_p, I]),
        "msplat_hip_alloc": (P, [SZ]),
        "msplat_hip_free": (I, [P]),
        "msplat_hip_memset": (I, [P, I, SZ]),
        "msplat_hip_upload": (I, [P, P, SZ]),
        "msplat_hip_download": (I, [P, P, SZ]),
        "msplat_hip_copy": (I, [P, P, SZ]),
        "msplat_hip_commit": (I, []),
        "msplat_hip_sync": (I, []),
        "msplat_hip_train_step": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, P, F, F, F, P, P, P,
                                      F, C.POINTER(MsplatAdam), c_float_p, C.POINTER(I64)]),
        "msplat_hip_render": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, C.POINTER(I64)]),
        "msplat_hip_image_to_rgba8": (I, [P, I64, P]),
        "msplat_hip_fused_adam": (I, [P, P, P, P, I64, F, F, F, F, F]),
        "msplat_hip_densify": (I, [I, I, F, F, F, I, F, F, F, I, P, P, P, F, P * 6, I, P * 6, P * 6, P,
                                   C.POINTER(I)]),
        "msplat_hip_clamp_max": (I, [P, I64, F]),
        "msplat_hip_loss_fwd_bwd": (I, [I, I, P, P, P, F, F, F, P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "msplat_hip_loss_fwd_bwd_noalloc": (I, [I, I, P, P, P, F, F, F, P, C.POINTER(C.c_double),
                                                C.POINTER(C.c_double)]),
        "msplat_hip_raster_bwd": (I, [P, P, P, P, P, P, P]),
        "msplat_hip_project_bwd": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, P, P, P, P, P, P, P,
                                       P, P, P, F]),
        "msplat_hip_project_bwd_adam": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, P, P, P, P, F,
                                            C.POINTER(MsplatAdam)]),
        "msplat_hip_last": (I, [I, C.POINTER(P), C.POINTER(I64)]),
        "msplat_hip_enable_timing": (I, [I]),
        "msplat_hip_stage_times": (I, [C.POINTER(C.c_char_p), c_float_p, I]),
        "msplat_hip_last_pairs_evaluated": (I64, []),
        "msplat_hip_last_raster_counts": (I, [P]),
        "msplat_hip_check_fast_rcp": (I, [I, I, C.POINTER(C.c_int64)]),
        "msplat_hip_set_wide_keys": (I, [I]),
        "msplat_hip_set_deep_tile_len": (I, [I]),
        "msplat_hip_set_loss_form": (I, [I]),
        "msplat_hip_set_log_pool_chunks": (I, [I]),
        "msplat_hip_log_pool_stats": (I, [P]),
        "msplat_hip_densify_3dgs": (I, [I, I, F, F, F, I, F, F, F, I, P, P, P, F, P * 6, I, P * 6, P * 6, P,
                                        C.POINTER(I)]),
        "msplat_hip_render_3dgs": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, C.POINTER(I64)]),
        "msplat_hip_train_step_3dgs": (I, [C.POINTER(MsplatCamera), C.POINTER(MsplatGaussians), P, P, F, F, P, P, P,
                                           F, C.POINTER(MsplatAdam), c_float_p, C.POINTER(I64)]),
        "msplat_hip_tsdf_integrate": (I, [P, I, I, I, c_float_p, F, C.POINTER(MsplatTsdfView), I, F, F]),
        "msplat_hip_marching_cubes": (I, [P, I, I, I, c_float_p, F, I64, P, C.POINTER(I64), C.POINTER(I64)]),
        "msplat_hip_mc_table": (I, [P]),
        "msplat_hip_unproject_depth": (I, [P, P, P, I, I, F, F, F, F, c_float_p, F, P, P, C.POINTER(I64)]),
        "msplat_synth_uniform": (None, [C.c_uint64, C.c_uint64, I64, C.c_double, C.c_double, P]),
        "msplat_synth_normal": (None, [C.c_uint64, C.c_uint64, I64, C.c_double, C.c_double, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise MsplatError(f"msplat engine error {rc}: {lib().msplat_hip_last_error().decode()}")


def init() -> None:
    check(lib().msplat_hip_init())


def device_name() -> str:
    buf = C.create_string_buffer(256)
    check(lib().msplat_hip_device_name(buf, 256))
    return buf.value.decode()


def sync() -> None:
    check(lib().msplat_hip_sync())


def cleanup() -> None:
    lib().msplat_hip_cleanup()


class DeviceArray:
    """A device allocation with a numpy shape/dtype (the host view of an
    MTensor).  Frees itself when garbage-collected unless `owned=False`."""

    def __init__(self, shape, dtype=np.float32, ptr=None, owned=True):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        if ptr is None:
            ptr = lib().msplat_hip_alloc(max(self.nbytes, 16))
            if not ptr:
                raise MsplatError(f"device allocation of {self.nbytes} bytes failed: "
                                  f"{lib().msplat_hip_last_error().decode()}")
            owned = True
        self.ptr = ptr
        self.owned = owned

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib().msplat_hip_upload(d.ptr, a.ctypes.data, a.nbytes))
        return d

    @classmethod
    def zeros(cls, shape, dtype=np.float32) -> "DeviceArray":
        d = cls(shape, dtype)
        check(lib().msplat_hip_memset(d.ptr, 0, max(d.nbytes, 16)))
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib().msplat_hip_upload(self.ptr, a.ctypes.data, a.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().msplat_hip_download(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def zero_(self) -> "DeviceArray":
        check(lib().msplat_hip_memset(self.ptr, 0, max(self.nbytes, 16)))
        return self

    def copy(self) -> "DeviceArray":
        d = DeviceArray(self.shape, self.dtype)
        check(lib().msplat_hip_copy(d.ptr, self.ptr, self.nbytes))
        return d

    def __del__(self):
        if getattr(self, "owned", False) and self.ptr and _lib is not None:
            try:
                _lib.msplat_hip_free(self.ptr)
            except Exception:
                pass
            self.ptr = None


def last(name: str, shape=None) -> np.ndarray | None:
    """Downloads a cached engine buffer (the msplat_last_* accessors)."""
    ptr = C.c_void_p()
    n = C.c_int64()
    check(lib().msplat_hip_last(LAST[name], C.byref(ptr), C.byref(n)))
    if not ptr.value or n.value == 0:
        return None
    dtype = np.int32 if name in _INT_BUFS else np.float32
    out = np.empty(n.value, dtype)
    check(lib().msplat_hip_download(out.ctypes.data, ptr.value, out.nbytes))
    return out.reshape(shape) if shape is not None else out


def last_ptr(name: str) -> tuple[int, int]:
    ptr = C.c_void_p()
    n = C.c_int64()
    check(lib().msplat_hip_last(LAST[name], C.byref(ptr), C.byref(n)))
    return ptr.value or 0, n.value


def prepare_camera(cam_to_world, fx, fy, cx, cy, width, height, degree=0, degrees_to_use=0) -> MsplatCamera:
    c2w = np.ascontiguousarray(cam_to_world, dtype=np.float32).reshape(16)
    cam = MsplatCamera()
    check(lib().msplat_hip_prepare_camera(c2w.ctypes.data_as(c_float_p), fx, fy, cx, cy, int(width), int(height),
                                          int(degree), int(degrees_to_use), C.byref(cam)))
    return cam


def enable_timing(on: bool = True, pairs: bool = False) -> None:
    """Per-stage HIP event timing; `pairs` also counts raster pairs."""
    check(lib().msplat_hip_enable_timing((1 if on else 0) | (2 if pairs else 0)))


def stage_times() -> dict[str, float]:
    names = (C.c_char_p * 16)()
    ms = (C.c_float * 16)()
    k = lib().msplat_hip_stage_times(names, ms, 16)
    return {names[i].decode(): float(ms[i]) for i in range(k)}


def pairs_evaluated() -> int:
    return int(lib().msplat_hip_last_pairs_evaluated())


def raster_counts() -> dict:
    """Counters of the most recent forward with the pair counter on."""
    out = (C.c_int64 * 5)()
    check(lib().msplat_hip_last_raster_counts(C.cast(out, C.c_void_p)))
    return {"pairs_evaluated": int(out[0]), "log_entries": int(out[1]), "pairs_blended": int(out[2]),
            "visits": int(out[3]), "visit_slots": int(out[4])}


def log_pool_stats() -> dict:
    """The blend-log pool: chunks of the frame's pool, chunks the last
    logging forward claimed, overflowed logs since init, worst-case chunks
    of the frame, device bytes its buffers hold."""
    out = (C.c_int64 * 5)()
    check(lib().msplat_hip_log_pool_stats(C.cast(out, C.c_void_p)))
    return {"chunks": int(out[0]), "taken": int(out[1]), "redos": int(out[2]), "worst": int(out[3]),
            "bytes": int(out[4])}


# ---- mesh extraction -------------------------------------------------------

def mc_table() -> np.ndarray:
    """The marching-cubes case table [256, 16] int8 (host only)."""
    t = np.zeros((256, 16), np.int8)
    check(lib().msplat_hip_mc_table(t.ctypes.data))
    return t


def _f3(v) -> C.Array:
    return (C.c_float * 3)(*[float(x) for x in v])


def tsdf_integrate(grid: "DeviceArray", origin, voxel_size, views, trunc_dist, alpha_thresh) -> None:
    """Folds views [(viewmat[16], fx, fy, cx, cy, depth DeviceArray [H,W],
    alpha DeviceArray [H,W]), ...] into grid (DeviceArray [Dz,Dy,Dx,2])."""
    dz, dy, dx = grid.shape[:3]
    arr = (MsplatTsdfView * max(len(views), 1))()
    for k, (vm, fx, fy, cx, cy, depth, alpha) in enumerate(views):
        arr[k].viewmat[:] = [float(x) for x in np.asarray(vm, np.float32).reshape(16)]
        arr[k].fx, arr[k].fy, arr[k].cx, arr[k].cy = fx, fy, cx, cy
        arr[k].height, arr[k].width = depth.shape
        arr[k].depth_dev, arr[k].alpha_dev = depth.ptr, alpha.ptr
    org = _f3(origin)
    check(lib().msplat_hip_tsdf_integrate(grid.ptr, dx, dy, dz, org, voxel_size, arr, len(views), trunc_dist,
                                          alpha_thresh))


def marching_cubes(grid: "DeviceArray", origin, voxel_size, max_triangles: int) -> tuple[np.ndarray, int]:
    """(triangles [n,3,3] float32 on the host, number the grid produces)."""
    dz, dy, dx = grid.shape[:3]
    out = DeviceArray((max(max_triangles, 1), 9))
    n, total = C.c_int64(), C.c_int64()
    org = _f3(origin)
    check(lib().msplat_hip_marching_cubes(grid.ptr, dx, dy, dz, org, voxel_size, max_triangles, out.ptr,
                                          C.byref(n), C.byref(total)))
    tris = np.empty((n.value, 9), np.float32)
    if n.value:
        check(lib().msplat_hip_download(tris.ctypes.data, out.ptr, tris.nbytes))
    return tris.reshape(-1, 3, 3), int(total.value)


def unproject_depth(img: "DeviceArray", depth: "DeviceArray", alpha: "DeviceArray", fx, fy, cx, cy, cam_to_world,
                    alpha_thresh) -> tuple[np.ndarray, np.ndarray]:
    """(xyz [n,3] float32, rgb [n,3] uint8) of one view."""
    h, w = depth.shape
    xyz = DeviceArray((max(h * w, 1), 3))
    rgb = DeviceArray((max(h * w, 1), 3), np.uint8)
    c2w = np.ascontiguousarray(cam_to_world, np.float32).reshape(16)
    n = C.c_int64()
    check(lib().msplat_hip_unproject_depth(img.ptr, depth.ptr, alpha.ptr, w, h, fx, fy, cx, cy,
                                           c2w.ctypes.data_as(c_float_p), alpha_thresh, xyz.ptr, rgb.ptr,
                                           C.byref(n)))
    hx, hr = np.empty((n.value, 3), np.float32), np.empty((n.value, 3), np.uint8)
    if n.value:
        check(lib().msplat_hip_download(hx.ctypes.data, xyz.ptr, hx.nbytes))
        check(lib().msplat_hip_download(hr.ctypes.data, rgb.ptr, hr.nbytes))
    return hx, hr
