"""ctypes binding of the public C ABI (include/msplat_c_api.h, the
reference's core/include/msplat_c_api.h:16-127 plus the extensions), for
callers without the msplat._core extension module: the structures and the
signatures of every function, bound on first use.  Ownership follows the
header: PixelBuffer.data is the caller's to free() (free_pixels), a dataset
must outlive the trainers made from it.
"""
from __future__ import annotations

import ctypes as C
import ctypes.util

from . import _engine


class Config(C.Structure):
    _fields_ = [("iterations", C.c_int), ("shDegree", C.c_int), ("shDegreeInterval", C.c_int),
                ("ssimWeight", C.c_float), ("numDownscales", C.c_int), ("resolutionSchedule", C.c_int),
                ("refineEvery", C.c_int), ("warmupLength", C.c_int), ("resetAlphaEvery", C.c_int),
                ("densifyGradThresh", C.c_float), ("densifySizeThresh", C.c_float), ("stopScreenSizeAt", C.c_int),
                ("splitScreenSize", C.c_float), ("keepCrs", C.c_bool), ("downscaleFactor", C.c_float),
                ("bgColor", C.c_float * 3)]


def default_config() -> Config:
    """msplat_default_config() (a static inline function of the header)."""
    c = Config(iterations=30000, shDegree=3, shDegreeInterval=1000, ssimWeight=0.2, numDownscales=2,
               resolutionSchedule=3000, refineEvery=100, warmupLength=500, resetAlphaEvery=30,
               densifyGradThresh=0.0002, densifySizeThresh=0.01, stopScreenSizeAt=4000, splitScreenSize=0.05,
               keepCrs=False, downscaleFactor=1.0)
    c.bgColor[:] = [0.6130, 0.0101, 0.3984]
    return c


class CameraImage(C.Structure):
    _fields_ = [("width", C.c_int), ("height", C.c_int), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float),
                ("cy", C.c_float), ("camToWorld", C.c_float * 16), ("rgb", C.c_void_p)]


class Stats(C.Structure):
    _fields_ = [("iteration", C.c_int), ("splatCount", C.c_int), ("msPerStep", C.c_float), ("loss", C.c_float)]


class PixelBuffer(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("width", C.c_int), ("height", C.c_int)]


class EvalMetrics(C.Structure):
    _fields_ = [("psnr", C.c_float), ("ssim", C.c_float), ("l1", C.c_float), ("numTest", C.c_int),
                ("numGaussians", C.c_int)]


_bound = None
_libc = None


def lib() -> C.CDLL:
    """libmsplat_hip.so with the C ABI's signatures set."""
    global _bound, _libc
    if _bound is not None:
        return _bound
    L = _engine.lib()
    V, P, I, F, B, S = C.c_void_p, C.c_char_p, C.c_int, C.c_float, C.c_bool, C.c_int64
    fp = C.POINTER(C.c_float)
    sig = {
        "msplat_dataset_create": (V, [P, F, B, I]),
        "msplat_dataset_create_from_memory": (V, [C.POINTER(CameraImage), I, V, V, S, B, I]),
        "msplat_dataset_destroy": (None, [V]),
        "msplat_dataset_num_train": (I, [V]),
        "msplat_dataset_num_test": (I, [V]),
        "msplat_dataset_camera_pose": (None, [V, I, fp]),
        "msplat_trainer_create": (V, [V, Config]),
        "msplat_trainer_destroy": (None, [V]),
        "msplat_trainer_step": (Stats, [V]),
        "msplat_trainer_train": (None, [V]),
        "msplat_trainer_evaluate": (EvalMetrics, [V]),
        "msplat_trainer_render": (PixelBuffer, [V, I, B]),
        "msplat_trainer_render_pose": (PixelBuffer, [V, fp, I]),
        "msplat_trainer_render_pose_to_buffer": (None, [V, fp, I, V, C.POINTER(I), C.POINTER(I)]),
        "msplat_trainer_export_ply": (None, [V, P]),
        "msplat_trainer_export_splat": (None, [V, P]),
        "msplat_trainer_extract_mesh": (S, [V, P, F, F, F, F]),
        "msplat_trainer_save_checkpoint": (None, [V, P]),
        "msplat_trainer_load_checkpoint": (I, [V, P]),
        "msplat_trainer_splat_count": (I, [V]),
        "msplat_trainer_iteration": (I, [V]),
        "msplat_trainer_load_ply": (I, [V, P]),
        "msplat_trainer_set_max_splats": (None, [V, I]),
        "msplat_trainer_set_cull_alpha": (None, [V, F]),
        "msplat_trainer_create_3dgs": (V, [V, Config]),
        "msplat_set_metallib_path": (None, [P]),
        "msplat_sync": (None, []),
        "msplat_cleanup": (None, []),
        "msplat_last_error": (P, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _libc = C.CDLL(ctypes.util.find_library("c"))
    _libc.free.argtypes = [C.c_void_p]
    _bound = L
    return L


def last_error() -> str:
    return (lib().msplat_last_error() or b"").decode()


def free_pixels(px: PixelBuffer) -> None:
    """Releases a PixelBuffer's data (malloc'd by the library)."""
    lib()
    if px.data:
        _libc.free(C.cast(px.data, C.c_void_p))
