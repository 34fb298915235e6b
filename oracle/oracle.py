"""ctypes binding of the CPU golden model (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  See golden.h for the
arithmetic contract and the deliberate deviations from the fork.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)


class OrcStepDetail(C.Structure):
    _fields_ = [("want_grads", C.c_int), ("num_isect", C.c_int64), ("tile_offsets", C.POINTER(C.c_int32)),
                ("ids", C.POINTER(C.c_int32)), ("grads16", C.POINTER(C.c_float)),
                ("grads16_abs", C.POINTER(C.c_float))]


class OrcCamera(C.Structure):
    _fields_ = [("viewmat", C.c_float * 16), ("projmat", C.c_float * 16), ("cam_pos", C.c_float * 3),
                ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float),
                ("width", C.c_int), ("height", C.c_int), ("tiles_x", C.c_int), ("tiles_y", C.c_int)]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P = C.c_void_p
        L.orc_expf.restype = C.c_float
        L.orc_expf.argtypes = [C.c_float]
        L.orc_expf_array.argtypes = [C.c_int64, P, P]
        L.orc_gauss.argtypes = [C.c_float]
        L.orc_gauss.restype = C.c_float
        L.orc_gauss_array.argtypes = [C.c_int64, P, P]
        L.orc_ssim_window.argtypes = [P]
        L.orc_num_threads.restype = C.c_int
        L.orc_prepare_cam.argtypes = [P, C.c_float, C.c_float, C.c_float, C.c_float, C.c_int, C.c_int,
                                      C.POINTER(OrcCamera)]
        L.orc_project_fwd.argtypes = [C.c_int] + [P] * 6 + [C.c_int, C.c_int, C.POINTER(OrcCamera), C.c_float,
                                                            C.c_float] + [P] * 8
        L.orc_count_tiles.restype = C.c_int64
        L.orc_count_tiles.argtypes = [C.c_int, P, P, C.c_int, C.c_int, P]
        L.orc_bin_sort.argtypes = [C.c_int, P, P, P, C.c_int, C.c_int, P, P, P, P]
        L.orc_raster_fwd.argtypes = [C.POINTER(OrcCamera)] + [P] * 15 + [C.POINTER(C.c_int64)]
        L.orc_loss_fwd_bwd.restype = C.c_double
        L.orc_loss_fwd_bwd.argtypes = [C.c_int, C.c_int, P, P, P, C.c_float, C.c_float, C.c_float, P, P,
                                       C.POINTER(C.c_double)]
        L.orc_raster_bwd.argtypes = [C.POINTER(OrcCamera), C.c_int] + [P] * 17
        L.orc_project_bwd.argtypes = [C.c_int, P, P, P, P, C.c_int, C.c_int, C.POINTER(OrcCamera), C.c_float,
                                      P, P, P, P, P, P, P, P, P, P, P, C.c_float]
        L.orc_adam.argtypes = [P, P, P, P, C.c_int64, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float]
        L.orc_densify.restype = C.c_int
        L.orc_densify.argtypes = [C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, C.c_int, C.c_float,
                                  C.c_float, C.c_float, C.c_int, P, P, P, C.c_float, P * 6, C.c_int, P * 6,
                                  P * 6, P]
        L.orc_densify_3dgs.restype = C.c_int
        L.orc_densify_3dgs.argtypes = L.orc_densify.argtypes
        L.orc_train_step.restype = C.c_double
        L.orc_train_step.argtypes = [C.c_int] + [P] * 6 + [C.c_int, C.c_int, C.POINTER(OrcCamera), P, P,
                                                          C.c_float, P * 6, P * 6, P, C.c_int, P, P, P, P, P,
                                                          C.POINTER(C.c_int64), C.POINTER(OrcStepDetail)]
        L.orc_free.argtypes = [P]
        F = C.c_float
        L.orc_tsdf_integrate.argtypes = [P, C.c_int, C.c_int, C.c_int, P, F, P, F, F, F, F, C.c_int, C.c_int, F, F,
                                         P, P]
        L.orc_marching_cubes.restype = C.c_int64
        L.orc_marching_cubes.argtypes = [P, C.c_int, C.c_int, C.c_int, P, F, P, C.c_int64, P]
        L.orc_project3d_fwd.argtypes = [C.c_int] + [P] * 5 + [C.c_int, C.c_int, C.POINTER(OrcCamera), F, F] + [P] * 7
        L.orc_raster3d_fwd.argtypes = [C.POINTER(OrcCamera)] + [P] * 10
        L.orc_raster3d_bwd.argtypes = [C.POINTER(OrcCamera), C.c_int] + [P] * 12
        L.orc_project3d_bwd.argtypes = ([C.c_int] + [P] * 4 + [C.c_int, C.c_int, C.POINTER(OrcCamera), F] + [P] * 11
                                        + [F])
        L.orc_unproject_depth.restype = C.c_int64
        L.orc_unproject_depth.argtypes = [P, P, P, C.c_int, C.c_int, F, F, F, F, P, F, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def expf(x: float) -> float:
    return float(lib().orc_expf(float(x)))


def expf_array(x: np.ndarray) -> np.ndarray:
    x = _f(x)
    y = np.empty_like(x)
    lib().orc_expf_array(x.size, _p(x), _p(y))
    return y


def gauss(rho: float) -> float:
    """The rasterizer's Gaussian falloff exp(-rho / 2)."""
    return float(lib().orc_gauss(rho))


def gauss_array(rho: np.ndarray) -> np.ndarray:
    rho = _f(rho)
    y = np.zeros_like(rho)
    lib().orc_gauss_array(rho.size, _p(rho), _p(y))
    return y


def ssim_window() -> np.ndarray:
    w = np.zeros(11, np.float32)
    lib().orc_ssim_window(_p(w))
    return w


def num_threads() -> int:
    return int(lib().orc_num_threads())


def prepare_cam(cam_to_world, fx, fy, cx, cy, width, height) -> OrcCamera:
    c2w = _f(cam_to_world).reshape(16)
    cam = OrcCamera()
    lib().orc_prepare_cam(c2w.ctypes.data, fx, fy, cx, cy, int(width), int(height), C.byref(cam))
    return cam


def project_fwd(scene_params: dict, cam: OrcCamera, degree: int, dtu: int, glob_scale=1.0, clip_thresh=0.01):
    m = _f(scene_params["means"])
    n = m.shape[0]
    fr = _f(scene_params["features_rest"])
    out = dict(xys=np.zeros((n, 2), np.float32), depths=np.zeros(n, np.float32), radii=np.zeros(n, np.int32),
               transmats=np.zeros((n, 9), np.float32), normal_opac=np.zeros((n, 4), np.float32),
               colors=np.zeros((n, 3), np.float32), tiles_hit=np.zeros(n, np.int32),
               rect=np.zeros((n, 4), np.int32))
    ins = [_f(scene_params[k]) for k in ("scales", "quats", "opacities", "features_dc")]
    lib().orc_project_fwd(n, _p(m), _p(ins[0]), _p(ins[1]), _p(ins[2]), _p(ins[3]), _p(fr), degree, dtu,
                          C.byref(cam), glob_scale, clip_thresh, *[_p(out[k]) for k in
                                                                   ("xys", "depths", "radii", "transmats",
                                                                    "normal_opac", "colors", "tiles_hit", "rect")])
    return out


def bin_sort(proj: dict, cam: OrcCamera):
    n = proj["radii"].shape[0]
    T = cam.tiles_x * cam.tiles_y
    counts = np.zeros(T, np.int32)
    I = lib().orc_count_tiles(n, _p(proj["radii"]), _p(proj["rect"]), cam.tiles_x, cam.tiles_y, _p(counts))
    offsets = np.zeros(T + 1, np.int32)
    keys = np.zeros(max(I, 1), np.uint64)
    ids = np.zeros(max(I, 1), np.int32)
    lib().orc_bin_sort(n, _p(proj["radii"]), _p(proj["rect"]), _p(proj["depths"]), cam.tiles_x, cam.tiles_y,
                       _p(counts), _p(offsets), _p(keys), _p(ids))
    return dict(tile_counts=counts, tile_offsets=offsets, keys=keys[:I], ids=ids[:I], num_intersections=int(I))


def raster_fwd(proj: dict, bins: dict, cam: OrcCamera, background):
    H, W = cam.height, cam.width
    o = dict(out_img=np.zeros((H, W, 3), np.float32), final_Ts=np.zeros((H, W, 3), np.float32),
             final_idx=np.zeros((H, W, 2), np.int32), out_depth=np.zeros((H, W), np.float32),
             out_normal=np.zeros((H, W, 3), np.float32), out_alpha=np.zeros((H, W), np.float32),
             out_median_depth=np.zeros((H, W), np.float32), out_distortion=np.zeros((H, W), np.float32))
    pairs = C.c_int64()
    bg = _f(background)
    ids = bins["ids"] if bins["ids"].size else np.zeros(1, np.int32)
    lib().orc_raster_fwd(C.byref(cam), _p(bins["tile_offsets"]), _p(ids), _p(proj["xys"]), _p(proj["transmats"]),
                         _p(proj["normal_opac"]), _p(proj["colors"]), _p(bg),
                         *[_p(o[k]) for k in ("out_img", "final_Ts", "final_idx", "out_depth", "out_normal",
                                              "out_alpha", "out_median_depth", "out_distortion")],
                         C.byref(pairs))
    o["pairs_evaluated"] = int(pairs.value)
    return o


def render(scene, cam_index=0, degrees_to_use=None):
    """Forward pass of the golden model for a synthetic Scene."""
    c = scene.cameras[cam_index]
    cam = prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
    dtu = scene.sh_degree if degrees_to_use is None else degrees_to_use
    params = dict(means=scene.means, scales=scene.scales, quats=scene.quats, opacities=scene.opacities,
                  features_dc=scene.features_dc, features_rest=scene.features_rest)
    proj = project_fwd(params, cam, scene.sh_degree, dtu)
    bins = bin_sort(proj, cam)
    fwd = raster_fwd(proj, bins, cam, scene.background)
    return cam, proj, bins, fwd


def loss_fwd_bwd(img, gt, distortion=None, lambda_l1=0.8, lambda_dist=0.0, lambda_dssim=0.2):
    img, gt = _f(img), _f(gt)
    H, W = img.shape[:2]
    dL = np.zeros_like(img)
    dd = np.zeros((H, W), np.float32)
    ssim = C.c_double()
    dist = None if distortion is None else _f(distortion)
    loss = lib().orc_loss_fwd_bwd(W, H, _p(img), _p(gt), _p(dist), lambda_l1, lambda_dist, lambda_dssim, _p(dL),
                                  _p(dd), C.byref(ssim))
    return float(loss), dL, dd, float(ssim.value)


def raster_bwd(proj, bins, fwd, cam, background, dL_dimg, dL_ddepth=None, dL_dalpha=None, dL_dnormal=None,
               dL_dmedian=None, dL_ddist=None, with_abs=False):
    """[N,16] raster gradients; with_abs also returns, per component, the
    sum of the magnitudes of its summands (the scale of a float summation's
    rounding error)."""
    n = proj["radii"].shape[0]
    g = np.zeros((n, 16), np.float32)
    ga = np.zeros((n, 16), np.float32) if with_abs else None
    ids = bins["ids"] if bins["ids"].size else np.zeros(1, np.int32)
    opt = [None if a is None else _f(a) for a in (dL_ddepth, dL_dalpha, dL_dnormal, dL_dmedian, dL_ddist)]
    bgf, dl = _f(background), _f(dL_dimg)  # converted arrays live until the call returns
    lib().orc_raster_bwd(C.byref(cam), n, _p(bins["tile_offsets"]), _p(ids), _p(proj["xys"]),
                         _p(proj["transmats"]), _p(proj["normal_opac"]), _p(proj["colors"]), _p(bgf),
                         _p(fwd["final_Ts"]), _p(fwd["final_idx"]), _p(dl), *[_p(a) for a in opt], _p(g), _p(ga))
    return (g, ga) if with_abs else g


def project_bwd(params: dict, cam, degree, dtu, radii, grads16, stats=None, glob_scale=1.0):
    m = _f(params["means"])
    n = m.shape[0]
    K = (degree + 1) ** 2 - 1
    out = dict(dmeans=np.zeros((n, 3), np.float32), dscales=np.zeros((n, 2), np.float32),
               dquats=np.zeros((n, 4), np.float32), dmean2d=np.zeros((n, 2), np.float32),
               dfdc=np.zeros((n, 3), np.float32), dfrest=np.zeros((n, max(K, 0), 3), np.float32))
    if stats is None:
        stats = dict(grad_norm=np.zeros(n, np.float32), vis=np.zeros(n, np.float32), max2d=np.zeros(n, np.float32))
    inv_max_dim = np.float32(1.0) / np.float32(max(cam.width, cam.height))
    sc, qu, fr = _f(params["scales"]), _f(params["quats"]), _f(params["features_rest"])
    rad, g16 = np.ascontiguousarray(radii, np.int32), _f(grads16)
    lib().orc_project_bwd(n, _p(m), _p(sc), _p(qu), _p(fr), degree, dtu, C.byref(cam), glob_scale, _p(rad), _p(g16),
                          *[_p(out[k]) for k in ("dmeans", "dscales", "dquats", "dmean2d", "dfdc", "dfrest")],
                          _p(stats["grad_norm"]), _p(stats["vis"]), _p(stats["max2d"]), float(inv_max_dim))
    out.update(stats)
    return out


def adam(params, grads, m, v, step_size, beta1=0.9, beta2=0.999, bc2_sqrt=1.0, eps=1e-8):
    lib().orc_adam(_p(params), _p(grads), _p(m), _p(v), params.size, step_size, beta1, beta2, bc2_sqrt, eps)


def densify(n, capacity, params6, exp_avg6, exp_avg_sq6, fr_stride, stats, random_samples, grad_thresh=0.0002,
            size_thresh=0.01, screen_thresh=0.05, check_screen=1, cull_alpha=0.1, cull_scale=0.5,
            cull_screen=0.15, check_huge=1, half_max_dim=648.5, scale_dim=2):
    """scale_dim 2 (surfels) or 3 (the 3DGS mode's Gaussians)."""
    P6 = C.c_void_p * 6
    rs = _f(random_samples)
    fn = {2: lib().orc_densify, 3: lib().orc_densify_3dgs}[scale_dim]
    r = fn(n, capacity, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha,
                          cull_scale, cull_screen, check_huge, _p(stats["grad_norm"]), _p(stats["vis"]),
                          _p(stats["max2d"]), half_max_dim, P6(*[_p(a) for a in params6]), fr_stride,
                          P6(*[_p(a) for a in exp_avg6]), P6(*[_p(a) for a in exp_avg_sq6]),
                          _p(rs))
    return int(r)


def train_step(params6, exp_avg6, exp_avg_sq6, cam, background, gt, degree, dtu, adam_lr, adam_step, stats,
               ssim_weight=0.2, detail=None):
    """One golden-model training step in place; returns (loss, img, stage_ms, I).
    detail: None, "bins" or "grads" -- fills `detail_out` (a dict passed as
    stats["detail"]) with the tile offsets and ids, plus the raster gradients
    and their summand magnitudes for "grads"."""
    m, s, q, dc, fr, op = params6
    n = m.shape[0]
    P6 = C.c_void_p * 6
    img = np.zeros((cam.height, cam.width, 3), np.float32)
    stage = np.zeros(8, np.float64)
    nis = C.c_int64()
    lr = np.asarray(adam_lr, np.float32)
    det = OrcStepDetail(want_grads=1 if detail == "grads" else 0) if detail else None
    bgf, gtf = _f(background), _f(gt)
    loss = lib().orc_train_step(n, _p(m), _p(s), _p(q), _p(op), _p(dc), _p(fr), degree, dtu, C.byref(cam),
                                _p(bgf), _p(gtf), ssim_weight, P6(*[_p(a) for a in exp_avg6]),
                                P6(*[_p(a) for a in exp_avg_sq6]), _p(lr), adam_step, _p(stats["grad_norm"]),
                                _p(stats["vis"]), _p(stats["max2d"]), _p(img), _p(stage), C.byref(nis),
                                C.byref(det) if det is not None else None)
    if det is not None:
        out = stats.setdefault("detail", {})
        T = cam.tiles_x * cam.tiles_y
        I = int(det.num_isect)

        def take(ptr, count, dtype):
            a = np.ctypeslib.as_array(ptr, shape=(count,)).astype(dtype, copy=True) if count else np.zeros(0, dtype)
            lib().orc_free(C.cast(ptr, C.c_void_p))
            return a

        out["tile_offsets"] = take(det.tile_offsets, T + 1, np.int32)
        out["ids"] = take(det.ids, I, np.int32)
        if det.want_grads:
            out["grads16"] = take(det.grads16, 16 * n, np.float32).reshape(n, 16)
            out["grads16_abs"] = take(det.grads16_abs, 16 * n, np.float32).reshape(n, 16)
    return float(loss), img, stage, int(nis.value)


def tsdf_integrate(grid, origin, voxel_size, viewmat, fx, fy, cx, cy, depth, alpha, trunc_dist, alpha_thresh):
    """Folds one view into grid ([Dz,Dy,Dx,2] float32, C-contiguous) in place."""
    assert grid.dtype == np.float32 and grid.flags.c_contiguous and grid.ndim == 4 and grid.shape[3] == 2
    dz, dy, dx = grid.shape[:3]
    depth, alpha = _f(depth), _f(alpha)
    h, w = depth.shape
    assert alpha.shape == (h, w)
    org, vm = _f(origin), _f(viewmat)  # held until the call returns
    lib().orc_tsdf_integrate(_p(grid), dx, dy, dz, _p(org), voxel_size, _p(vm), fx, fy, cx, cy, w, h,
                             trunc_dist, alpha_thresh, _p(depth), _p(alpha))


def marching_cubes(grid, origin, voxel_size, table, max_triangles=None):
    """(triangles [n, 3, 3] float32, number the grid produces) for a
    [Dz,Dy,Dx,2] grid; table is the 256 x 16 int8 case table."""
    grid = _f(grid)
    dz, dy, dx = grid.shape[:3]
    tab = np.ascontiguousarray(table, np.int8).reshape(256, 16)
    org = _f(origin)
    if max_triangles is None:
        total = lib().orc_marching_cubes(_p(grid), dx, dy, dz, _p(org), voxel_size, _p(tab), 0, None)
        max_triangles = total
    out = np.zeros((max(max_triangles, 1), 9), np.float32)
    total = lib().orc_marching_cubes(_p(grid), dx, dy, dz, _p(org), voxel_size, _p(tab), max_triangles, _p(out))
    return out[:min(total, max_triangles)].reshape(-1, 3, 3), int(total)


def unproject_depth(img, depth, alpha, fx, fy, cx, cy, cam_to_world, alpha_thresh):
    """(xyz [n,3] float32, rgb [n,3] uint8) of one view."""
    img, depth, alpha = _f(img), _f(depth), _f(alpha)
    h, w = depth.shape
    xyz = np.zeros((h * w, 3), np.float32)
    rgb = np.zeros((h * w, 3), np.uint8)
    c2w = _f(cam_to_world)
    n = lib().orc_unproject_depth(_p(img), _p(depth), _p(alpha), w, h, fx, fy, cx, cy, _p(c2w), alpha_thresh,
                                  _p(xyz), _p(rgb))
    return xyz[:n], rgb[:n]


# ---- 3DGS mode ---------------------------------------------------------------

def project3d_fwd(params: dict, cam: OrcCamera, degree: int, dtu: int, glob_scale=1.0, clip_thresh=0.01):
    """3DGS projection: dict(xys, conics, depths, radii, rect, colors, cov2d).
    params: means [N,3], scales [N,3] (log), quats [N,4], features_dc,
    features_rest."""
    m = _f(params["means"])
    n = m.shape[0]
    sc, qu, dc, fr = _f(params["scales"]), _f(params["quats"]), _f(params["features_dc"]), _f(params["features_rest"])
    assert sc.shape == (n, 3)
    out = dict(xys=np.zeros((n, 2), np.float32), conics=np.zeros((n, 3), np.float32),
               depths=np.zeros(n, np.float32), radii=np.zeros(n, np.int32), rect=np.zeros((n, 4), np.int32),
               colors=np.zeros((n, 3), np.float32), cov2d=np.zeros((n, 3), np.float32))
    lib().orc_project3d_fwd(n, _p(m), _p(sc), _p(qu), _p(dc), _p(fr), degree, dtu, C.byref(cam), glob_scale,
                            clip_thresh, _p(out["xys"]), _p(out["conics"]), _p(out["depths"]), _p(out["radii"]),
                            _p(out["rect"]), _p(out["colors"]), _p(out["cov2d"]))
    return out


def raster3d_fwd(proj: dict, bins: dict, cam: OrcCamera, opacities, background):
    H, W = cam.height, cam.width
    out = dict(out_img=np.zeros((H, W, 3), np.float32), final_T=np.zeros((H, W), np.float32),
               final_idx=np.zeros((H, W), np.int32))
    ids = bins["ids"] if bins["ids"].size else np.zeros(1, np.int32)
    op, bgf = _f(opacities).reshape(-1), _f(background)
    lib().orc_raster3d_fwd(C.byref(cam), _p(bins["tile_offsets"]), _p(ids), _p(proj["xys"]), _p(proj["conics"]),
                           _p(proj["colors"]), _p(op), _p(bgf), _p(out["out_img"]), _p(out["final_T"]),
                           _p(out["final_idx"]))
    return out


def raster3d_bwd(proj, bins, fwd, cam, opacities, background, dL_dimg, with_abs=False):
    """[N,9] = (dL/dxy 2, dL/dconic 3, dL/dopacity logit, dL/dcolor 3)."""
    n = proj["radii"].shape[0]
    g = np.zeros((n, 9), np.float32)
    ga = np.zeros((n, 9), np.float32) if with_abs else None
    ids = bins["ids"] if bins["ids"].size else np.zeros(1, np.int32)
    op, bgf, dl = _f(opacities).reshape(-1), _f(background), _f(dL_dimg)
    lib().orc_raster3d_bwd(C.byref(cam), n, _p(bins["tile_offsets"]), _p(ids), _p(proj["xys"]), _p(proj["conics"]),
                           _p(proj["colors"]), _p(op), _p(bgf), _p(fwd["final_T"]), _p(fwd["final_idx"]), _p(dl),
                           _p(g), _p(ga))
    return (g, ga) if with_abs else g


def project3d_bwd(params: dict, cam, degree, dtu, radii, grads9, stats=None, glob_scale=1.0):
    m = _f(params["means"])
    n = m.shape[0]
    K = (degree + 1) ** 2 - 1
    out = dict(dmeans=np.zeros((n, 3), np.float32), dscales=np.zeros((n, 3), np.float32),
               dquats=np.zeros((n, 4), np.float32), dmean2d=np.zeros((n, 2), np.float32),
               dfdc=np.zeros((n, 3), np.float32), dfrest=np.zeros((n, max(K, 0), 3), np.float32))
    if stats is None:
        stats = dict(grad_norm=np.zeros(n, np.float32), vis=np.zeros(n, np.float32), max2d=np.zeros(n, np.float32))
    inv_max_dim = np.float32(1.0) / np.float32(max(cam.width, cam.height))
    sc, qu, fr = _f(params["scales"]), _f(params["quats"]), _f(params["features_rest"])
    rad, g9 = np.ascontiguousarray(radii, np.int32), _f(grads9)
    lib().orc_project3d_bwd(n, _p(m), _p(sc), _p(qu), _p(fr), degree, dtu, C.byref(cam), glob_scale, _p(rad), _p(g9),
                            *[_p(out[k]) for k in ("dmeans", "dscales", "dquats", "dmean2d", "dfdc", "dfrest")],
                            _p(stats["grad_norm"]), _p(stats["vis"]), _p(stats["max2d"]), float(inv_max_dim))
    out.update(stats)
    return out


def train_step3d(params: dict, exp_avg: dict, exp_avg_sq: dict, cam, background, gt, degree, dtu, adam_lr,
                 adam_step, stats, ssim_weight=0.2):
    """One golden-model 3DGS training step in place (Model::fullIteration,
    core/src/model.cpp:762-829, in the 3DGS mode): projection, binning,
    compositing, SSIM + L1 (no distortion), the raster and projection
    backwards, Adam on the six groups with the step's bias corrections
    (model.cpp:767-768).  params / exp_avg / exp_avg_sq: dicts of the six
    groups (scales [N,3]).  Returns (loss, image, intersections)."""
    proj = project3d_fwd(params, cam, degree, dtu)
    bins = bin_sort(proj, cam)
    fwd = raster3d_fwd(proj, bins, cam, params["opacities"], background)
    loss, dL, _, _ = loss_fwd_bwd(fwd["out_img"], gt, lambda_l1=1.0 - ssim_weight, lambda_dssim=ssim_weight)
    g9 = raster3d_bwd(proj, bins, fwd, cam, params["opacities"], background, dL)
    g = project3d_bwd(params, cam, degree, dtu, proj["radii"], g9, stats)
    grads = dict(means=g["dmeans"], scales=g["dscales"], quats=g["dquats"], features_dc=g["dfdc"],
                 features_rest=g["dfrest"], opacities=np.ascontiguousarray(g9[:, 5:6]))
    b1, b2 = np.float32(0.9), np.float32(0.999)
    bc1 = np.float32(1.0 - np.power(np.float64(b1), adam_step))
    bc2 = np.float32(1.0 - np.power(np.float64(b2), adam_step))
    bc2_sqrt = float(np.sqrt(bc2, dtype=np.float32))
    for k, lr in zip(("means", "scales", "quats", "features_dc", "features_rest", "opacities"), adam_lr):
        pk = params[k]
        assert pk.dtype == np.float32 and pk.flags.c_contiguous
        adam(pk, np.ascontiguousarray(grads[k], np.float32).reshape(pk.shape), exp_avg[k], exp_avg_sq[k],
             float(np.float32(lr) / bc1), float(b1), float(b2), bc2_sqrt, 1e-8)
    return float(loss), fwd["out_img"], int(bins["num_intersections"])
