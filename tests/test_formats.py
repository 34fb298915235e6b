"""On-disk formats, byte for byte, against golden layouts built here from the
reference writers' specifications:

  .msplat  core/src/model.cpp:343-498: u32 magic 0x4C50534D, u32 version 1,
           u32 step / num_active / shDegree / adam_step_count, f32 adam_lr[6],
           f32 means lr init / final, then 18 tensors (6 parameter groups, 6
           first and 6 second moments) as u32 ndim, i64 shape[ndim],
           u64 nbytes, raw float32;
  PLY      core/src/loaders/save_gaussians.cpp:11-58: the text header
           (comment "msplat v<step>", the property list in order) and rows of
           x y z, three zero normals, f_dc_0..2, f_rest channel-major,
           opacity, scale_0..S-1, rot_0..3;
  .splat   save_gaussians.cpp:60-112: 32-byte rows sorted by decreasing
           (sum of exp(scale)) * sigmoid(opacity): position, exp(scale) with
           the surfel's third axis 1e-5, RGB (uint8)clamp((dc C0 + 0.5) 255)
           in double, alpha (uint8)clamp(sigmoid 255), rotation
           (uint8)clamp(q 128 + 128).
The writers under test are the C++ Model's (through the C ABI) and the
package's Python checkpoint writer; PLY resume reads 2- and 3-scale rows.
"""
import ctypes as C
import ctypes.util
import struct

import numpy as np
import pytest

SH_C0 = 0.28209479177387814
LIBM = C.CDLL(ctypes.util.find_library("m"))
LIBM.expf.restype = C.c_float
LIBM.expf.argtypes = [C.c_float]


def expf(x):
    """libm expf: the float exp the C++ writers call (std::exp(float))."""
    return np.float32(LIBM.expf(float(x)))


def _scene(n=97, seed=3):
    """Parameters with distinct values (no ties in the .splat order)."""
    rng = np.random.default_rng(seed)
    p = dict(means=rng.normal(0, 1, (n, 3)), scales=rng.normal(-3, 0.7, (n, 2)),
             quats=rng.normal(0, 1, (n, 4)), features_dc=rng.normal(0, 1, (n, 3)),
             features_rest=rng.normal(0, 0.1, (n, 15, 3)), opacities=rng.normal(0, 1.5, (n, 1)))
    p["quats"] /= np.linalg.norm(p["quats"], axis=1, keepdims=True)
    return {k: v.astype(np.float32) for k, v in p.items()}


ORDER = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")


def golden_msplat(p, step, sh, adam_step, lr, lr0, lr1, m=None, v=None):
    out = bytearray(struct.pack("<I", 0x4C50534D) + struct.pack("<I", 1))
    out += struct.pack("<IIII", step, p["means"].shape[0], sh, adam_step)
    out += b"".join(struct.pack("<f", x) for x in lr) + struct.pack("<f", lr0) + struct.pack("<f", lr1)
    tensors = [p[k] for k in ORDER]
    tensors += m if m is not None else [np.zeros_like(t) for t in tensors[:6]]
    tensors += v if v is not None else [np.zeros_like(t) for t in tensors[:6]]
    for t in tensors:
        out += struct.pack("<I", t.ndim)
        for s in t.shape:
            out += struct.pack("<q", s)
        out += struct.pack("<Q", t.size * 4)
        out += np.ascontiguousarray(t, "<f4").tobytes()
    return bytes(out)


def golden_ply(p, step, scales=None, comment=None):
    sc = p["scales"] if scales is None else scales
    n, nfr, ns = p["means"].shape[0], p["features_rest"].shape[1], sc.shape[1]
    head = ["ply", "format binary_little_endian 1.0", comment or f"comment msplat v{step}", f"element vertex {n}"]
    head += [f"property float {c}" for c in ("x", "y", "z", "nx", "ny", "nz")]
    head += [f"property float f_dc_{i}" for i in range(3)]
    head += [f"property float f_rest_{i}" for i in range(3 * nfr)]
    head += ["property float opacity"] + [f"property float scale_{i}" for i in range(ns)]
    head += [f"property float rot_{i}" for i in range(4)] + ["end_header"]
    rows = []
    for i in range(n):
        r = list(p["means"][i]) + [0.0, 0.0, 0.0] + list(p["features_dc"][i])
        r += [p["features_rest"][i, b, ch] for ch in range(3) for b in range(nfr)]
        r += [p["opacities"][i, 0]] + list(sc[i]) + list(p["quats"][i])
        rows.append(struct.pack(f"<{len(r)}f", *r))
    return ("\n".join(head) + "\n").encode() + b"".join(rows)


def golden_splat(p):
    n = p["means"].shape[0]
    one = np.float32(1.0)
    key = []
    for i in range(n):
        s = np.float32(0.0)
        for j in range(p["scales"].shape[1]):
            s = np.float32(s + expf(p["scales"][i, j]))
        key.append(np.float32(s / np.float32(one + expf(-p["opacities"][i, 0]))))
    order = sorted(range(n), key=lambda i: -key[i])
    assert len(set(key)) == n
    out = bytearray()
    for i in order:
        out += struct.pack("<3f", *p["means"][i])
        sc = [expf(p["scales"][i, 0]), expf(p["scales"][i, 1]), np.float32(1e-5)]
        out += struct.pack("<3f", *sc)
        rgb = [int(min(max((float(p["features_dc"][i, j]) * SH_C0 + 0.5) * 255.0, 0.0), 255.0)) for j in range(3)]
        sig = np.float32(one / np.float32(one + expf(-p["opacities"][i, 0])))
        a = int(min(max(np.float32(sig * np.float32(255.0)), 0.0), 255.0))
        q = [int(min(max(np.float32(p["quats"][i, j] * np.float32(128.0) + np.float32(128.0)), 0.0), 255.0))
             for j in range(4)]
        out += bytes(rgb + [a] + q)
    return bytes(out)


# ---------------------------------------------------------------- CPU ----
def test_python_checkpoint_writer_is_byte_exact(tmp_path):
    from msplat import formats
    p = _scene()
    lr = (0.0001, 0.004, 0.002, 0.003, 0.0001, 0.04)
    rng = np.random.default_rng(9)
    m = [rng.normal(size=p[k].shape).astype(np.float32) for k in ORDER]
    v = [rng.uniform(size=p[k].shape).astype(np.float32) for k in ORDER]
    path = tmp_path / "a.msplat"
    formats.write_checkpoint(path, p, 3, step=1234, adam_step=77, adam_lr=lr, means_lr=(2e-4, 2e-6), exp_avg=m,
                             exp_avg_sq=v)
    assert path.read_bytes() == golden_msplat(p, 1234, 3, 77, lr, 2e-4, 2e-6, m, v)
    back = formats.read_checkpoint(path)
    assert back["step"] == 1234 and back["adam_step"] == 77 and back["sh_degree"] == 3
    for k in ORDER:
        assert np.array_equal(back["params"][k], p[k])
    for a, b in zip(back["exp_avg"] + back["exp_avg_sq"], m + v):
        assert np.array_equal(a, b)


def test_golden_layouts_are_what_the_spec_says():
    """Sizes and offsets of the golden layouts themselves."""
    p = _scene(n=5)
    ply = golden_ply(p, 12)
    head, body = ply.split(b"end_header\n")
    assert head.startswith(b"ply\nformat binary_little_endian 1.0\ncomment msplat v12\nelement vertex 5\n")
    assert len(body) == 5 * 4 * (3 + 3 + 3 + 45 + 1 + 2 + 4)
    row0 = struct.unpack("<61f", body[:244])
    assert row0[6:9] == tuple(np.float32(p["features_dc"][0]).tolist())
    assert row0[9] == np.float32(p["features_rest"][0, 0, 0]) and row0[10] == np.float32(p["features_rest"][0, 1, 0])
    assert row0[9 + 15] == np.float32(p["features_rest"][0, 0, 1])  # channel-major
    assert len(golden_splat(p)) == 5 * 32
    ck = golden_msplat(p, 1, 3, 0, (0.1,) * 6, 0.1, 0.01)
    assert ck[:4] == b"MSPL" and len(ck) == 8 + 16 + 32 + sum(4 + 8 * p[k].ndim + 8 + p[k].size * 4 for k in ORDER) * 3


# ---------------------------------------------------------------- GPU ----
@pytest.fixture
def trainer():
    from msplat import capi
    L = capi.lib()
    img = np.zeros((24, 32, 3), np.float32)
    cam = capi.CameraImage(width=32, height=24, fx=32.0, fy=32.0, cx=16.0, cy=12.0)
    cam.camToWorld[:] = [1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 3, 0, 0, 0, 1]
    cam.rgb = img.ctypes.data
    pts = np.random.default_rng(1).uniform(-1, 1, (16, 3)).astype(np.float32)
    rgb = np.full((16, 3), 100, np.uint8)
    ds = L.msplat_dataset_create_from_memory(C.byref(cam), 1, pts.ctypes.data, rgb.ctypes.data, 16, False, 8)
    assert ds, capi.last_error()
    tr = L.msplat_trainer_create(ds, capi.default_config())
    assert tr, capi.last_error()
    yield L, tr
    L.msplat_trainer_destroy(tr)
    L.msplat_dataset_destroy(ds)


@pytest.mark.gpu
def test_checkpoint_ply_and_splat_writers_are_byte_exact(trainer, tmp_path, eng):
    L, tr = trainer
    p = _scene()
    lr = (0.0001, 0.004, 0.002, 0.003, 0.0001, 0.04)
    rng = np.random.default_rng(4)
    m = [rng.normal(size=p[k].shape).astype(np.float32) for k in ORDER]
    v = [rng.uniform(size=p[k].shape).astype(np.float32) for k in ORDER]
    src = tmp_path / "in.msplat"
    src.write_bytes(golden_msplat(p, 4321, 3, 55, lr, 3e-4, 3e-6, m, v))
    assert L.msplat_trainer_load_checkpoint(tr, str(src).encode()) == 4321
    assert L.msplat_trainer_splat_count(tr) == p["means"].shape[0]
    out = tmp_path / "out.msplat"
    L.msplat_trainer_save_checkpoint(tr, str(out).encode())
    assert out.read_bytes() == src.read_bytes()
    ply = tmp_path / "s.ply"
    L.msplat_trainer_export_ply(tr, str(ply).encode())
    assert ply.read_bytes() == golden_ply(p, 4321)
    spl = tmp_path / "s.splat"
    L.msplat_trainer_export_splat(tr, str(spl).encode())
    assert spl.read_bytes() == golden_splat(p)


@pytest.mark.gpu
def test_ply_resume_two_and_three_scales(trainer, tmp_path, eng):
    from msplat import formats
    L, tr = trainer
    p = _scene(n=61, seed=8)
    for scales, comment, step in [(p["scales"], None, 900),
                                  (np.c_[p["scales"], np.full((61, 1), -7.0, np.float32)],
                                   "comment Generated by msplat at iteration 1234", 1234)]:
        src = tmp_path / f"r{scales.shape[1]}.ply"
        src.write_bytes(golden_ply(p, step, scales, comment))
        assert L.msplat_trainer_load_ply(tr, str(src).encode()) == step
        assert L.msplat_trainer_iteration(tr) == step
        ck = tmp_path / f"r{scales.shape[1]}.msplat"
        L.msplat_trainer_save_checkpoint(tr, str(ck).encode())
        back = formats.read_checkpoint(ck)
        assert back["step"] == step and back["sh_degree"] == 3 and back["adam_step"] == 0
        for k in ORDER:
            assert np.array_equal(back["params"][k], p[k]), k  # 3-scale rows keep the first two scales
        assert all(not a.any() for a in back["exp_avg"] + back["exp_avg_sq"])
        # the optimiser starts over: the reference's learning-rate table
        assert np.allclose(back["adam_lr"], (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05))
        # and the resumed scene trains
        s = L.msplat_trainer_step(tr)
        assert s.iteration == step + 1 and np.isfinite(s.loss)
    bad = tmp_path / "bad.ply"
    bad.write_bytes(golden_ply(p, 1).replace(b"property float scale_1\n", b""))
    assert L.msplat_trainer_load_ply(tr, str(bad).encode()) == -1
