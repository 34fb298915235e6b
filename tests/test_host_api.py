"""Host layer on the CPU: the trainer's C ABI exports, the Python surface of
the reference's msplat._core stubs, image decoding and the dataset loaders
(COLMAP / Nerfstudio / Polycam).  Nothing here touches the GPU."""
from __future__ import annotations

import ctypes as C
import json
import os
import re
import struct
import subprocess
import sys
import zlib
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]


def _header_functions(path: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msplat_\w+)\s*\(", text)))


def test_c_api_header_symbols_are_exported():
    from msplat import _engine as E

    lib = E.lib()
    names = _header_functions(REPO / "include" / "msplat_c_api.h")
    # every function of the reference's C ABI is declared (msplat_c_api.h:83-127)
    reference = {
        "msplat_dataset_create", "msplat_dataset_destroy", "msplat_dataset_num_train", "msplat_dataset_num_test",
        "msplat_dataset_camera_pose", "msplat_trainer_create", "msplat_trainer_destroy", "msplat_trainer_step",
        "msplat_trainer_train", "msplat_trainer_evaluate", "msplat_trainer_render", "msplat_trainer_render_pose",
        "msplat_trainer_render_pose_to_buffer", "msplat_trainer_export_ply", "msplat_trainer_export_splat",
        "msplat_trainer_extract_mesh", "msplat_trainer_save_checkpoint", "msplat_trainer_load_checkpoint",
        "msplat_trainer_splat_count", "msplat_trainer_iteration", "msplat_set_metallib_path", "msplat_sync",
        "msplat_cleanup",
    }
    assert reference <= set(names)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_c_api_config_struct_layout():
    """MsplatConfig is 16 fields (msplat_c_api.h:16-33): 13 x 4-byte fields,
    a bool, a float and float[3], with natural alignment -> 72 bytes."""
    class MsplatConfig(C.Structure):
        _fields_ = [("iterations", C.c_int), ("shDegree", C.c_int), ("shDegreeInterval", C.c_int),
                    ("ssimWeight", C.c_float), ("numDownscales", C.c_int), ("resolutionSchedule", C.c_int),
                    ("refineEvery", C.c_int), ("warmupLength", C.c_int), ("resetAlphaEvery", C.c_int),
                    ("densifyGradThresh", C.c_float), ("densifySizeThresh", C.c_float),
                    ("stopScreenSizeAt", C.c_int), ("splitScreenSize", C.c_float), ("keepCrs", C.c_bool),
                    ("downscaleFactor", C.c_float), ("bgColor", C.c_float * 3)]
    assert C.sizeof(MsplatConfig) == 72
    from msplat import _engine as E

    lib = E.lib()
    lib.msplat_dataset_create.restype = C.c_void_p
    lib.msplat_last_error.restype = C.c_char_p
    # a failing create returns NULL and records the message (no exception crosses the ABI)
    assert lib.msplat_dataset_create(b"/nonexistent/dataset", C.c_float(1.0), False, 8) is None
    assert b"Unrecognized dataset format" in lib.msplat_last_error()


def test_python_surface_matches_reference_stubs():
    import msplat

    c = msplat.TrainingConfig()
    expected = dict(iterations=30000, sh_degree=3, sh_degree_interval=1000, ssim_weight=0.2, num_downscales=2,
                    resolution_schedule=3000, refine_every=100, warmup_length=500, reset_alpha_every=30,
                    densify_grad_thresh=0.0002, densify_size_thresh=0.01, stop_screen_size_at=4000,
                    split_screen_size=0.05, keep_crs=False, downscale_factor=1.0, output="splat.ply", save_every=-1)
    for k, v in expected.items():
        assert getattr(c, k) == pytest.approx(v), k
    assert c.bg_color == pytest.approx([0.6130, 0.0101, 0.3984])
    c2 = msplat.TrainingConfig(iterations=7, bg_color=[0.0, 0.5, 1.0])
    assert c2.iterations == 7 and c2.bg_color == [0.0, 0.5, 1.0]
    with pytest.raises(ValueError):
        msplat.TrainingConfig(bg_color=[1.0, 2.0])
    with pytest.raises(ValueError):
        c2.bg_color = [1.0]
    for name in ("step", "train", "evaluate", "render", "render_from_pose", "export_ply", "export_splat",
                 "save_checkpoint", "load_checkpoint", "splat_count", "iteration"):
        assert hasattr(msplat.GaussianTrainer, name), name
    for name in ("num_train", "num_test", "camera_pose"):
        assert hasattr(msplat.Dataset, name), name
    for name in ("iteration", "splat_count", "ms_per_step"):
        assert hasattr(msplat.TrainingStats, name), name
    for name in ("TrainingConfig", "TrainingStats", "Dataset", "GaussianTrainer", "sync", "cleanup",
                 "load_dataset"):
        assert name in msplat.__all__
    with pytest.raises(RuntimeError):
        msplat.load_dataset("/nonexistent/dataset")


def test_core_stub_matches_module():
    """msplat/_core.pyi declares exactly the module's public classes,
    functions, methods and properties."""
    import ast

    from msplat import _core

    stub = ast.parse((REPO / "msplat-ios_amd" / "msplat" / "_core.pyi").read_text())
    declared = {}
    for node in stub.body:
        if isinstance(node, ast.ClassDef):
            members = set()
            for item in node.body:
                if isinstance(item, ast.FunctionDef) and not item.name.startswith("__"):
                    members.add(item.name)
                elif isinstance(item, ast.AnnAssign):
                    members.add(item.target.id)
            declared[node.name] = members
        elif isinstance(node, ast.FunctionDef):
            declared[node.name] = None
    public = {n for n in dir(_core) if not n.startswith("_")}
    assert set(declared) == public
    for name, members in declared.items():
        if members is None:
            continue
        actual = {m for m in dir(getattr(_core, name)) if not m.startswith("_")}
        assert members == actual, (name, members ^ actual)


# ---------------------------------------------------------------- images --

def _png(path: Path, rows: np.ndarray, color_type: int, depth: int, palette=None, interlace=False, filters=None):
    """Independent PNG encoder for the decoder test: rows is (H, W, C) of
    integer samples; every scanline uses filters[y % len(filters)]."""
    h, w = rows.shape[:2]
    chans = rows.shape[2]
    filters = filters or [0, 1, 2, 3, 4]

    def pack(img):
        out = []
        for y in range(img.shape[0]):
            samples = img[y].reshape(-1)
            if depth == 16:
                raw = b"".join(struct.pack(">H", int(s)) for s in samples)
            elif depth == 8:
                raw = bytes(int(s) for s in samples)
            else:
                bits = "".join(format(int(s), f"0{depth}b") for s in samples)
                bits += "0" * (-len(bits) % 8)
                raw = bytes(int(bits[i:i + 8], 2) for i in range(0, len(bits), 8))
            out.append(raw)
        return out

    bpp = max(1, chans * depth // 8)

    def filt(lines, y0):
        res = b""
        prev = bytes(len(lines[0])) if lines else b""
        for y, line in enumerate(lines):
            f = filters[(y0 + y) % len(filters)]
            o = bytearray()
            for i, x in enumerate(line):
                a = line[i - bpp] if i >= bpp else 0
                b = prev[i]
                c = prev[i - bpp] if i >= bpp else 0
                if f == 0:
                    p = 0
                elif f == 1:
                    p = a
                elif f == 2:
                    p = b
                elif f == 3:
                    p = (a + b) // 2
                else:
                    pa, pb, pc = abs(b - c), abs(a - c), abs(a + b - 2 * c)
                    p = a if pa <= pb and pa <= pc else (b if pb <= pc else c)
                o.append((x - p) & 255)
            res += bytes([f]) + bytes(o)
            prev = line
        return res

    if not interlace:
        data = filt(pack(rows), 0)
    else:
        data = b""
        for sx, sy, dx, dy in ((0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2),
                               (0, 1, 1, 2)):
            sub = rows[sy::dy, sx::dx]
            if sub.shape[0] and sub.shape[1]:
                data += filt(pack(sub), 0)

    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)

    ihdr = struct.pack(">IIBBBBB", w, h, depth, color_type, 0, 0, 1 if interlace else 0)
    blob = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", ihdr)
    if palette is not None:
        blob += chunk(b"PLTE", bytes(palette.astype(np.uint8).reshape(-1)))
    blob += chunk(b"IDAT", zlib.compress(data)) + chunk(b"IEND", b"")
    path.write_bytes(blob)


@pytest.mark.parametrize("case", ["rgb8", "rgba8", "gray8", "gray16", "rgb16", "graya8", "gray1", "gray4",
                                  "palette8", "palette2", "rgb8_adam7", "gray2_adam7"])
def test_png_decoder(case, tmp_path):
    from msplat import _core

    rng = np.random.default_rng(hash(case) % 2**32)
    h, w = 13, 11
    if case.startswith("rgb8"):
        s = rng.integers(0, 256, (h, w, 3))
        exp = s / 255.0
        _png(tmp_path / "a.png", s, 2, 8, interlace="adam7" in case)
    elif case == "rgba8":
        s = rng.integers(0, 256, (h, w, 4))
        exp = s[..., :3] / 255.0
        _png(tmp_path / "a.png", s, 6, 8)
    elif case == "gray8":
        s = rng.integers(0, 256, (h, w, 1))
        exp = np.repeat(s / 255.0, 3, 2)
        _png(tmp_path / "a.png", s, 0, 8)
    elif case == "gray16":
        s = rng.integers(0, 65536, (h, w, 1))
        exp = np.repeat(s / 65535.0, 3, 2)
        _png(tmp_path / "a.png", s, 0, 16)
    elif case == "rgb16":
        s = rng.integers(0, 65536, (h, w, 3))
        exp = s / 65535.0
        _png(tmp_path / "a.png", s, 2, 16)
    elif case == "graya8":
        s = rng.integers(0, 256, (h, w, 2))
        exp = np.repeat(s[..., :1] / 255.0, 3, 2)
        _png(tmp_path / "a.png", s, 4, 8)
    elif case.startswith("gray") and case[4].isdigit():
        d = int(case[4])
        s = rng.integers(0, 2 ** d, (h, w, 1))
        exp = np.repeat(s / (2 ** d - 1), 3, 2)
        _png(tmp_path / "a.png", s, 0, d, interlace="adam7" in case)
    else:  # palette
        d = int(case[-1])
        pal = rng.integers(0, 256, (2 ** d, 3))
        s = rng.integers(0, 2 ** d, (h, w, 1))
        exp = pal[s[..., 0]] / 255.0
        _png(tmp_path / "a.png", s, 3, d, palette=pal)
    got = _core._read_image(str(tmp_path / "a.png"))
    assert got.shape == (h, w, 3)
    assert np.abs(got - exp).max() < 1e-6
    if case in ("rgb8", "rgba8", "gray8", "palette8", "rgb8_adam7"):
        # the test's encoder agrees with an independent decoder
        from PIL import Image

        ref = np.asarray(Image.open(tmp_path / "a.png").convert("RGB"), np.float64) / 255.0
        assert np.abs(ref - exp).max() < 1e-6


def test_pnm_decoder(tmp_path):
    from msplat import _core

    rng = np.random.default_rng(3)
    s = rng.integers(0, 256, (5, 7, 3)).astype(np.uint8)
    (tmp_path / "a.ppm").write_bytes(b"P6\n# comment\n7 5\n255\n" + s.tobytes())
    assert np.abs(_core._read_image(str(tmp_path / "a.ppm")) - s / 255.0).max() < 1e-6
    g = rng.integers(0, 65536, (4, 3)).astype(">u2")
    (tmp_path / "b.pgm").write_bytes(b"P5 3 4 65535\n" + g.tobytes())
    assert np.abs(_core._read_image(str(tmp_path / "b.pgm")) - np.repeat(g[..., None] / 65535.0, 3, 2)).max() < 1e-6
    with pytest.raises(RuntimeError):
        _core._read_image(str(tmp_path / "missing.png"))


# ------------------------------------------------------------------ JPEG --
JPEG_DIR = Path(__file__).resolve().parent / "golden" / "jpeg"


def test_jpeg_decoder_matches_libjpeg_fixtures():
    """Baseline (4:2:0, 4:2:2, 4:4:4, odd sizes, greyscale, optimised
    tables, low quality), progressive and restart-interval JPEGs encoded by
    PIL, against PIL's own decoding (tests/golden/make_jpeg_fixtures.py).
    Both decoders run a compliant 8x8 inverse DCT, and two compliant
    inverse DCTs may differ by one level per sample (IEEE 1180); the colour
    transform carries a chroma difference into RGB scaled by up to 1.772.
    So greyscale must agree to +-1, colour to +-3 with under 1% of samples
    off by more than 1 and a mean difference under 0.1 levels."""
    from msplat import _core
    exp = np.load(JPEG_DIR / "jpeg_expected.npz")
    assert len(exp.files) >= 12
    for name in exp.files:
        got = np.asarray(_core._read_image(str(JPEG_DIR / f"{name}.jpg")))
        want = exp[name].astype(np.int32)
        assert got.shape == want.shape, name
        d = np.abs(np.round(got * 255.0).astype(np.int32) - want)
        grey = "grey" in name
        assert d.max() <= (1 if grey else 3), (name, d.max())
        assert (d > 1).mean() < 0.01 and d.mean() < 0.1, (name, (d > 1).mean(), d.mean())


def test_jpeg_decoder_rejects_bad_input(tmp_path):
    """Truncated data, arithmetic coding, 12-bit samples and garbage raise
    (a RuntimeError through the bindings), they do not crash."""
    from msplat import _core
    raw = (JPEG_DIR / "base420.jpg").read_bytes()
    cases = {"trunc_header": raw[:40], "garbage": b"\xff\xd8" + bytes(range(256)) * 4}
    sof = raw.index(b"\xff\xc0")
    cases["arith"] = raw[:sof] + b"\xff\xc9" + raw[sof + 2:]
    cases["12bit"] = raw[:sof + 4] + b"\x0c" + raw[sof + 5:]
    for name, blob in cases.items():
        (tmp_path / f"{name}.jpg").write_bytes(blob)
        with pytest.raises(RuntimeError):
            _core._read_image(str(tmp_path / f"{name}.jpg"))


def test_jpeg_decoder_survives_corruption(tmp_path):
    """Hundreds of randomly truncated or byte-flipped fixtures decode or
    raise; the process must not crash (run in a child process)."""
    script = tmp_path / "fuzz.py"
    script.write_text(f"""
import sys, random
sys.path.insert(0, {str(Path(__file__).resolve().parent.parent / 'msplat-ios_amd')!r})
from pathlib import Path
from msplat import _core
rng = random.Random(7)
files = sorted(Path({str(JPEG_DIR)!r}).glob('*.jpg'))
out = Path({str(tmp_path)!r}) / 'x.jpg'
ok = bad = 0
for k in range(400):
    raw = bytearray(rng.choice(files).read_bytes())
    if k % 2:
        raw = raw[: rng.randrange(2, len(raw))]
    for _ in range(rng.randrange(1, 6)):
        raw[rng.randrange(2, len(raw))] = rng.randrange(256)
    out.write_bytes(bytes(raw))
    try:
        _core._read_image(str(out))
        ok += 1
    except RuntimeError:
        bad += 1
print(ok, bad)
""")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    ok, bad = map(int, r.stdout.split())
    assert ok + bad == 400


def test_colmap_loader_with_jpeg_images(tmp_path):
    """A COLMAP capture whose images are JPEG (as real captures ship) loads
    through the dataset API; the decoded pixels reach the cameras."""
    import msplat
    from PIL import Image

    sp = tmp_path / "sparse" / "0"
    sp.mkdir(parents=True)
    (tmp_path / "images").mkdir()
    rng = np.random.default_rng(6)
    for i in range(3):
        s = (rng.uniform(0, 1, (12, 16, 3)) * 255).astype(np.uint8)
        Image.fromarray(s).save(tmp_path / "images" / f"frame_{i:03d}.jpg", quality=90)
    poses_gl = [_look_at_c2w((2 * np.cos(a), 0.5, 2 * np.sin(a))) for a in (0.1, 1.2, 2.3)]
    with open(sp / "cameras.bin", "wb") as f:
        f.write(struct.pack("<Q", 1))
        f.write(struct.pack("<IiQQ", 1, 1, 16, 12) + struct.pack("<4d", 20.0, 21.0, 8.0, 6.0))
    with open(sp / "images.bin", "wb") as f:
        f.write(struct.pack("<Q", 3))
        for i, c2w in enumerate(poses_gl):
            cv = c2w.copy()
            cv[:3, 1:3] *= -1
            R = cv[:3, :3].T
            t = -R @ cv[:3, 3]
            f.write(struct.pack("<I", i + 1) + struct.pack("<4d", *_qvec(R)) + struct.pack("<3d", *t))
            f.write(struct.pack("<I", 1) + f"frame_{i:03d}.jpg".encode() + b"\0")
            f.write(struct.pack("<Q", 0))
    with open(sp / "points3D.bin", "wb") as f:
        f.write(struct.pack("<Q", 4))
        for k, p in enumerate(rng.normal(size=(4, 3))):
            f.write(struct.pack("<Q3d3Bd", k, *p, 1, 2, 3, 0.5) + struct.pack("<Q", 1) + struct.pack("<II", 1, 0))
    ds = msplat.Dataset(str(tmp_path))
    assert ds.num_train == 3


# --------------------------------------------------------------- loaders --

def _look_at_c2w(eye, target=(0.0, 0.0, 0.0)):
    """Camera-to-world, OpenGL axes (x right, y up, z back)."""
    eye = np.asarray(eye, np.float64)
    z = eye - np.asarray(target)
    z /= np.linalg.norm(z)
    x = np.cross([0.0, 1.0, 0.0], z)
    x /= np.linalg.norm(x)
    y = np.cross(z, x)
    m = np.eye(4)
    m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = x, y, z, eye
    return m


def _normalised(poses):
    """autoScaleAndCenter (input_data.cpp:124-160) in numpy."""
    t = np.stack([p[:3, 3] for p in poses])
    mean = t.mean(0)
    t = t - mean
    s = 1.0 / np.abs(t).max()
    out = []
    for p, ti in zip(poses, t):
        q = p.copy()
        q[:3, 3] = ti * s
        out.append(q)
    return out, mean, s


def _write_images(folder: Path, n, h=12, w=16):
    folder.mkdir(parents=True, exist_ok=True)
    rng = np.random.default_rng(5)
    imgs = []
    for i in range(n):
        s = rng.integers(0, 256, (h, w, 3))
        _png(folder / f"frame_{i:03d}.png", s, 2, 8)
        imgs.append(s / 255.0)
    return imgs


def test_nerfstudio_loader(tmp_path):
    import msplat

    poses = [_look_at_c2w((3 * np.cos(a), 1.0, 3 * np.sin(a))) for a in np.linspace(0, 5, 6)]
    _write_images(tmp_path / "images", 6)
    frames = [dict(file_path=f"images/frame_{i:03d}", transform_matrix=p.tolist()) for i, p in enumerate(poses)]
    (tmp_path / "transforms.json").write_text(json.dumps(dict(w=16, h=12, fl_x=20.0, fl_y=21.0, cx=8.0, cy=6.0,
                                                              frames=frames[::-1])))
    pts = np.random.default_rng(1).normal(size=(40, 3)).astype(np.float32)
    with open(tmp_path / "points3D.ply", "w") as f:
        f.write("ply\nformat ascii 1.0\nelement vertex 40\nproperty float x\nproperty float y\nproperty float z\n"
                "property uchar red\nproperty uchar green\nproperty uchar blue\nend_header\n")
        for p in pts:
            f.write(f"{p[0]} {p[1]} {p[2]} 10 20 30\n")
    ds = msplat.Dataset(str(tmp_path), eval_mode=True, test_every=3)
    assert (ds.num_train, ds.num_test) == (4, 2)
    norm, _, _ = _normalised(poses)
    train_ids = [i for i in range(6) if i % 3 != 0]  # frames sorted by path, every 3rd held out
    for k, i in enumerate(train_ids):
        assert np.abs(ds.camera_pose(k) - norm[i]).max() < 1e-5
    with pytest.raises(RuntimeError):
        ds.camera_pose(4)


def test_nerfstudio_camera_angle_intrinsics(tmp_path):
    """Original-NeRF transforms.json: only camera_angle_x; w, h come from the
    first image (load_nerfstudio.cpp:78-118)."""
    import msplat

    poses = [_look_at_c2w((0.0, 0.0, 2.0 + i)) for i in range(2)]
    _write_images(tmp_path, 2)
    frames = [dict(file_path=f"frame_{i:03d}.png", transform_matrix=p.tolist()) for i, p in enumerate(poses)]
    (tmp_path / "transforms.json").write_text(json.dumps(dict(camera_angle_x=0.8, frames=frames)))
    ds = msplat.Dataset(str(tmp_path))
    assert ds.num_train == 2


def _qvec(R):
    """Rotation matrix -> quaternion (w, x, y, z)."""
    w = np.sqrt(max(0.0, 1 + R[0, 0] + R[1, 1] + R[2, 2])) / 2
    x = np.copysign(np.sqrt(max(0.0, 1 + R[0, 0] - R[1, 1] - R[2, 2])) / 2, R[2, 1] - R[1, 2])
    y = np.copysign(np.sqrt(max(0.0, 1 - R[0, 0] + R[1, 1] - R[2, 2])) / 2, R[0, 2] - R[2, 0])
    z = np.copysign(np.sqrt(max(0.0, 1 - R[0, 0] - R[1, 1] + R[2, 2])) / 2, R[1, 0] - R[0, 1])
    return np.array([w, x, y, z])


def test_colmap_loader(tmp_path):
    """COLMAP binary model: world-to-camera (q, t) in OpenCV axes become
    OpenGL camera-to-world poses, then centred and scaled."""
    import msplat

    sp = tmp_path / "sparse" / "0"
    sp.mkdir(parents=True)
    _write_images(tmp_path / "images", 4)
    poses_gl = [_look_at_c2w((2 * np.cos(a), 0.5, 2 * np.sin(a))) for a in (0.1, 1.2, 2.3, 3.4)]
    with open(sp / "cameras.bin", "wb") as f:
        f.write(struct.pack("<Q", 1))
        f.write(struct.pack("<IiQQ", 1, 1, 16, 12) + struct.pack("<4d", 20.0, 21.0, 8.0, 6.0))  # PINHOLE
    with open(sp / "images.bin", "wb") as f:
        f.write(struct.pack("<Q", 4))
        for i, c2w in enumerate(poses_gl):
            cv = c2w.copy()
            cv[:3, 1:3] *= -1  # OpenGL -> OpenCV camera axes
            R = cv[:3, :3].T
            t = -R @ cv[:3, 3]
            f.write(struct.pack("<I", i + 1) + struct.pack("<4d", *_qvec(R)) + struct.pack("<3d", *t))
            f.write(struct.pack("<I", 1) + f"frame_{i:03d}.png".encode() + b"\0")
            f.write(struct.pack("<Q", 2) + struct.pack("<ddq", 1.0, 2.0, -1) * 2)
    pts = np.random.default_rng(2).normal(size=(10, 3))
    with open(sp / "points3D.bin", "wb") as f:
        f.write(struct.pack("<Q", 10))
        for k, p in enumerate(pts):
            f.write(struct.pack("<Q3d3Bd", k, *p, 1, 2, 3, 0.5) + struct.pack("<Q", 1) + struct.pack("<II", 1, 0))
    ds = msplat.Dataset(str(tmp_path))
    assert ds.num_train == 4
    norm, _, _ = _normalised(poses_gl)
    for i in range(4):
        assert np.abs(ds.camera_pose(i) - norm[i]).max() < 1e-5


def test_polycam_cameras_json_loader(tmp_path):
    import msplat

    _write_images(tmp_path, 3)
    poses = [_look_at_c2w((1.0 + i, 0.3, 2.0)) for i in range(3)]
    frames = [dict(width=16, height=12, fx=20.0, fy=20.0, file_path=f"frame_{i:03d}.png",
                   transform_matrix=p.tolist()) for i, p in enumerate(poses)]
    (tmp_path / "cameras.json").write_text(json.dumps(dict(frames=frames)))
    ds = msplat.Dataset(str(tmp_path), eval_mode=True, test_every=8)
    assert (ds.num_train, ds.num_test) == (2, 1)


def test_dataset_from_arrays_validation():
    import msplat

    img = np.zeros((8, 8, 3), np.float32)
    with pytest.raises(ValueError):
        msplat.Dataset.from_arrays([img], np.eye(4, dtype=np.float32)[None], np.zeros((1, 3), np.float32))
    ds = msplat.Dataset.from_arrays([img, img], np.stack([np.eye(4)] * 2).astype(np.float32),
                                    np.array([[10, 10, 4, 4]] * 2, np.float32))
    assert ds.num_train == 2 and ds.num_test == 0


def _jpeg_segments(raw: bytes):
    """(marker, payload offset, payload length) of each header segment of a
    JPEG file up to its first scan."""
    out, p = [], 2
    while p + 4 <= len(raw):
        marker, ln = raw[p + 1], int.from_bytes(raw[p + 2:p + 4], "big")
        out.append((marker, p + 4, ln - 2))
        if marker == 0xDA:
            break
        p += 2 + ln
    return out


def _jpeg_crafted() -> dict:
    """Malformed variants of base420.jpg that a careless decoder would read
    or write out of bounds on: DHT counts that are not a prefix code (a DC
    and an AC table with every code at length 1), Huffman values outside
    the 8-bit ranges (a DC category of 15, an AC size of 14), and a frame
    with luma 3x3 and chroma 2x2 sampling (ratio 1.5)."""
    raw = (JPEG_DIR / "base420.jpg").read_bytes()
    seg = _jpeg_segments(raw)
    tables = []  # (class, counts offset, values offset, total)
    for marker, off, ln in seg:
        if marker != 0xC4:
            continue
        i = off
        while i < off + ln:
            total = sum(raw[i + 1:i + 17])
            tables.append((raw[i] >> 4, i + 1, i + 17, total))
            i += 17 + total
    out = {}
    for cls, name in ((0, "dc"), (1, "ac")):
        _, c_off, v_off, total = next(t for t in tables if t[0] == cls)
        b = bytearray(raw)
        b[c_off:c_off + 16] = bytes([total] + [0] * 15)  # all codes at length 1
        out[f"overfull_{name}"] = bytes(b)
        b = bytearray(raw)
        b[v_off] = 15 if cls == 0 else 0x0E
        out[f"badvalue_{name}"] = bytes(b)
    marker, off, ln = next(s for s in seg if s[0] == 0xC0)
    b = bytearray(raw)
    b[off + 7] = 0x33  # Y 3x3
    b[off + 10] = 0x22  # Cb 2x2
    b[off + 13] = 0x22  # Cr 2x2
    out["ratio_3_2"] = bytes(b)
    return out


def test_jpeg_decoder_rejects_malformed_tables(tmp_path):
    """Each crafted variant raises cleanly, in a child process so that a
    crash fails the test rather than ending the test run."""
    paths = []
    for name, blob in _jpeg_crafted().items():
        (tmp_path / f"{name}.jpg").write_bytes(blob)
        paths.append(str(tmp_path / f"{name}.jpg"))
    script = tmp_path / "crafted.py"
    script.write_text(f"""
import sys
sys.path.insert(0, {str(Path(__file__).resolve().parent.parent / 'msplat-ios_amd')!r})
from msplat import _core
for p in {paths!r}:
    try:
        _core._read_image(p)
        print('decoded', p)
    except RuntimeError as e:
        print('raised', p, e)
""")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.splitlines()
    assert len(lines) == len(paths) and all(ln.startswith("raised") for ln in lines), lines


def test_jpeg_decoder_under_address_sanitizer(tmp_path):
    """The decoder built with AddressSanitizer and UBSan (tests/native/
    jpeg_check.cpp, host code only) over every fixture, the crafted
    malformed files and 300 random corruptions: no sanitizer report, the
    fixtures decode, the crafted files are refused."""
    import shutil
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    repo = Path(__file__).resolve().parent.parent
    exe = tmp_path / "jpeg_check"
    cmd = [gxx, "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           f"-I{repo / 'msplat-ios_amd/csrc/host'}", f"-I{repo / 'include'}",
           str(repo / "tests/native/jpeg_check.cpp"), str(repo / "msplat-ios_amd/csrc/host/jpeg.cpp"), "-o", str(exe)]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if b.returncode != 0:
        pytest.skip(f"sanitizer build unavailable: {b.stderr[-500:]}")
    fixtures = sorted(JPEG_DIR.glob("*.jpg"))
    crafted = []
    for name, blob in _jpeg_crafted().items():
        (tmp_path / f"{name}.jpg").write_bytes(blob)
        crafted.append(tmp_path / f"{name}.jpg")
    rng = np.random.default_rng(11)
    fuzz = []
    for k in range(300):
        raw = bytearray(fixtures[k % len(fixtures)].read_bytes())
        if k % 2:
            raw = raw[: int(rng.integers(2, len(raw)))]
        for _ in range(int(rng.integers(1, 6))):
            raw[int(rng.integers(2, len(raw)))] = int(rng.integers(256))
        fuzz.append(tmp_path / f"f{k}.jpg")
        fuzz[-1].write_bytes(bytes(raw))
    files = fixtures + crafted + fuzz
    r = subprocess.run([str(exe), *map(str, files)], capture_output=True, text=True, timeout=600,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=0"})
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    lines = r.stdout.splitlines()
    assert len(lines) == len(files)
    assert all(ln.startswith("ok") for ln in lines[:len(fixtures)])
    assert all(ln.startswith("error") for ln in lines[len(fixtures):len(fixtures) + len(crafted)])


# ------------------------------------------------- evaluation metrics --
def _ssim_brute(a, b, pad="clamp"):
    """Mean SSIM over pixels and channels of (H, W, C) images with the 2D
    11x11 Gaussian window (sigma 1.5) applied directly (no separable pass),
    in float64: each window tap reads the pixel at the clamped coordinate
    (pad="clamp") or zero outside the image (pad="zero")."""
    H, W, C = a.shape
    x = np.arange(11) - 5
    g = np.exp(-(x * x) / (2 * 1.5 * 1.5))
    g /= g.sum()
    w2 = np.outer(g, g)
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    tot = 0.0
    for c in range(C):
        def blur(img):
            out = np.zeros((H, W))
            for y in range(H):
                for xx in range(W):
                    s = 0.0
                    for j in range(11):
                        for k in range(11):
                            yy, xk = y + j - 5, xx + k - 5
                            if pad == "clamp":
                                s += w2[j, k] * img[min(max(yy, 0), H - 1), min(max(xk, 0), W - 1)]
                            elif 0 <= yy < H and 0 <= xk < W:
                                s += w2[j, k] * img[yy, xk]
                    out[y, xx] = s
            return out
        p, q = a[..., c].astype(np.float64), b[..., c].astype(np.float64)
        m1, m2 = blur(p), blur(q)
        s11, s22, s12 = blur(p * p) - m1 * m1, blur(q * q) - m2 * m2, blur(p * q) - m1 * m2
        tot += (((2 * m1 * m2 + c1) * (2 * s12 + c2)) / ((m1 * m1 + m2 * m2 + c1) * (s11 + s22 + c2))).sum()
    return tot / (H * W * C)


def test_eval_metrics_known_answers():
    """PSNR / SSIM / L1 of Trainer.evaluate (csrc/host/eval.cpp after
    core/src/model.cpp:26-43 and core/src/ssim.cpp:37-123): identical images
    give SSIM 1 and L1 0; a constant offset d gives L1 = d and PSNR =
    -20 log10 d; SSIM equals a float64 brute-force 2D 11x11 window with
    clamp-to-edge padding on small images (smaller than the window, so most
    taps are clamped), and differs from the zero-padded one there, so a
    padding, window or normaliser slip fails."""
    from msplat import _core
    rng = np.random.default_rng(5)
    a = rng.uniform(0.1, 0.9, (9, 13, 3)).astype(np.float32)
    m = _core._metrics(a, a)
    assert abs(m["ssim"] - 1.0) < 1e-6 and m["l1"] == 0.0 and m["psnr"] > 200
    for d in (0.05, 0.0625, 0.1):
        b = a + np.float32(d)
        m = _core._metrics(b, a)
        dd = float(np.float32(b - a).mean())  # the offset after float32 rounding
        assert abs(m["l1"] - dd) < 1e-6
        mse = float(((b.astype(np.float64) - a) ** 2).mean())
        assert abs(m["psnr"] - 10 * np.log10(1 / mse)) < 1e-4
        assert abs(m["psnr"] + 20 * np.log10(d)) < 2e-3
    for shape in ((9, 13, 3), (16, 7, 3), (5, 5, 1)):
        p = rng.uniform(0, 1, shape).astype(np.float32)
        q = np.clip(p + rng.normal(0, 0.1, shape), 0, 1).astype(np.float32)
        got = _core._metrics(p, q)["ssim"]
        want = _ssim_brute(p, q)
        assert abs(got - want) < 2e-5, (shape, got, want)
        assert abs(_ssim_brute(p, q, pad="zero") - want) > 1e-3  # the padding matters here
    with pytest.raises(Exception):
        _core._metrics(a, a[:8])


@pytest.mark.parametrize("scale_env", [None, "5"])
def test_nerfstudio_face_centred_transform(tmp_path, monkeypatch, scale_env):
    """MSPLAT_FACE_DISTANCE = d > 0 replaces the auto centring with the
    face-capture normalisation (load_nerfstudio.cpp:135-146,
    input_data.cpp:82-110): the origin moves to the point d in front of the
    first camera, M0 (0, 0, -d, 1), and positions (cameras and points) are
    scaled by MSPLAT_SCALE_FACTOR (10 when unset) about it; rotations are
    kept."""
    import msplat

    monkeypatch.setenv("MSPLAT_FACE_DISTANCE", "0.4")
    if scale_env is None:
        monkeypatch.delenv("MSPLAT_SCALE_FACTOR", raising=False)
    else:
        monkeypatch.setenv("MSPLAT_SCALE_FACTOR", scale_env)
    scale = 10.0 if scale_env is None else float(scale_env)
    poses = [_look_at_c2w((3 * np.cos(a), 1.0, 3 * np.sin(a))) for a in np.linspace(0, 2, 4)]
    _write_images(tmp_path / "images", 4)
    frames = [dict(file_path=f"images/frame_{i:03d}", transform_matrix=p.tolist()) for i, p in enumerate(poses)]
    (tmp_path / "transforms.json").write_text(json.dumps(dict(w=16, h=12, fl_x=20.0, fl_y=21.0, cx=8.0, cy=6.0,
                                                              frames=frames[::-1])))
    ds = msplat.Dataset(str(tmp_path))
    M0 = np.asarray(poses[0], np.float64)
    face = M0[:3, 2] * -0.4 + M0[:3, 3]
    for k in range(4):
        got = ds.camera_pose(k)
        want = np.asarray(poses[k], np.float64).copy()
        want[:3, 3] = (want[:3, 3] - face) * scale
        assert np.abs(got - want).max() < 1e-4 * scale, (k, got, want)
    # the first camera now sits d * scale from the origin, looking at it
    assert abs(np.linalg.norm(ds.camera_pose(0)[:3, 3]) - 0.4 * scale) < 1e-4 * scale
