"""Writes the JPEG decoder's fixtures: small synthetic images encoded by PIL
(libjpeg) in the variants capture pipelines produce, each with the pixels
PIL decodes from it (its default decoding: accurate integer IDCT, smooth
2:1 chroma upsampling, JFIF YCbCr -> RGB).

    python tests/golden/make_jpeg_fixtures.py

Output: tests/golden/jpeg/<name>.jpg and jpeg_expected.npz (uint8 [H,W,3]
per name).  Run once; the fixtures are committed.
"""
from pathlib import Path

import numpy as np
from PIL import Image

OUT = Path(__file__).resolve().parent / "jpeg"


def pattern(w, h, seed):
    """Smooth colour gradients, sharp edges and noise, so every coding path
    (DC, many AC terms, long zero runs) occurs."""
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:h, 0:w].astype(np.float64)
    r = 128 + 100 * np.sin(x / 7.0) * np.cos(y / 9.0)
    g = 255 * (x / max(w - 1, 1))
    b = 255 * ((x // 8 + y // 8) % 2)
    img = np.stack([r, g, b], -1) + rng.normal(0, 12, (h, w, 3))
    img[h // 3: h // 2, :, :] = [250, 20, 40]
    return np.clip(img, 0, 255).astype(np.uint8)


CASES = {
    "base420": dict(size=(64, 48), quality=90, subsampling=2),
    "base422": dict(size=(37, 29), quality=85, subsampling=1),
    "base444": dict(size=(33, 17), quality=95, subsampling=0),
    "base420_odd": dict(size=(45, 31), quality=75, subsampling=2),
    "grey": dict(size=(29, 23), quality=90, mode="L"),
    "prog420": dict(size=(64, 48), quality=90, subsampling=2, progressive=True),
    "prog444": dict(size=(40, 24), quality=80, subsampling=0, progressive=True),
    "prog_grey": dict(size=(31, 19), quality=85, mode="L", progressive=True),
    "restart420": dict(size=(56, 40), quality=88, subsampling=2, restart_marker_blocks=3),
    "prog_restart": dict(size=(48, 40), quality=88, subsampling=2, progressive=True, restart_marker_blocks=2),
    "optimized": dict(size=(50, 34), quality=70, subsampling=2, optimize=True),
    "lowq": dict(size=(40, 40), quality=20, subsampling=2),
}


def main():
    OUT.mkdir(parents=True, exist_ok=True)
    expected = {}
    for i, (name, kw) in enumerate(CASES.items()):
        kw = dict(kw)
        w, h = kw.pop("size")
        mode = kw.pop("mode", "RGB")
        img = Image.fromarray(pattern(w, h, i))
        if mode == "L":
            img = img.convert("L")
        path = OUT / f"{name}.jpg"
        img.save(path, "JPEG", **kw)
        expected[name] = np.asarray(Image.open(path).convert("RGB"), np.uint8)
    np.savez_compressed(OUT / "jpeg_expected.npz", **expected)
    print("wrote", len(CASES), "fixtures to", OUT)


if __name__ == "__main__":
    main()
