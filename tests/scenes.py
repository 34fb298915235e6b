"""Synthetic scenes shared by the tests."""
import numpy as np

from msplat import synthetic as S


def adversarial(n, seed, width=160, height=112):
    """Splats built to stress the ellipse test: random orientations with one
    axis squashed by up to 1e4 (edge-on and needle-like), scales spanning
    seven decades, opacities from barely visible to saturated, centres
    spread beyond the image and towards the camera."""
    scene = S.make_scene(1, n=n, width=width, height=height, seed=seed)
    rng = np.random.default_rng(seed)
    scene.means[:] = rng.uniform(-2.5, 2.5, (n, 3)).astype(np.float32)
    scene.means[: n // 8, 2] = rng.uniform(1.5, 2.9, n // 8).astype(np.float32)  # near the camera at z = 3
    s = rng.uniform(-7.0, 0.5, (n, 2)).astype(np.float32)
    s[:, 1] = s[:, 0] - rng.uniform(0.0, 9.0, n).astype(np.float32)  # anisotropy up to e^9
    scene.scales[:] = s
    q = rng.normal(size=(n, 4)).astype(np.float32)
    q[: n // 4] = np.float32([0.7071, 0.7071, 0.0, 0.0]) + 1e-3 * q[: n // 4]  # plane nearly edge-on
    scene.quats[:] = q
    scene.opacities[:] = rng.uniform(-6.0, 8.0, (n, 1)).astype(np.float32)
    return scene
