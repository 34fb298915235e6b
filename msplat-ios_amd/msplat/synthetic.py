"""Seeded synthetic scenes and cameras for the five benchmark workloads.

All randomness comes from a SplitMix64 stream (seed 0xC0FFEE + workload
index) with Box-Muller normals, so the same arrays are produced on any host
and fed to both the HIP engine and the CPU golden model.

Workloads (2DGS: two log-scales per splat):
  1  forward only: 16,384 splats, means U[-1,1]^3, log-scales N(-4,0.5),
     SH degree 0 with colours U(0,1); camera 3 units from the origin,
     256x256, fx=fy=256.
  2  train step: 500k splats from 64 isotropic blobs (sigma 0.3) in [-2,2]^3,
     SH degree 3 (DC U(0,1), higher bands N(0,0.05)), log-scales N(-4,0.5),
     1297x840, 32 cameras on a radius-4 orbit at 20 degrees elevation.
  3  the same at 3M splats, log-scales N(-5,0.7), 5187x3361.
  4  overflow stress: 1M splats, 40% in a 0.1-radius ball on the optical
     axis, 60% U[-2,2]^3, 1920x1080.
  5  densification: 200k blob splats, 1297x840.
Targets are renders of the same scene with means jittered by N(0, 0.01).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SH_C0 = 0.28209479177387814
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
DEFAULT_BG = np.array([0.6130, 0.0101, 0.3984], np.float32)  # msplat_api.hpp:32


class SplitMix64:
    def __init__(self, seed: int):
        self._state = np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)

    def u64(self, n: int) -> np.ndarray:
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = self._state + idx * GOLDEN
        self._state = self._state + np.array([n], dtype=np.uint64) * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))

    def uniform(self, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
        u = (self.u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        return lo + (hi - lo) * u

    def normal(self, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        m = (n + 1) // 2
        u1 = 1.0 - self.uniform(m)
        u2 = self.uniform(m)
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * m)
        z[0::2] = r * np.cos(2.0 * np.pi * u2)
        z[1::2] = r * np.sin(2.0 * np.pi * u2)
        return mean + std * z[:n]


@dataclass
class Camera:
    cam_to_world: np.ndarray  # 4x4 row-major, OpenGL convention (-Z forward)
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int


@dataclass
class Scene:
    means: np.ndarray
    scales: np.ndarray
    quats: np.ndarray
    opacities: np.ndarray
    features_dc: np.ndarray
    features_rest: np.ndarray
    sh_degree: int
    cameras: list[Camera] = field(default_factory=list)
    background: np.ndarray = field(default_factory=lambda: DEFAULT_BG.copy())
    name: str = ""

    @property
    def n(self) -> int:
        return int(self.means.shape[0])

    def params(self) -> list[np.ndarray]:
        return [self.means, self.scales, self.quats, self.features_dc, self.features_rest, self.opacities]

    def jittered(self, std: float, seed: int) -> "Scene":
        rng = SplitMix64(seed)
        means = (self.means + rng.normal(self.means.size, 0.0, std).reshape(self.means.shape)).astype(np.float32)
        return Scene(means, self.scales, self.quats, self.opacities, self.features_dc, self.features_rest,
                     self.sh_degree, self.cameras, self.background, self.name + "+jitter")


def look_at(position, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)) -> np.ndarray:
    """Camera-to-world (OpenGL: x right, y up, -z forward), row-major 4x4."""
    c = np.asarray(position, np.float64)
    f = np.asarray(target, np.float64) - c
    f /= np.linalg.norm(f)
    r = np.cross(f, np.asarray(up, np.float64))
    r /= np.linalg.norm(r)
    u = np.cross(r, f)
    m = np.eye(4)
    m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = r, u, -f, c
    return m.astype(np.float32)


def orbit_cameras(count: int, radius: float, elevation_deg: float, width: int, height: int,
                  fx: float | None = None) -> list[Camera]:
    el = np.deg2rad(elevation_deg)
    fx = float(width) if fx is None else fx
    cams = []
    for k in range(count):
        az = 2.0 * np.pi * k / count
        pos = radius * np.array([np.cos(el) * np.cos(az), np.sin(el), np.cos(el) * np.sin(az)])
        cams.append(Camera(look_at(pos), fx, fx, width / 2.0, height / 2.0, width, height))
    return cams


def _quats(rng: SplitMix64, n: int) -> np.ndarray:
    q = rng.normal(4 * n).reshape(n, 4)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def _blob_means(rng: SplitMix64, n: int, blobs: int = 64, sigma: float = 0.3) -> np.ndarray:
    centres = rng.uniform(3 * blobs, -2.0, 2.0).reshape(blobs, 3)
    which = np.minimum((rng.uniform(n) * blobs).astype(np.int64), blobs - 1)
    return (centres[which] + rng.normal(3 * n, 0.0, sigma).reshape(n, 3)).astype(np.float32)


def _sh(rng: SplitMix64, n: int, degree: int, dc_from_rgb: bool) -> tuple[np.ndarray, np.ndarray]:
    nb = (degree + 1) ** 2
    if dc_from_rgb:
        fdc = ((rng.uniform(3 * n) - 0.5) / SH_C0).reshape(n, 3)
    else:
        fdc = rng.uniform(3 * n).reshape(n, 3)
    frest = rng.normal(3 * n * (nb - 1), 0.0, 0.05).reshape(n, nb - 1, 3)
    return fdc.astype(np.float32), frest.astype(np.float32)


def make_scene(workload: int, n: int | None = None, width: int | None = None, height: int | None = None,
               seed: int | None = None, num_cameras: int | None = None) -> Scene:
    """Builds workload 1..5; n / width / height shrink it for parity tests."""
    seed = 0xC0FFEE + workload if seed is None else seed
    rng = SplitMix64(seed)
    if workload == 1:
        n = 16384 if n is None else n
        W = 256 if width is None else width
        H = 256 if height is None else height
        means = rng.uniform(3 * n, -1.0, 1.0).reshape(n, 3).astype(np.float32)
        scales = rng.normal(2 * n, -4.0, 0.5).reshape(n, 2).astype(np.float32)
        quats = _quats(rng, n)
        opac = rng.normal(n).reshape(n, 1).astype(np.float32)
        fdc, frest = _sh(rng, n, 0, dc_from_rgb=True)
        f = 256.0 * W / 256.0
        cams = [Camera(look_at((0.0, 0.0, 3.0)), f, f, W / 2.0, H / 2.0, W, H)]
        return Scene(means, scales, quats, opac, fdc, frest, 0, cams, name="forward-16k-256")
    if workload in (2, 3, 5):
        defaults = {2: (500_000, 1297, 840, -4.0, 0.5), 3: (3_000_000, 5187, 3361, -5.0, 0.7),
                    5: (200_000, 1297, 840, -4.0, 0.5)}[workload]
        n = defaults[0] if n is None else n
        W = defaults[1] if width is None else width
        H = defaults[2] if height is None else height
        means = _blob_means(rng, n)
        scales = rng.normal(2 * n, defaults[3], defaults[4]).reshape(n, 2).astype(np.float32)
        quats = _quats(rng, n)
        opac = rng.normal(n).reshape(n, 1).astype(np.float32)
        fdc, frest = _sh(rng, n, 3, dc_from_rgb=False)
        cams = orbit_cameras(32 if num_cameras is None else num_cameras, 4.0, 20.0, W, H)
        name = {2: "train-500k-1297x840", 3: "train-3M-5187x3361", 5: "densify-200k-1297x840"}[workload]
        return Scene(means, scales, quats, opac, fdc, frest, 3, cams, name=name)
    if workload == 4:
        n = 1_000_000 if n is None else n
        W = 1920 if width is None else width
        H = 1080 if height is None else height
        nb = int(0.4 * n)
        d = rng.normal(3 * nb).reshape(nb, 3)
        d /= np.linalg.norm(d, axis=1, keepdims=True)
        r = 0.1 * np.cbrt(rng.uniform(nb))[:, None]
        ball = d * r
        rest = rng.uniform(3 * (n - nb), -2.0, 2.0).reshape(n - nb, 3)
        means = np.concatenate([ball, rest]).astype(np.float32)
        scales = rng.normal(2 * n, -4.5, 0.5).reshape(n, 2).astype(np.float32)
        quats = _quats(rng, n)
        opac = rng.normal(n).reshape(n, 1).astype(np.float32)
        fdc, frest = _sh(rng, n, 3, dc_from_rgb=False)
        cams = orbit_cameras(32 if num_cameras is None else num_cameras, 4.0, 20.0, W, H)
        return Scene(means, scales, quats, opac, fdc, frest, 3, cams, name="overflow-1M-1920x1080")
    raise ValueError(f"unknown workload {workload}")
