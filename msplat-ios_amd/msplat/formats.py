"""The .msplat checkpoint layout (core/src/model.cpp:343-498), readable and
writable from numpy: what Model::saveCheckpoint writes and
Model::loadCheckpoint reads, so scenes built on the host (e.g. the
synthetic benchmark workloads) can be loaded into a Trainer.

Layout, little-endian:
  u32 magic 0x4C50534D ("MSPL"), u32 version 1,
  u32 step, u32 num_active, u32 shDegree, u32 adam_step_count,
  f32 adam_lr[6], f32 means_lr_init, f32 means_lr_final,
  18 tensors (means, scales, quats, features_dc, features_rest, opacities,
  then the six first moments, then the six second moments), each
  u32 ndim, i64 shape[ndim], u64 nbytes, raw float32 data.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

MAGIC = 0x4C50534D
VERSION = 1
GROUPS = ("means", "scales", "quats", "features_dc", "features_rest", "opacities")
# Model's learning-rate table (core/src/model.cpp:142), in GROUPS order
DEFAULT_LR = (0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05)


def _write_tensor(f, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a, np.float32)
    f.write(struct.pack("<I", a.ndim))
    f.write(struct.pack(f"<{a.ndim}q", *a.shape))
    f.write(struct.pack("<Q", a.nbytes))
    f.write(a.tobytes())


def _read_tensor(f) -> np.ndarray:
    (nd,) = struct.unpack("<I", f.read(4))
    if nd == 0 or nd > 8:
        raise ValueError("checkpoint: corrupt tensor header")
    shape = struct.unpack(f"<{nd}q", f.read(8 * nd))
    (nbytes,) = struct.unpack("<Q", f.read(8))
    if nbytes != 4 * int(np.prod(shape, dtype=np.int64)):
        raise ValueError("checkpoint: tensor size mismatch")
    return np.frombuffer(f.read(nbytes), np.float32).reshape(shape).copy()


def write_checkpoint(path, params: dict, sh_degree: int, step: int = 0, adam_step: int = 0,
                     adam_lr=DEFAULT_LR, means_lr=(0.00016, 0.0000016), exp_avg=None, exp_avg_sq=None) -> None:
    """params: the six groups by name (features_rest as [N,K,3], opacities
    as [N,1]); Adam moments default to zeros."""
    p = [np.ascontiguousarray(params[k], np.float32) for k in GROUPS]
    n = p[0].shape[0]
    m = exp_avg or [np.zeros_like(a) for a in p]
    v = exp_avg_sq or [np.zeros_like(a) for a in p]
    with open(path, "wb") as f:
        f.write(struct.pack("<II", MAGIC, VERSION))
        f.write(struct.pack("<4I", step, n, sh_degree, adam_step))
        f.write(struct.pack("<6f", *adam_lr))
        f.write(struct.pack("<2f", *means_lr))
        for a in p + list(m) + list(v):
            _write_tensor(f, a)


def read_checkpoint(path) -> dict:
    with open(Path(path), "rb") as f:
        magic, version = struct.unpack("<II", f.read(8))
        if magic != MAGIC:
            raise ValueError("Not a valid msplat checkpoint file")
        if version != VERSION:
            raise ValueError(f"Unsupported checkpoint version: {version}")
        step, n, sh, adam_step = struct.unpack("<4I", f.read(16))
        lr = struct.unpack("<6f", f.read(24))
        lr0, lr1 = struct.unpack("<2f", f.read(8))
        t = [_read_tensor(f) for _ in range(18)]
    return dict(step=step, num_active=n, sh_degree=sh, adam_step=adam_step, adam_lr=lr, means_lr=(lr0, lr1),
                params=dict(zip(GROUPS, t[:6])), exp_avg=t[6:12], exp_avg_sq=t[12:18])
