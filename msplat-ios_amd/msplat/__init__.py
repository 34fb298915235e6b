"""msplat on MI355X: the 2DGS Gaussian-splatting training step as hand-written
gfx950 HIP kernels behind msplat's C ABI.

The public surface mirrors the reference package (python/msplat/__init__.py):
TrainingConfig, TrainingStats, Dataset, GaussianTrainer, load_dataset, sync,
cleanup.  Lower-level access to the engine lives in msplat._engine and
msplat.device.
"""
from . import _engine, synthetic
from ._engine import MsplatError, cleanup, sync

__all__ = ["MsplatError", "cleanup", "sync", "synthetic", "_engine"]
