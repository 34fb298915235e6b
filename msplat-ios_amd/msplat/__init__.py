"""msplat on MI355X: 2D Gaussian Splatting training with hand-written gfx950
HIP kernels.

The public surface is the reference package's (python/msplat/__init__.py):
TrainingConfig, TrainingStats, Dataset, GaussianTrainer, sync, cleanup and
load_dataset, implemented by the compiled msplat._core module over the C++
trainer.  Dataset.from_arrays builds a dataset from in-memory images.
Lower-level access to the engine's C ABI lives in msplat._engine and
msplat.device; msplat.synthetic generates seeded test scenes.
"""
import atexit

from msplat._core import (
    Dataset,
    GaussianTrainer,
    TrainingConfig,
    TrainingStats,
    sync,
)
from msplat._core import cleanup as _cleanup_raw

from . import _engine, synthetic
from ._engine import MsplatError

_cleaned_up = False


def cleanup():
    """Frees the engine's device buffers, streams and pinned staging memory;
    later calls do nothing (it also runs at interpreter exit)."""
    global _cleaned_up
    if not _cleaned_up:
        _cleaned_up = True
        _cleanup_raw()


atexit.register(cleanup)

__all__ = [
    "TrainingConfig",
    "TrainingStats",
    "Dataset",
    "GaussianTrainer",
    "sync",
    "cleanup",
    "load_dataset",
    "MsplatError",
    "synthetic",
]

__version__ = "1.1.3"


def load_dataset(path: str, downscale_factor: float = 1.0, eval_mode: bool = False, test_every: int = 8) -> Dataset:
    """A Dataset from a capture directory, its format (COLMAP, Nerfstudio or
    Polycam) detected from the files present; images are box-downscaled by
    downscale_factor, and with eval_mode every test_every-th image is held
    out."""
    return Dataset(path, downscale_factor, eval_mode, test_every)
