"""Type stubs for msplat._core, the pybind11 module over the C++ trainer
(the surface of the reference package's python/msplat/_core.pyi, plus the
extensions marked below)."""
from typing import Callable, Optional, Sequence

import numpy as np
from numpy.typing import NDArray

class TrainingConfig:
    iterations: int
    sh_degree: int
    sh_degree_interval: int
    ssim_weight: float
    num_downscales: int
    resolution_schedule: int
    refine_every: int
    warmup_length: int
    reset_alpha_every: int
    densify_grad_thresh: float
    densify_size_thresh: float
    stop_screen_size_at: int
    split_screen_size: float
    keep_crs: bool
    downscale_factor: float
    output: str
    save_every: int
    bg_color: list[float]
    """[R, G, B] in [0, 1]; exactly three values (ValueError otherwise)."""

    def __init__(
        self,
        iterations: int = 30000,
        sh_degree: int = 3,
        sh_degree_interval: int = 1000,
        ssim_weight: float = 0.2,
        num_downscales: int = 2,
        resolution_schedule: int = 3000,
        refine_every: int = 100,
        warmup_length: int = 500,
        reset_alpha_every: int = 30,
        densify_grad_thresh: float = 0.0002,
        densify_size_thresh: float = 0.01,
        stop_screen_size_at: int = 4000,
        split_screen_size: float = 0.05,
        keep_crs: bool = False,
        downscale_factor: float = 1.0,
        output: str = "splat.ply",
        save_every: int = -1,
        bg_color: list[float] = ...,
    ) -> None: ...

class TrainingStats:
    @property
    def iteration(self) -> int: ...
    @property
    def splat_count(self) -> int: ...
    @property
    def ms_per_step(self) -> float: ...
    @property
    def loss(self) -> float: ...

class Dataset:
    def __init__(self, path: str, downscale_factor: float = 1.0, eval_mode: bool = False,
                 test_every: int = 8) -> None: ...
    @staticmethod
    def from_arrays(
        images: Sequence[NDArray[np.float32]],
        cam_to_world: NDArray[np.float32],
        intrinsics: NDArray[np.float32],
        points_xyz: Optional[NDArray[np.float32]] = None,
        points_rgb: Optional[NDArray[np.uint8]] = None,
        eval_mode: bool = False,
        test_every: int = 8,
    ) -> "Dataset":
        """Extension: (H, W, 3) float32 images, (N, 4, 4) poses, (N, 4)
        intrinsics fx, fy, cx, cy, optional (P, 3) point cloud."""
        ...
    @property
    def num_train(self) -> int: ...
    @property
    def num_test(self) -> int: ...
    def camera_pose(self, index: int) -> NDArray[np.float32]: ...

class GaussianTrainer:
    def __init__(self, dataset: Dataset, config: TrainingConfig, primitive: str = "2dgs") -> None:
        """primitive (extension): "2dgs" surfels (the reference's trainer)
        or "3dgs" 3D Gaussians."""
        ...
    @property
    def primitive(self) -> str: ...
    def step(self) -> TrainingStats: ...
    def train(self, callback: Optional[Callable[[TrainingStats], object]] = None,
              callback_every: int = 100) -> None: ...
    def evaluate(self) -> dict[str, float]: ...
    def render(self, cam_idx: int, use_test: bool = False) -> NDArray[np.float32]: ...
    def render_from_pose(self, cam_to_world: NDArray[np.float32], ref_cam_idx: int = 0) -> NDArray[np.float32]: ...
    def export_ply(self, path: str) -> None: ...
    def export_splat(self, path: str) -> None: ...
    def extract_mesh(self, path: str, voxel_size: float = 0.004, bound_radius: float = 0.3,
                     alpha_thresh: float = 0.5, trunc_multiplier: float = 4.0) -> int: ...
    def export_point_cloud(self, path: str, alpha_thresh: float = 0.5) -> int: ...
    def save_checkpoint(self, path: str) -> None: ...
    def load_checkpoint(self, path: str) -> None: ...
    def load_ply(self, path: str) -> int: ...
    def set_max_splats(self, max_splats: int) -> None: ...
    def set_cull_alpha(self, thresh: float) -> None: ...
    @property
    def splat_count(self) -> int: ...
    @property
    def iteration(self) -> int: ...

def sync() -> None: ...
def cleanup() -> None: ...
