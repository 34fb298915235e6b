"""Builds libmsplat_hip.so (HIP kernels for gfx950 + the C-ABI engine + the
C++ host layer) in-tree, next to the Python package that loads it.

    python msplat-ios_amd/build.py        # or __graft_entry__.build()

Every translation unit is compiled with -ffp-contract=off (multiply-adds are
explicit fmaf calls, the arithmetic contract of the kernels) and with packed
FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "msplat"
LIB = OUT_DIR / "libmsplat_hip.so"
BUILD_DIR = REPO / "_build" / "msplat_hip"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    f"-I{REPO / 'include'}", f"-I{CSRC}", f"-I{CSRC / 'host'}",
    "-Wall", "-Wno-unused-result",
]
DEVICE = [
    f"--offload-arch={ARCH}", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file device flags.  The rasterizers claim blend-log chunks with a
# one-lane atomic whose result is used only once the chunk is full; the
# atomic optimizer rewrites such an atomic into a wave reduction whose
# result is broadcast at once, which waits for the atomic right where it is
# issued.
FILE_FLAGS = {
    "k_raster.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
    "k_raster3d.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def sources() -> list[Path]:
    srcs = sorted(CSRC.glob("*.hip"))
    srcs += sorted((CSRC / "host").glob("*.cpp"))
    return srcs


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD_DIR / (src.stem + (".hip.o" if src.suffix == ".hip" else ".cpp.o"))
    if src.suffix == ".hip":
        cmd = [HIPCC, *DEVICE, *FILE_FLAGS.get(src.name, []), *COMMON, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON, "-fopenmp", "-x", "c++", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, log in ex.map(_compile, srcs):
            objs.append(obj)
            if verbose and log.strip():
                print(log, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    # --no-undefined: a missing host symbol fails here, not at load time
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           "-fopenmp", "-lz", "-lpthread", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_core()
    return LIB


def build_core() -> Path:
    """The msplat._core Python extension (pybind11) over the C++ trainer
    API, linked against libmsplat_hip.so next to it."""
    import sysconfig

    import pybind11

    out = OUT_DIR / ("_core" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [HIPCC, "-x", "c++", *COMMON, "-fvisibility=hidden", f"-I{pybind11.get_include()}",
           f"-I{sysconfig.get_paths()['include']}", "-shared", "-o", str(tmp),
           str(CSRC / "python" / "core_module.cpp"), f"-L{OUT_DIR}", "-lmsplat_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"_core build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
