"""The C-ABI boundary, checked on the CPU: the library loads, exports every
entry point its headers declare, and the host-side camera set-up equals the
golden model's (no GPU compute is invoked here)."""
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
LIB = REPO / "msplat-ios_amd" / "msplat" / "libmsplat_hip.so"


def _declared(header: Path) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)  # header-only helpers
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(msplat_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def _exported() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


@pytest.mark.parametrize("header", sorted((REPO / "include").glob("*.h")), ids=lambda p: p.name)
def test_library_exports_every_declared_symbol(header):
    assert LIB.exists(), "build the library first (python msplat-ios_amd/build.py)"
    declared = _declared(header)
    assert declared, header
    missing = [n for n in declared if n not in _exported()]
    assert not missing, f"{header.name}: not exported: {missing}"


def test_python_binding_covers_engine_header():
    from msplat import _engine as E
    assert sorted(E.EXPORTS) == _declared(REPO / "include" / "msplat_engine.h")
    E.lib()  # binds every signature


def test_prepare_camera_matches_oracle(orc):
    from msplat import _engine as E
    from msplat import synthetic as S
    cams = S.orbit_cameras(8, 4.0, 20.0, 1297, 840) + S.make_scene(1, n=8).cameras
    for c in cams:
        o = orc.prepare_cam(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height)
        g = E.prepare_camera(c.cam_to_world, c.fx, c.fy, c.cx, c.cy, c.width, c.height, 3, 2)
        assert np.array_equal(np.array(g.viewmat), np.array(o.viewmat))
        assert np.array_equal(np.array(g.projmat), np.array(o.projmat))
        assert np.array_equal(np.array(g.cam_pos), np.array(o.cam_pos))
        assert (g.tiles_x, g.tiles_y) == (o.tiles_x, o.tiles_y)
        assert (g.degree, g.degrees_to_use, g.glob_scale, g.clip_thresh) == (3, 2, 1.0, np.float32(0.01))


def test_prepare_camera_rejects_bad_sizes():
    from msplat import _engine as E
    with pytest.raises(E.MsplatError):
        E.prepare_camera(np.eye(4), 100.0, 100.0, 50.0, 50.0, 0, 10)


def test_ctypes_binding_covers_c_api_header():
    """msplat.capi binds every function of the public C ABI."""
    import re as _re

    from msplat import capi
    src = (REPO / "msplat-ios_amd" / "msplat" / "capi.py").read_text()
    bound = set(_re.findall(r'"(msplat_\w+)":', src))
    assert sorted(bound) == _declared(REPO / "include" / "msplat_c_api.h")
    capi.lib()  # every signature binds
