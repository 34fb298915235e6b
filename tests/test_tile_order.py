"""The rasterizers' XCD-aware workgroup -> tile order is a bijection (CPU).

k_raster_fwd and k_raster_bwd run xcd_strip_grid(tx, ty) workgroups and
map each to a tile with xcd_strip_tile (XCD bands walked in column
strips), padding workgroups exiting at once.  Every tile must be rendered
exactly once, for grid shapes that are not multiples of the strip width or
of the 8 XCDs, down to a single tile.  tests/native/libquadmask.so compiles
the product header for the host.
"""
import ctypes as C
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent / "native" / "libquadmask.so"


@pytest.mark.parametrize("tx,ty", [(1, 1), (3, 2), (8, 8), (16, 16), (17, 9), (82, 53), (325, 211), (7, 100),
                                   (100, 7), (9, 15)])
def test_tile_order_is_a_bijection(tx, ty):
    if not LIB.exists():
        pytest.fail(f"{LIB} is missing: build it with `make -C tests/native` (build() does)")
    L = C.CDLL(str(LIB))
    L.tile_order_check.restype = C.c_int64
    L.tile_order_check.argtypes = [C.c_int, C.c_int]
    assert L.tile_order_check(tx, ty) == 0
