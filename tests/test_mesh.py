"""Mesh extraction: TSDF fusion (msplat_metal.metal:2223-2280), marching
cubes (:2606-2687) and the depth unprojection of Model::exportPointCloud
(model.cpp:565-640).

The oracle is pinned by closed forms: a sphere and a tilted plane through
marching cubes (surface area, enclosed volume, distance of every vertex to
the surface, Euler characteristic, winding), watertightness on random
fields, the sign-change structure of the case table, the TSDF of planar
depth maps (truncated signed distance and the weighted mean of two views),
and the unprojection of a planar depth map.  The GPU path is compared with
the oracle bit for bit, then checked end to end on a rendered sphere of
surfels.  The case table is this build's own (generated from the corner
signs); the reference's triangulation is not reproduced, only its vertex
placement, winding and skip rules.
"""
import math

import numpy as np
import pytest

EDGES = [(0, 1), (1, 2), (2, 3), (3, 0), (4, 5), (5, 6), (6, 7), (7, 4), (0, 4), (1, 5), (2, 6), (3, 7)]
CORNERS = [(0, 0, 0), (1, 0, 0), (1, 1, 0), (0, 1, 0), (0, 0, 1), (1, 0, 1), (1, 1, 1), (0, 1, 1)]


@pytest.fixture(scope="module")
def table():
    from msplat import _engine as E
    return E.mc_table()


def _grid(sdf, weight=None):
    g = np.zeros(sdf.shape + (2,), np.float32)
    g[..., 0] = sdf
    g[..., 1] = 1.0 if weight is None else weight
    return g


def _edge_keys(tris):
    """Grid-edge id of every vertex of a unit-voxel, origin -0.5 grid (so
    voxel centres sit on integers): two coordinates are integers, the third
    lies strictly between two."""
    v = tris.reshape(-1, 3).astype(np.float64)
    fl = np.floor(v)
    frac = v - fl
    axis = np.argmax(frac, axis=1)
    assert np.all(np.sum(frac > 0, axis=1) == 1), "a vertex off the grid edges"
    return [(int(a), int(x), int(y), int(z)) for a, (x, y, z) in zip(axis, fl)]


# ---------------------------------------------------------------- table ----
def test_case_table_follows_the_corner_signs(table):
    """Every triangle joins crossings of sign-changing edges, every
    sign-changing edge is used, at most 5 triangles, none degenerate."""
    for m in range(256):
        inside = [(m >> c) & 1 for c in range(8)]
        crossed = {e for e, (a, b) in enumerate(EDGES) if inside[a] != inside[b]}
        row = [int(x) for x in table[m]]
        n = 0
        while n < 16 and row[n] >= 0:
            n += 1
        assert n % 3 == 0 and n <= 15 and all(x == -1 for x in row[n:]), m
        tris = [row[i:i + 3] for i in range(0, n, 3)]
        used = {e for t in tris for e in t}
        assert used == crossed, m
        assert all(len(set(t)) == 3 for t in tris), m
    assert not (table[0] >= 0).any() and not (table[255] >= 0).any()


def test_case_one_matches_the_reference_triangle(table):
    """Corner 0 inside: the triangle of edges 0, 8, 3 (the reference
    table's first row, in any rotation), normal towards the corner."""
    row = [int(x) for x in table[1][:3]]
    assert row in ([0, 8, 3], [8, 3, 0], [3, 0, 8])


@pytest.mark.parametrize("seed", range(6))
def test_random_fields_give_closed_oriented_surfaces(orc, table, seed):
    """Random corner values, positive on the boundary: after welding by grid
    edge, every directed triangle edge is matched by exactly one reverse
    edge (closed, manifold, consistently wound)."""
    rng = np.random.default_rng(seed)
    D = 14
    f = rng.normal(size=(D, D, D)).astype(np.float32)
    f[[0, -1], :, :] = 1
    f[:, [0, -1], :] = 1
    f[:, :, [0, -1]] = 1
    tris, total = orc.marching_cubes(_grid(f), [-0.5, -0.5, -0.5], 1.0, table)
    assert total == len(tris) > 100
    keys = _edge_keys(tris)
    ids = {k: i for i, k in enumerate(sorted(set(keys)))}
    t = np.array([ids[k] for k in keys]).reshape(-1, 3)
    directed = {}
    for a, b, c in t:
        for e in ((a, b), (b, c), (c, a)):
            directed[e] = directed.get(e, 0) + 1
    assert all(cnt == 1 for cnt in directed.values())
    assert all(directed.get((b, a), 0) == 1 for (a, b) in directed)


# ---------------------------------------------------------- closed forms ----
def _sphere_grid(D, c, r):
    z, y, x = np.meshgrid(*[np.arange(D, dtype=np.float64)] * 3, indexing="ij")
    return np.sqrt((x - c[0]) ** 2 + (y - c[1]) ** 2 + (z - c[2]) ** 2) - r


def _area_volume(tris):
    t = tris.astype(np.float64)
    cr = np.cross(t[:, 1] - t[:, 0], t[:, 2] - t[:, 0])
    area = 0.5 * np.linalg.norm(cr, axis=1).sum()
    vol = np.einsum("ij,ij->i", t[:, 0], np.cross(t[:, 1], t[:, 2])).sum() / 6.0
    return area, vol, cr


def test_sphere_area_volume_distance_topology_and_winding(orc, table):
    D, c, r = 34, np.array([16.23, 15.71, 16.38]), 10.31
    sdf = _sphere_grid(D, c, r)
    assert (sdf != 0).all()  # a zero corner puts a vertex on a grid point (degenerate triangles)
    tris, total = orc.marching_cubes(_grid(sdf), [-0.5, -0.5, -0.5], 1.0, table)
    assert total == len(tris)
    area, vol, cr = _area_volume(tris - c)
    # piecewise-linear interpolation of a smooth surface at unit voxels
    assert abs(area / (4 * math.pi * r * r) - 1) < 0.01
    # the winding puts the right-hand normal towards negative SDF (the
    # inside), so the signed volume is negative
    assert abs(-vol / (4 / 3 * math.pi * r ** 3) - 1) < 0.01
    cen = tris.astype(np.float64).mean(axis=1) - c
    assert np.all(np.einsum("ij,ij->i", cr, cen) < 0)
    d = np.linalg.norm(tris.reshape(-1, 3).astype(np.float64) - c, axis=1)
    assert np.abs(d - r).max() < 0.05
    # one closed genus-0 surface: V - E + F = 2 after welding
    keys = _edge_keys(tris)
    V = len(set(keys))
    ids = {k: i for i, k in enumerate(sorted(set(keys)))}
    t = np.array([ids[k] for k in keys]).reshape(-1, 3)
    E = len({tuple(sorted(e)) for a, b, cc in t for e in ((a, b), (b, cc), (cc, a))})
    assert V - E + len(t) == 2


def test_tilted_plane_is_exact(orc, table):
    """A linear field is interpolated exactly: every vertex lies on the
    plane, and the surface is the rectangle the plane cuts from the box of
    voxel centres."""
    D = 20
    th = 0.3
    n = np.array([math.sin(th), 0.0, math.cos(th)])
    dd = 9.7
    z, y, x = np.meshgrid(*[np.arange(D, dtype=np.float64)] * 3, indexing="ij")
    sdf = n[0] * x + n[2] * z - dd
    tris, _ = orc.marching_cubes(_grid(sdf), [0.0, 0.0, 0.0], 1.0, table)
    v = tris.reshape(-1, 3).astype(np.float64) - 0.5  # back to voxel-index coordinates
    assert np.abs(v @ n - dd).max() < 2e-5
    area, _, cr = _area_volume(tris)
    # x spans [0, D-1], y spans [0, D-1]; the plane stays inside z in [0, D-1]
    assert abs(area - (D - 1) * (D - 1) / math.cos(th)) < 1e-3
    # normals point towards -n (negative SDF)
    assert np.all(cr @ n < 0)


def test_unobserved_voxels_suppress_their_cells(orc, table):
    D = 16
    sdf = _sphere_grid(D, np.array([7.3, 7.6, 7.1]), 5.2)
    w = np.ones_like(sdf)
    w[7, 2, 7] = 0.0  # a voxel next to the surface (z, y, x)
    full, _ = orc.marching_cubes(_grid(sdf), [0, 0, 0], 1.0, table)
    cut, _ = orc.marching_cubes(_grid(sdf, w), [0, 0, 0], 1.0, table)
    assert 0 < len(cut) < len(full)
    # no triangle of the cut mesh touches the 8 cells around voxel (7, 2, 7)
    cen = cut.astype(np.float64).mean(axis=1) - 0.5  # voxel-index coordinates (x, y, z)
    inside = np.all(np.abs(cen - np.array([7, 2, 7])) < 1.0, axis=1)
    assert not inside.any()
    full_cen = full.astype(np.float64).mean(axis=1) - 0.5
    near = np.all(np.abs(full_cen - np.array([7, 2, 7])) < 1.0, axis=1)
    assert near.sum() == len(full) - len(cut)


def test_triangle_cap_keeps_the_first_triangles(orc, table):
    sdf = _sphere_grid(12, np.array([5.5, 5.2, 5.7]), 3.9)
    tris, total = orc.marching_cubes(_grid(sdf), [0, 0, 0], 1.0, table)
    part, total2 = orc.marching_cubes(_grid(sdf), [0, 0, 0], 1.0, table, max_triangles=17)
    assert total2 == total and len(part) == 17 and np.array_equal(part, tris[:17])


def _look_at_identity_view():
    """World = OpenCV camera frame (viewmat identity)."""
    return np.eye(4, dtype=np.float32)


def test_tsdf_of_two_planar_views_is_the_weighted_mean(orc):
    """A wide camera at the origin looking down +z sees every voxel; depth
    maps of constant depth D1, D2 with alphas a1, a2 give the truncated
    signed distances clamp(D - z) averaged with weights a."""
    dz, dy, dx = 12, 10, 9
    origin = np.array([-0.45, -0.5, 1.0], np.float32)
    vs = 0.1
    trunc = 0.25
    W = H = 64
    f = 20.0
    grid = np.zeros((dz, dy, dx, 2), np.float32)
    views = [(1.43, 0.8), (1.72, 0.3)]  # no voxel sits at exactly -trunc
    for D, a in views:
        orc.tsdf_integrate(grid, origin, vs, _look_at_identity_view(), f, f, W / 2, H / 2,
                           np.full((H, W), D, np.float32), np.full((H, W), a, np.float32), trunc, 0.2)
    z = origin[2] + (np.arange(dz) + 0.5) * vs
    num = np.zeros(dz)
    den = np.zeros(dz)
    for D, a in views:
        s = D - z
        ok = s >= -trunc
        num += np.where(ok, np.clip(s, -trunc, trunc) * a, 0)
        den += np.where(ok, a, 0)
    exp_w = den
    exp_s = np.where(den > 0, num / np.where(den > 0, den, 1), 0)
    assert np.allclose(grid[..., 1], exp_w[:, None, None], atol=1e-6)
    assert np.allclose(grid[..., 0], exp_s[:, None, None], atol=2e-6)
    # the views see every voxel: each slice is uniform
    assert np.ptp(grid[..., 0], axis=(1, 2)).max() == 0


def test_tsdf_skips(orc):
    """Behind the camera, outside the image, alpha below the threshold,
    non-finite or non-positive depth, and far behind the surface: no
    update."""
    grid = np.zeros((4, 4, 4, 2), np.float32)
    base = grid.copy()
    vm = _look_at_identity_view()
    W = H = 32
    args = (vm, 10.0, 10.0, 16.0, 16.0)
    # grid behind the camera (z < 0.01)
    orc.tsdf_integrate(grid, [-0.2, -0.2, -0.5], 0.1, *args, np.ones((H, W), np.float32),
                       np.ones((H, W), np.float32), 0.3, 0.5)
    assert np.array_equal(grid, base)
    for depth, alpha in [(np.ones((H, W)), np.full((H, W), 0.49)), (np.full((H, W), np.nan), np.ones((H, W))),
                         (np.full((H, W), np.inf), np.ones((H, W))), (np.zeros((H, W)), np.ones((H, W))),
                         (np.full((H, W), 0.2), np.ones((H, W)))]:  # 0.2 - z < -trunc for z in [1, 1.4]
        orc.tsdf_integrate(grid, [-0.2, -0.2, 1.0], 0.1, *args, depth.astype(np.float32),
                           alpha.astype(np.float32), 0.3, 0.5)
        assert np.array_equal(grid, base)
    # a narrow camera: voxels that project outside the image are skipped
    orc.tsdf_integrate(grid, [-2.0, -0.2, 1.0], 0.1, vm, 10.0, 10.0, 16.0, 16.0, np.ones((H, W), np.float32),
                       np.ones((H, W), np.float32), 0.3, 0.5)
    seen = grid[..., 1] > 0
    assert seen.any() and not seen.all()


def test_unprojected_plane(orc):
    """Constant depth sum D*a with alpha a: every point sits at depth D on
    the pixel-centre ray; camToWorld identity maps OpenCV (x, y, z) to
    world (x, -y, -z)."""
    W, H, f, D, a = 13, 9, 11.0, 2.5, 0.8
    cx, cy = 6.1, 4.3
    alpha = np.full((H, W), a, np.float32)
    alpha[2, 3] = 0.3  # below the threshold
    depth = (np.float32(D) * alpha).astype(np.float32)
    img = np.random.default_rng(0).uniform(-0.2, 1.2, (H, W, 3)).astype(np.float32)
    xyz, rgb = orc.unproject_depth(img, depth, alpha, f, f, cx, cy, np.eye(4, dtype=np.float32), 0.5)
    assert len(xyz) == W * H - 1
    py, px = np.nonzero(alpha >= 0.5)
    exp = np.stack([(px + 0.5 - cx) * D / f, -(py + 0.5 - cy) * D / f, -np.full(px.shape, D)], 1)
    assert np.abs(xyz - exp).max() < 1e-5
    exp_rgb = np.clip(img[py, px] * 255.0, 0, 255).astype(np.uint8)
    assert np.array_equal(rgb, exp_rgb)


# ---------------------------------------------------------------- GPU ----
def _rand_grid(rng, shape, zero_frac=0.05):
    sdf = rng.normal(size=shape).astype(np.float32)
    w = rng.uniform(0.1, 2.0, size=shape).astype(np.float32)
    w[rng.uniform(size=shape) < zero_frac] = 0.0
    return _grid(sdf, w)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(23, 29, 37), (2, 2, 2), (5, 1, 7), (17, 64, 65), (40, 33, 130)])
def test_gpu_marching_cubes_matches_oracle(orc, table, eng, shape):
    from msplat import _engine as E
    rng = np.random.default_rng(sum(shape))
    g = _rand_grid(rng, shape)
    origin, vs = [-1.3, 0.4, 2.1], 0.037
    exp, total = orc.marching_cubes(g, origin, vs, table)
    dg = E.DeviceArray.from_numpy(g)
    got, gtotal = E.marching_cubes(dg, origin, vs, total + 5)
    assert gtotal == total and np.array_equal(got, exp)
    if total > 10:
        part, ptotal = E.marching_cubes(dg, origin, vs, total // 3)
        assert ptotal == total and np.array_equal(part, exp[:total // 3])
    none, ntotal = E.marching_cubes(dg, origin, vs, 0)
    assert ntotal == total and len(none) == 0


@pytest.mark.gpu
def test_gpu_marching_cubes_sphere_closed_form(orc, table, eng):
    from msplat import _engine as E
    D, c, r = 70, np.array([33.2, 35.7, 34.4]), 27.1
    g = _grid(_sphere_grid(D, c, r))
    tris, total = E.marching_cubes(E.DeviceArray.from_numpy(g), [-0.5, -0.5, -0.5], 1.0, 1 << 20)
    assert total == len(tris)
    area, vol, _ = _area_volume(tris - c)
    assert abs(area / (4 * math.pi * r * r) - 1) < 0.005
    assert abs(-vol / (4 / 3 * math.pi * r ** 3) - 1) < 0.002
    exp, _ = orc.marching_cubes(g, [-0.5, -0.5, -0.5], 1.0, table)
    assert np.array_equal(tris, exp)


def _random_view(rng, center, H, W):
    """A camera 2-3 units from `center` looking at it (OpenCV viewmat)."""
    eye = center + rng.uniform(2.0, 3.0) * _unit(rng.normal(size=3))
    fwd = _unit(center - eye)
    right = _unit(np.cross(fwd, rng.normal(size=3)))
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd])
    vm = np.eye(4)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ eye
    return vm.astype(np.float32), float(rng.uniform(0.8, 1.2) * W), float(rng.uniform(0.8, 1.2) * W), W / 2 + 0.3, \
        H / 2 - 0.2


def _unit(v):
    return v / np.linalg.norm(v)


@pytest.mark.gpu
def test_gpu_tsdf_matches_oracle(orc, eng):
    from msplat import _engine as E
    rng = np.random.default_rng(11)
    dz, dy, dx = 31, 26, 45
    origin, vs = np.array([-0.8, -0.65, -0.75], np.float32), 0.034
    center = origin + vs * np.array([dx, dy, dz]) / 2
    g0 = _rand_grid(rng, (dz, dy, dx), zero_frac=0.3) * np.float32(0.1)
    grid = g0.copy()
    dev = E.DeviceArray.from_numpy(g0)
    views, keep = [], []
    for k in range(4):
        H, W = 61 + 7 * k, 83 - 5 * k
        vm, fx, fy, cx, cy = _random_view(rng, center, H, W)
        depth = rng.uniform(1.5, 3.5, (H, W)).astype(np.float32)
        depth[rng.uniform(size=(H, W)) < 0.03] = np.nan
        depth[rng.uniform(size=(H, W)) < 0.03] = -1.0
        depth[rng.uniform(size=(H, W)) < 0.03] = np.inf
        alpha = rng.uniform(0.0, 1.0, (H, W)).astype(np.float32)
        orc.tsdf_integrate(grid, origin, vs, vm, fx, fy, cx, cy, depth, alpha, 0.136, 0.3)
        dd, da = E.DeviceArray.from_numpy(depth), E.DeviceArray.from_numpy(alpha)
        keep += [dd, da]
        views.append((vm, fx, fy, cx, cy, dd, da))
    assert (grid != g0).any()
    # the first view alone, then the other three in one call
    E.tsdf_integrate(dev, origin, vs, views[:1], 0.136, 0.3)
    E.tsdf_integrate(dev, origin, vs, views[1:], 0.136, 0.3)
    got = dev.numpy()
    assert np.array_equal(got.view(np.uint32), grid.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("hw", [(37, 53), (64, 64), (1, 5000)])
def test_gpu_unprojection_matches_oracle(orc, eng, hw):
    from msplat import _engine as E
    H, W = hw
    rng = np.random.default_rng(H * W)
    img = rng.uniform(-0.3, 1.3, (H, W, 3)).astype(np.float32)
    img.reshape(-1)[rng.integers(0, img.size, 20)] = np.nan
    alpha = rng.uniform(0, 1, (H, W)).astype(np.float32)
    depth = (rng.uniform(0.5, 4.0, (H, W)) * alpha).astype(np.float32)
    depth[rng.uniform(size=(H, W)) < 0.05] = -1.0
    depth[rng.uniform(size=(H, W)) < 0.05] = np.nan
    c2w = np.eye(4, dtype=np.float32)
    c2w[:3, :3] = np.linalg.qr(rng.normal(size=(3, 3)))[0]
    c2w[:3, 3] = rng.normal(size=3)
    args = (W * 0.9, W * 1.1, W / 2, H / 2, c2w, 0.4)
    exp_xyz, exp_rgb = orc.unproject_depth(img, depth, alpha, *args)
    got_xyz, got_rgb = E.unproject_depth(E.DeviceArray.from_numpy(img), E.DeviceArray.from_numpy(depth),
                                         E.DeviceArray.from_numpy(alpha), *args)
    assert len(exp_xyz) > 0
    assert np.array_equal(got_xyz, exp_xyz) and np.array_equal(got_rgb, exp_rgb)


# ------------------------------------------------------------ end to end ----
def _sphere_surfels(n, R):
    """n surfels on a sphere of radius R (Fibonacci lattice), each lying in
    the tangent plane (local z along the normal), overlapping neighbours."""
    i = np.arange(n) + 0.5
    z = 1 - 2 * i / n
    phi = i * math.pi * (3 - math.sqrt(5))
    nrm = np.stack([np.sqrt(1 - z * z) * np.cos(phi), np.sqrt(1 - z * z) * np.sin(phi), z], 1)
    # rotation taking (0, 0, 1) to the normal: w = 1 + nz, xyz = (0,0,1) x n
    q = np.stack([1 + nrm[:, 2], -nrm[:, 1], nrm[:, 0], np.zeros(n)], 1)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    sigma = 0.7 * math.sqrt(4 * math.pi * R * R / n)
    return dict(means=(R * nrm).astype(np.float32), quats=q.astype(np.float32),
                scales=np.full((n, 2), math.log(sigma), np.float32),
                opacities=np.full((n, 1), 4.0, np.float32),
                features_dc=np.tile(np.float32([0.8, -0.3, 0.2]), (n, 1)),
                features_rest=np.zeros((n, 15, 3), np.float32))


def _write_ply(path, p, step):
    n = p["means"].shape[0]
    head = ["ply", "format binary_little_endian 1.0", f"comment msplat v{step}", f"element vertex {n}"]
    head += [f"property float {c}" for c in ("x", "y", "z", "nx", "ny", "nz")]
    head += [f"property float f_dc_{i}" for i in range(3)] + [f"property float f_rest_{i}" for i in range(45)]
    head += ["property float opacity", "property float scale_0", "property float scale_1"]
    head += [f"property float rot_{i}" for i in range(4)] + ["end_header"]
    rows = np.concatenate([p["means"], np.zeros((n, 3), np.float32), p["features_dc"],
                           p["features_rest"].transpose(0, 2, 1).reshape(n, 45), p["opacities"], p["scales"],
                           p["quats"]], 1).astype("<f4")
    path.write_bytes(("\n".join(head) + "\n").encode() + rows.tobytes())


def _orbit_poses(n, dist):
    """OpenGL camera-to-world poses on a sphere of radius dist, looking at
    the origin."""
    out = []
    for k in range(n):
        z = 1 - 2 * (k + 0.5) / n
        phi = k * math.pi * (3 - math.sqrt(5))
        eye = dist * np.array([math.sqrt(1 - z * z) * math.cos(phi), math.sqrt(1 - z * z) * math.sin(phi), z])
        back = eye / np.linalg.norm(eye)
        up0 = np.array([0.0, 0.0, 1.0]) if abs(back[2]) < 0.9 else np.array([1.0, 0.0, 0.0])
        right = np.cross(up0, back)
        right /= np.linalg.norm(right)
        up = np.cross(back, right)
        m = np.eye(4)
        m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = right, up, back, eye
        out.append(m)
    return np.array(out, np.float32)


def _read_mesh_ply(path):
    data = path.read_bytes()
    end = data.index(b"end_header\n") + len(b"end_header\n")
    head = data[:end].decode().splitlines()
    nv = int(next(h for h in head if h.startswith("element vertex")).split()[-1])
    nf = int(next(h for h in head if h.startswith("element face")).split()[-1])
    verts = np.frombuffer(data, "<f4", nv * 3, end).reshape(nv, 3)
    faces = np.frombuffer(data, np.uint8, nf * 13, end + nv * 12).reshape(nf, 13)
    return head, verts, faces


@pytest.mark.gpu
def test_extract_mesh_and_point_cloud_of_a_rendered_sphere(tmp_path, eng):
    """Surfels on a sphere of radius 0.2, 24 views from distance 1: the TSDF
    of their rendered median depth (4 mm voxels, 30 cm bound, 4-voxel
    truncation: the reference's defaults) meshes to the sphere, and the
    unprojected depth lands on it."""
    import msplat
    R, n_cams, W = 0.2, 24, 160
    poses = _orbit_poses(n_cams, 1.0)
    images = [np.zeros((W, W, 3), np.float32) for _ in range(n_cams)]
    intr = np.tile(np.float32([240.0, 240.0, W / 2, W / 2]), (n_cams, 1))
    ds = msplat.Dataset.from_arrays(images, poses, intr)
    tr = msplat.GaussianTrainer(ds, msplat.TrainingConfig(iterations=100))
    ply = tmp_path / "sphere.ply"
    _write_ply(ply, _sphere_surfels(20000, R), 30000)
    assert tr.load_ply(str(ply)) == 30000

    mesh = tmp_path / "mesh.ply"
    ntri = tr.extract_mesh(str(mesh))  # voxel 0.004, bound 0.3, alpha 0.5, trunc 4 voxels
    head, verts, faces = _read_mesh_ply(mesh)
    assert head == ["ply", "format binary_little_endian 1.0", "comment msplat 2c.3 Marching Cubes mesh (non-indexed)",
                    f"element vertex {3 * ntri}", "property float x", "property float y", "property float z",
                    f"element face {ntri}", "property list uchar int vertex_indices", "end_header"]
    assert ntri > 10000
    assert np.all(faces[:, 0] == 3)
    idx = faces[:, 1:].copy().view("<i4").reshape(ntri, 3)
    assert np.array_equal(idx, np.arange(3 * ntri, dtype=np.int32).reshape(ntri, 3))
    d = np.linalg.norm(verts.astype(np.float64), axis=1)
    assert np.median(np.abs(d - R)) < 0.002 and np.percentile(np.abs(d - R), 99) < 0.006
    area, vol, cr = _area_volume(verts.reshape(-1, 3, 3))
    assert abs(area / (4 * math.pi * R * R) - 1) < 0.05
    assert abs(-vol / (4 / 3 * math.pi * R ** 3) - 1) < 0.05  # inward winding

    pc = tmp_path / "points.ply"
    npts = tr.export_point_cloud(str(pc), 0.5)
    data = pc.read_bytes()
    end = data.index(b"end_header\n") + len(b"end_header\n")
    assert f"element vertex {npts}".encode() in data[:end]
    assert b"comment msplat 2c.0 point cloud (unprojected depth, 24 views)" in data[:end]
    rows = np.frombuffer(data, np.uint8, npts * 15, end).reshape(npts, 15)
    xyz = rows[:, :12].copy().view("<f4").reshape(npts, 3)
    # every view sees a disc of radius ~49 px
    assert npts > n_cams * 0.8 * math.pi * 45 ** 2
    dd = np.linalg.norm(xyz.astype(np.float64), axis=1)
    assert np.median(np.abs(dd - R)) < 0.003
