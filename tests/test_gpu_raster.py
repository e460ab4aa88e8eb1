"""Rasterize on the GPU against the CPU oracle: ids bit-exact, values and gradients to tolerance.

The oracle (oracle/reference.py) restates the reference backend's visibility arithmetic op for
op, so every pixel of every depth layer must pick the same triangle. Barycentrics, depth and
rast_db must agree within 1e-5 relative (normalised by max(|value|, 1)), gradients within 1e-4.
"""

import numpy as np
import pytest
import torch

import diffrast_amd as dr
from diffrast_amd.backends import hip
from helpers import mixed_mesh, random_mesh, rel_error, tiny_mesh
from oracle import reference as R

pytestmark = pytest.mark.gpu

VALUE_TOL = 1e-5
GRAD_TOL = 1e-4


def gpu_layers(pos, tri, res, count, grad_db=True):
    state, out = None, []
    for _ in range(count):
        rast, db, state = hip.rasterize_layer(pos.cuda(), tri.cuda(), res, grad_db, state)
        out.append((rast.cpu(), db.cpu()))
    return out


def oracle_layers(pos, tri, res, count):
    state, out = None, []
    for _ in range(count):
        rast, db, state = R.rasterize_layer(pos, tri, res, True, state)
        out.append((rast, db))
    return out


def assert_layers_match(pos, tri, res, count=1):
    ours = gpu_layers(pos, tri, res, count)
    ref = oracle_layers(pos, tri, res, count)
    for layer, ((r, d), (er, ed)) in enumerate(zip(ours, ref)):
        assert torch.equal(r[..., 3], er[..., 3]), f"layer {layer}: ids differ at " \
            f"{(r[..., 3] != er[..., 3]).sum().item()} pixels"
        assert rel_error(r[..., :3], er[..., :3]) < VALUE_TOL, f"layer {layer} rast"
        assert rel_error(d, ed) < VALUE_TOL, f"layer {layer} rast_db"
    return ref


def test_golden_fixtures_bit_exact_ids():
    g = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "raster.npz")
    for name in ("random", "crossing", "clipped", "tiny"):
        pos = torch.from_numpy(g[f"{name}/pos"])
        tri = torch.from_numpy(g[f"{name}/tri"])
        res = tuple(int(v) for v in g[f"{name}/res"])
        ours = gpu_layers(pos, tri, res, 4)
        for layer, (rast, db) in enumerate(ours):
            expected = torch.from_numpy(g[f"{name}/rast{layer}"])
            assert torch.equal(rast[..., 3], expected[..., 3]), (name, layer)
            assert rel_error(rast[..., :3], expected[..., :3]) < VALUE_TOL, (name, layer)
            if layer == 0:
                assert rel_error(db, torch.from_numpy(g[f"{name}/db0"])) < VALUE_TOL, name


@pytest.mark.parametrize("resolution", [(16, 16), (37, 61), (128, 96)])
def test_random_meshes(resolution):
    pos, tri = random_mesh(200, torch.Generator().manual_seed(0))
    ref = assert_layers_match(pos, tri, resolution)
    assert (ref[0][0][..., 3] > 0).float().mean() > 0.5


def test_batch_of_views():
    pos, tri = random_mesh(50, torch.Generator().manual_seed(1), batch=4)
    assert_layers_match(pos, tri, (48, 64))


def test_triangles_crossing_the_camera_plane():
    pos, tri = random_mesh(60, torch.Generator().manual_seed(2), w_range=(-1.0, 2.0))
    ref = assert_layers_match(pos, tri, (64, 64))
    assert (ref[0][0][..., 3] > 0).any()


def test_depth_clipping_and_culling():
    pos, tri = random_mesh(100, torch.Generator().manual_seed(3), z_range=2.0, xy_range=3.0)
    assert_layers_match(pos, tri, (64, 64))


def test_many_overlapping_triangles_in_one_tile():
    # More triangles per tile than one work chunk holds.
    pos, tri = random_mesh(700, torch.Generator().manual_seed(4), xy_range=0.9)
    assert_layers_match(pos, tri, (16, 16), count=3)


@pytest.mark.parametrize("size", [0.03, 3e-4])
def test_tiny_triangles(size):
    pos, tri = tiny_mesh(3000, torch.Generator().manual_seed(6), size, batch=2)
    assert_layers_match(pos, tri, (64, 64))


def test_mixed_triangle_sizes():
    pos, tri = mixed_mesh(torch.Generator().manual_seed(7))
    assert_layers_match(pos, tri, (96, 80), count=2)


def test_large_mesh_in_spatial_order_keeps_index_tie_break():
    # Meshes of 8192 triangles or more are processed in a spatially sorted order. Copies of
    # earlier triangles appended at the end tie in depth with their originals, which must win;
    # non-finite and camera-crossing triangles must not disturb the sort's bounds.
    gen = torch.Generator().manual_seed(21)
    small, small_tri = tiny_mesh(9000, gen, 0.05, batch=2)
    large, large_tri = random_mesh(60, gen, batch=2, w_range=(-1.0, 2.0))
    pos = torch.cat([small, large], 1)
    tri = torch.cat([small_tri, large_tri + small.shape[1]])
    tri = torch.cat([tri, tri[:700].flip(0)])
    pos[:, 5, :] = float("nan")
    pos[1, 40, 0] = float("inf")
    assert tri.shape[0] >= 8192
    ref = assert_layers_match(pos, tri, (64, 72), count=3)
    ids = ref[0][0][..., 3]
    assert (ids > 0).any() and not (ids > tri.shape[0] - 700).any()


def test_triangles_behind_a_covered_tile_are_skipped_exactly():
    # A dense front layer of small quads (drawn before the tile pass) covers every pixel; large
    # triangles entirely behind it may be skipped, large ones that reach in front, touch its
    # farthest depth or intersect it may not. Every layer must match the oracle.
    gen = torch.Generator().manual_seed(23)
    n = 20  # quads per side
    ys, xs = torch.meshgrid(torch.linspace(-1.05, 1.05, n + 1), torch.linspace(-1.05, 1.05, n + 1),
                            indexing="ij")
    z = (torch.rand(n + 1, n + 1, generator=gen) - 0.5) * 0.4
    grid = torch.stack([xs, ys, z, torch.ones_like(z)], -1).reshape(-1, 4)
    idx = torch.arange((n + 1) * (n + 1)).view(n + 1, n + 1)
    a, b_, c, d = idx[:-1, :-1], idx[:-1, 1:], idx[1:, :-1], idx[1:, 1:]
    front_tri = torch.cat([torch.stack([a, b_, c], -1), torch.stack([b_, d, c], -1)]).view(-1, 3)
    behind, _ = random_mesh(150, gen, z_range=1.0, xy_range=1.0)
    behind[..., 2] = (0.3 + 0.6 * torch.rand(behind.shape[1], generator=gen)) * behind[..., 3]
    across, _ = random_mesh(60, gen, z_range=0.5, xy_range=1.0)
    touching, _ = random_mesh(20, gen, xy_range=1.0)
    touching[..., 2] = z.max() * touching[..., 3]
    extra = torch.cat([behind[0], across[0], touching[0]])
    pos = torch.cat([grid, extra])[None]
    tri = torch.cat([front_tri.to(torch.int32),
                     (torch.arange(extra.shape[0]) + grid.shape[0]).view(-1, 3).to(torch.int32)])
    assert_layers_match(pos, tri, (64, 64), count=3)


def test_subdivided_sphere_in_spatial_order():
    from diffrast_amd import workloads as W
    gen = torch.Generator().manual_seed(22)
    verts, tri = W.icosphere(5)
    verts = verts * (1 + 0.02 * torch.randn(verts.shape[0], 1, generator=gen))
    pos = W.clip_positions(verts, W.random_eyes(2, 3.0, gen), 1.0)
    assert tri.shape[0] >= 8192
    assert_layers_match(pos, tri, (96, 96), count=2)


@pytest.mark.parametrize("resolution", [(97, 131), (48, 40)])
def test_mesh_outgrowing_an_l2_every_pixel_from_ids(resolution):
    # icosphere(7), 327,680 triangles: the index rows and vertices one image's pixels gather
    # outgrow an XCD's L2, so resolve and interpolate take their tile layout. At sizes that are
    # not multiples of the tiles, rast, rast_db and the interpolated attributes of every pixel
    # must match the oracle run from the GPU's ids (ids bit-exact against brute force at
    # sampled pixels).
    from diffrast_amd import workloads as W
    gen = torch.Generator().manual_seed(31)
    verts, tri = W.icosphere(7)
    verts = verts * (1 + 0.02 * torch.randn(verts.shape[0], 1, generator=gen))
    h, w = resolution
    pos = W.clip_positions(verts, W.random_eyes(3, 2.5, gen), w / h)
    rast, db, _ = hip.rasterize_layer(pos.cuda(), tri.cuda(), resolution, True, None)
    rast, db = rast.cpu(), db.cpu()
    ids = rast[..., 3].long() - 1
    assert (ids >= 0).sum() > 0.2 * ids.numel()
    b = torch.arange(3).repeat_interleave(16)
    row = torch.randint(0, h, (48,), generator=gen)
    col = torch.randint(0, w, (48,), generator=gen)
    _, expect_ids = R.visible_at(pos, tri, h, w, b, row, col)
    assert torch.equal(ids[b, row, col], expect_ids)
    ref, ref_db = R.rasterize_from_ids(pos, tri, ids, True)
    assert torch.equal(rast[..., 3], ref[..., 3])
    assert rel_error(rast[..., :3], ref[..., :3]) < VALUE_TOL
    assert rel_error(db, ref_db) < VALUE_TOL
    attr = torch.randn(verts.shape[0], 8, generator=gen)
    uv = W.spherical_uv(verts)
    for a, diff in ((attr, ()), (uv, (0, 1))):
        out, out_da = hip.interpolate(a.cuda(), rast.cuda(), tri.cuda(), db.cuda(), diff)
        e_out, e_da = R.interpolate(a, rast, tri, db, list(diff))
        assert torch.equal(out.cpu(), e_out)
        if diff:
            assert rel_error(out_da.cpu(), e_da) < VALUE_TOL


def test_processing_order_is_reused_per_tri_and_recomputed_when_tri_changes():
    # A large mesh's processing order is computed once per tri and reused with other
    # positions (the keys do not depend on it); an in-place change of tri makes a new one.
    from diffrast_amd import workloads as W
    gen = torch.Generator().manual_seed(23)
    verts, tri = W.icosphere(5)
    tri_dev = tri.cuda()
    hip._ORDERS.clear()
    for eyes_seed in (1, 2):
        eyes = W.random_eyes(2, 3.0, torch.Generator().manual_seed(eyes_seed))
        pos = W.clip_positions(verts * (1 + 0.02 * torch.randn(verts.shape[0], 1, generator=gen)),
                               eyes, 1.0)
        rast, db, _ = hip.rasterize_layer(pos.cuda(), tri_dev, (64, 80), True, None)
        (er, ed), = oracle_layers(pos, tri, (64, 80), 1)
        assert torch.equal(rast[..., 3].cpu(), er[..., 3])
        assert rel_error(rast[..., :3].cpu(), er[..., :3]) < VALUE_TOL
        assert len(hip._ORDERS) == 1
    order = next(iter(hip._ORDERS.values())).tensor
    # Reverse every triangle's winding in place: a new tri, a new order.
    tri_dev[:, [1, 2]] = tri_dev[:, [2, 1]]
    flipped = tri[:, [0, 2, 1]].contiguous()
    rast, db, _ = hip.rasterize_layer(pos.cuda(), tri_dev, (64, 80), True, None)
    (er, ed), = oracle_layers(pos, flipped, (64, 80), 1)
    assert torch.equal(rast[..., 3].cpu(), er[..., 3])
    assert rel_error(db.cpu(), ed) < VALUE_TOL
    assert len(hip._ORDERS) == 2
    assert all(e.tensor.data_ptr() != order.data_ptr() or e.tensor is order
               for e in hip._ORDERS.values())


def test_depth_peelers_share_the_processing_order_of_their_tri():
    # A peeler rasterizes a copy of tri. A peeler made before tri has a processing order
    # computes one for its copy and hands it back to tri; a later peeler's copy takes tri's
    # instead of computing its own. The layers are the oracle's either way.
    from diffrast_amd import workloads as W
    verts, tri = W.icosphere(5)
    pos_cpu = W.clip_positions(verts, W.random_eyes(2, 3.0, torch.Generator().manual_seed(25)),
                               1.0)
    pos, tri_dev, res = pos_cpu.cuda(), tri.cuda(), (64, 80)
    ctx = dr.RasterizeContext("cuda")
    hip._ORDERS.clear()
    with dr.DepthPeeler(ctx, pos, tri_dev, res) as peeler:
        first = [peeler.rasterize_next_layer()[0] for _ in range(2)]
    assert any(e.ref() is tri_dev for e in hip._ORDERS.values())
    computed = {id(e.tensor) for e in hip._ORDERS.values()}
    assert len(computed) == 1
    with dr.DepthPeeler(ctx, pos, tri_dev, res) as peeler:
        assert sum(e.ref() is peeler._geometry[1] for e in hip._ORDERS.values()) == 1
        second = [peeler.rasterize_next_layer()[0] for _ in range(2)]
    assert {id(e.tensor) for e in hip._ORDERS.values()} == computed
    for layer, (a, b, (er, _)) in enumerate(zip(first, second, oracle_layers(pos_cpu, tri, res, 2))):
        assert torch.equal(a, b), layer
        assert torch.equal(a[..., 3].cpu(), er[..., 3]), layer
    # A tri changed in place after its peeler was made keeps its own state: the peeler's copy
    # holds the old triangles, so its order is not handed back.
    hip._ORDERS.clear()
    flipped = tri_dev.clone()
    with dr.DepthPeeler(ctx, pos, flipped, res) as peeler:
        flipped[:, [1, 2]] = flipped[:, [2, 1]]
        peeler.rasterize_next_layer()
    assert not any(e.ref() is flipped for e in hip._ORDERS.values())


@pytest.mark.parametrize("w_range", [(1.0, 2.0), (-1.0, 2.0)])
def test_every_pixel_of_every_layer(w_range):
    gen = torch.Generator().manual_seed(9)
    xy = torch.rand(2, 900, 2, generator=gen) * 3 - 1.5
    z = torch.rand(2, 900, 1, generator=gen) * 2.4 - 1.2
    w = torch.rand(2, 900, 1, generator=gen) * (w_range[1] - w_range[0]) + w_range[0]
    pos = torch.cat([xy * w, z * w, w], -1)
    tri = torch.arange(900, dtype=torch.int32).view(300, 3)
    for resolution in ((64, 64), (37, 61), (255, 257)):
        ref = assert_layers_match(pos, tri, resolution, count=4)
        assert (ref[3][0][..., 3] > 0).any()


def test_equal_depths_resolve_in_index_order():
    quad = [[-0.2, -0.2, 0.25, 1.0], [0.2, -0.2, 0.25, 1.0], [0.0, 0.2, 0.25, 1.0]]
    pos = torch.tensor([quad * 3])
    tri = torch.tensor([[6, 7, 8], [0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    layers = gpu_layers(pos, tri, (8, 8), 4)
    covered = layers[0][0][..., 3] > 0
    assert covered.any()
    for (rast, _), expected in zip(layers, [1, 2, 3, 0]):
        assert (rast[..., 3][covered] == expected).all()


def test_negative_and_zero_depth_ordering():
    def flat(z):
        return [[-1.0, -1.0, z, 1.0], [3.0, -1.0, z, 1.0], [-1.0, 3.0, z, 1.0]]

    pos = torch.tensor([flat(0.5) + flat(-0.0) + flat(-0.5) + flat(0.0)])
    tri = torch.arange(12, dtype=torch.int32).view(4, 3)
    (rast, _), = gpu_layers(pos, tri, (8, 8), 1)
    assert (rast[..., 3] == 3).all()
    layers = gpu_layers(pos, tri, (8, 8), 4)
    ref = oracle_layers(pos, tri, (8, 8), 4)
    for (r, _), (e, _) in zip(layers, ref):
        assert torch.equal(r[..., 3], e[..., 3])


def test_empty_and_fully_culled_meshes():
    pos = torch.tensor([[[-0.5, -0.5, 0.0, -1.0], [0.5, -0.5, 0.0, -1.0], [0.0, 0.5, 0.0, -1.0]]])
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    for t in (tri, tri[:0]):
        (rast, db), = gpu_layers(pos, t, (16, 16), 1)
        assert (rast == 0).all() and (db == 0).all()


@pytest.mark.parametrize("value", [float("nan"), float("inf")])
def test_non_finite_vertices_are_culled(value):
    pos, tri = random_mesh(200, torch.Generator().manual_seed(8))
    pos[0, ::7, 3] = value  # breaks some triangles, not all
    ref = assert_layers_match(pos, tri, (64, 64))
    (rast, db), = gpu_layers(pos, tri, (64, 64), 1)
    assert torch.isfinite(rast).all() and torch.isfinite(db).all()
    assert (ref[0][0][..., 3] > 0).any()


def test_collinear_and_repeated_index_triangles_are_not_drawn():
    gen = torch.Generator().manual_seed(0)
    ends = torch.randint(-9, 10, (4000, 2, 2), generator=gen).float() / 10
    xy = torch.cat([ends, ends.mean(1, keepdim=True)], 1).reshape(1, -1, 2)
    w = 1 + torch.rand(1, xy.shape[1], 1, generator=gen)
    pos = torch.cat([xy * w, torch.zeros_like(w), w], -1)
    tri = torch.arange(pos.shape[1], dtype=torch.int32).view(-1, 3)
    (rast, _), = gpu_layers(pos, tri, (100, 100), 1)
    assert (rast[..., 3] == 0).all()
    i, j = torch.randint(0, pos.shape[1], (2, 3000), generator=gen)
    rep = torch.cat([torch.stack([i, i, j], -1), torch.stack([i, j, i], -1)]).int()
    (rast, _), = gpu_layers(pos, rep, (100, 100), 1)
    assert (rast[..., 3] == 0).all()


def lattice(cols, rows, resolution, w=1.0, z=0.0):
    """Vertices projecting exactly onto pixel centres (computed like the rasterizer's)."""
    height, width = resolution
    x = (cols.float() * 2 + 1) / width - 1
    y = (rows.float() * 2 + 1) / height - 1
    w = torch.as_tensor(w, dtype=torch.float32).expand(x.shape)
    return torch.stack([x * w, y * w, z * w, w], -1)[None]


def grid_triangles(nx, ny, gen):
    idx = torch.arange((nx + 1) * (ny + 1)).view(ny + 1, nx + 1)
    a, b, c, d = (t.flatten() for t in (idx[:-1, :-1], idx[:-1, 1:], idx[1:, 1:], idx[1:, :-1]))
    flip = (torch.rand(nx * ny, generator=gen) < 0.5)[:, None]
    first = torch.where(flip, torch.stack([a, b, d], -1), torch.stack([a, b, c], -1))
    second = torch.where(flip, torch.stack([b, c, d], -1), torch.stack([a, c, d], -1))
    tri = torch.cat([first, second])
    order = torch.stack([torch.randperm(3, generator=gen) for _ in range(tri.shape[0])])
    return tri.gather(1, order).int()


@pytest.mark.parametrize("resolution", [(100, 100), (255, 255), (600, 800)])
def test_meshes_through_pixel_centres_cover_every_pixel_once(resolution):
    gen = torch.Generator().manual_seed(2)
    height, width = resolution
    cell = 20
    nx, ny = (width + 1) // cell + 1, (height + 1) // cell + 1
    rows, cols = torch.meshgrid(torch.arange(ny + 1) * cell - 1, torch.arange(nx + 1) * cell - 1,
                                indexing="ij")
    w = torch.rand(rows.numel(), generator=gen) + 0.5
    pos = lattice(cols.flatten(), rows.flatten(), resolution, w=w)
    tri = grid_triangles(nx, ny, gen)
    first, second = gpu_layers(pos, tri, resolution, 2)
    assert (first[0][..., 3] > 0).all(), "holes"
    assert (second[0][..., 3] == 0).all(), "pixels covered twice"


def test_quad_diagonal_goes_to_the_triangle_on_its_right():
    for size in (8, 100, 255, 1000):
        pos = torch.tensor([[[-1.0, -1.0, 0.0, 1.0], [1.0, -1.0, 0.0, 1.0], [1.0, 1.0, 0.0, 1.0],
                             [-1.0, 1.0, 0.0, 1.0]]])
        tri = torch.tensor([[0, 1, 2], [0, 2, 3]], dtype=torch.int32)
        (rast, _), = gpu_layers(pos, tri, (size, size), 1)
        row, col = torch.meshgrid(torch.arange(size), torch.arange(size), indexing="ij")
        expected = torch.where(col >= row, 1.0, 2.0)
        assert torch.equal(rast[0, ..., 3], expected)


@pytest.mark.parametrize("size", [80001, 200003])
def test_very_wide_images(size):
    # Opposite quad sides on pixel-centre columns: the bounding boxes must keep them.
    gen = torch.Generator().manual_seed(8)
    first = torch.randint(0, size - 8, (3000,), generator=gen)
    last = first + torch.randint(1, 4, (3000,), generator=gen)
    along = torch.stack([first, last, last, first], -1).flatten()
    across = torch.tensor([-2, -2, 4, 4]).repeat(3000)
    pos = lattice(along, across, (2, size))
    quad = torch.tensor([[0, 1, 2], [0, 2, 3]])
    tri = (quad[None] + torch.arange(3000)[:, None, None] * 4).view(-1, 3).int()
    edges = torch.zeros(size + 1)
    edges.index_add_(0, first, torch.ones(3000)).index_add_(0, last, -torch.ones(3000))
    expected = (edges.cumsum(0)[:size] > 0).expand(2, size)
    (rast, _), = gpu_layers(pos, tri, (2, size), 1)
    assert torch.equal(rast[0, ..., 3] > 0, expected)


def test_range_mode_matches_per_item_oracle():
    gen = torch.Generator().manual_seed(11)
    pos, tri = random_mesh(120, gen, batch=1)
    pos = pos[0]
    ranges = torch.tensor([[0, 40], [30, 50], [100, 20], [0, 0], [60, 60]], dtype=torch.int32)
    rast, db, _ = hip.rasterize_ranges(pos.cuda(), tri.cuda(), (40, 48), True, ranges)
    ref, ref_db = R.rasterize_ranges(pos, tri, (40, 48), ranges)
    assert torch.equal(rast.cpu()[..., 3], ref[..., 3])
    assert rel_error(rast.cpu()[..., :3], ref[..., :3]) < VALUE_TOL
    assert rel_error(db.cpu(), ref_db) < VALUE_TOL


def test_range_mode_depth_peeling_matches_oracle():
    gen = torch.Generator().manual_seed(12)
    pos, tri = random_mesh(90, gen, batch=1, xy_range=0.7)
    pos = pos[0]
    ranges = torch.tensor([[0, 45], [45, 45], [20, 60]], dtype=torch.int32)
    state = None
    ref_states = [None] * 3
    for layer in range(3):
        rast, _, state = hip.rasterize_ranges(pos.cuda(), tri.cuda(), (32, 32), True, ranges, state)
        for item, (start, count) in enumerate(ranges.tolist()):
            r, _, ref_states[item] = R.rasterize_layer(pos[None], tri[start:start + count],
                                                       (32, 32), True, ref_states[item])
            ids = torch.where(r[..., 3] > 0, r[..., 3] + start, r[..., 3])
            assert torch.equal(rast.cpu()[item, ..., 3], ids[0]), (layer, item)


@pytest.mark.parametrize("grad_db", [True, False])
@pytest.mark.parametrize("use", ["rast", "db", "both"])
def test_gradients_match_oracle(grad_db, use):
    pos, tri = random_mesh(80, torch.Generator().manual_seed(1), batch=2, w_range=(-1.0, 2.0))
    gen = torch.Generator().manual_seed(0)
    w_rast = torch.randn(2, 40, 56, 4, generator=gen)
    w_db = torch.randn(2, 40, 56, 4, generator=gen)

    def run(fn, p, device):
        p = p.clone().to(device).requires_grad_(True)
        rast, db = fn(p, tri.to(device), (40, 56), grad_db)
        loss = 0
        if use in ("rast", "both"):
            loss = loss + (rast[..., :3] * w_rast[..., :3].to(device)).sum()
        if use in ("db", "both") and db.requires_grad:
            loss = loss + (db * w_db.to(device)).sum()
        if not torch.is_tensor(loss) or not loss.requires_grad:
            return None
        loss.backward()
        return p.grad.cpu()

    ours = run(hip.rasterize, pos, "cuda")
    ref = run(R.rasterize, pos, "cpu")
    if ref is None:
        assert ours is None
        return
    scale = ref.abs().max().item()
    torch.testing.assert_close(ours, ref, atol=GRAD_TOL * scale, rtol=GRAD_TOL)


def test_gradients_of_large_triangles_sharing_vertices():
    pos, tri = random_mesh(6, torch.Generator().manual_seed(2), xy_range=0.9)
    gen = torch.Generator().manual_seed(3)
    w_rast = torch.randn(1, 256, 256, 4, generator=gen)
    grads = []
    for fn, device in ((hip.rasterize, "cuda"), (R.rasterize, "cpu")):
        p = pos.clone().to(device).requires_grad_(True)
        rast, db = fn(p, tri.to(device), (256, 256), True)
        ((rast[..., :3] * w_rast[..., :3].to(device)).sum() + (db * w_rast.to(device)).sum()
         ).backward()
        grads.append(p.grad.cpu())
    scale = grads[1].abs().max().item()
    torch.testing.assert_close(grads[0], grads[1], atol=GRAD_TOL * scale, rtol=GRAD_TOL)


def test_public_api_and_double_backward_guard():
    ctx = dr.RasterizeContext("cuda")
    pos, tri = random_mesh(20, torch.Generator().manual_seed(5))
    pos = pos.cuda().requires_grad_(True)
    rast, db = dr.rasterize(ctx, pos, tri.cuda(), (16, 16))
    assert rast.shape == db.shape == (1, 16, 16, 4)
    with pytest.raises(RuntimeError, match="no second-order gradients"):
        torch.autograd.grad(rast[..., :3].square().sum(), pos, create_graph=True)


def test_outputs_no_gradient_reaches_add_zero_gradient():
    # rast that only feeds antialias (which has no gradient for it) and an interpolate whose
    # derivative output is unused: the positions' and attributes' gradients are those of the
    # paths that do carry one, and a leaf reached only through such outputs gets zeros.
    ctx = dr.RasterizeContext("cuda")
    gen = torch.Generator().manual_seed(17)
    pos0, tri = random_mesh(60, gen, batch=2)
    pos0, tri = pos0.cuda(), tri.cuda()
    color = torch.rand(2, 40, 48, 3, generator=gen).cuda()
    pos = pos0.clone().requires_grad_(True)
    rast, _ = dr.rasterize(ctx, pos, tri, (40, 48))
    dr.antialias(color, rast, pos, tri).square().sum().backward()
    expected = pos0.clone().requires_grad_(True)
    dr.antialias(color, rast.detach(), expected, tri).square().sum().backward()
    torch.testing.assert_close(pos.grad, expected.grad, rtol=1e-6,
                               atol=1e-6 * expected.grad.abs().max().item())
    # Only the derivative-free output used, against the same loss with the derivatives given a
    # zero weight.
    attr0 = torch.randn(pos0.shape[1], 3, generator=gen).cuda()
    grads = []
    for weigh_da in (False, True):
        p, attr = pos0.clone().requires_grad_(True), attr0.clone().requires_grad_(True)
        r, db = dr.rasterize(ctx, p, tri, (40, 48))
        out, out_da = dr.interpolate(attr, r, tri, db, diff_attrs="all")
        loss = out.square().sum() + (0.0 * out_da.sum() if weigh_da else 0.0)
        loss.backward()
        grads.append((p.grad, attr.grad))
    for a, b in zip(*grads):
        torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6 * b.abs().max().item())
    # A leaf reached only through an output without gradient still gets a (zero) gradient, as
    # from the reference's resolve backward run on zeros.
    p = pos0.clone().requires_grad_(True)
    c = color.clone().requires_grad_(True)
    r, _ = dr.rasterize(ctx, p, tri, (40, 48))
    dr.antialias(c, r, pos0, tri).square().sum().backward()
    assert c.grad is not None and p.grad is not None and not p.grad.any()


def test_depth_peeler_range_mode_through_public_api():
    ctx = dr.RasterizeContext("cuda")
    gen = torch.Generator().manual_seed(13)
    pos, tri = random_mesh(60, gen, batch=1, xy_range=0.6)
    pos, tri = pos[0].cuda(), tri.cuda()
    ranges = torch.tensor([[0, 30], [30, 30]], dtype=torch.int32)
    with dr.DepthPeeler(ctx, pos, tri, (24, 24), ranges=ranges) as peeler:
        first, _ = peeler.rasterize_next_layer()
        second, _ = peeler.rasterize_next_layer()
    both = (first[..., 3] > 0) & (second[..., 3] > 0)
    assert both.any()
    assert (second[..., 2][both] >= first[..., 2][both]).all()
    with pytest.raises(RuntimeError, match="closed"):
        peeler.rasterize_next_layer()


def _keys_through_abi(pos, tri, res, capacity, prev=None):
    """Keys from dr_raster_visibility_start with binning and the tile pass queued at once into
    an entry buffer of `capacity` (none when 0), completed with a buffer of the exact size
    when the lists do not fit."""
    import ctypes

    from diffrast_amd.backends import _lib

    geo = hip._Geometry(pos, tri, res)
    keys = torch.empty(geo.shape, dtype=torch.int64, device=pos.device)
    size = ctypes.c_size_t()
    _lib.call("dr_raster_workspace_size", _lib.ref(geo.struct), ctypes.byref(size))
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=pos.device)
    host = torch.full((4,), -1, dtype=torch.int32, pin_memory=True)
    stream = _lib.stream(pos.device)
    _lib.call("dr_raster_visibility_start", _lib.ref(geo.struct), _lib.ptr(prev),
              _lib.ptr(keys), _lib.ptr(workspace), size.value, host.data_ptr(), stream)
    arrived = torch.cuda.Event()
    arrived.record()
    entries = torch.empty(max(capacity, 1), dtype=torch.int64, device=pos.device)
    if capacity:
        spec = (ctypes.c_uint32 * 4)(0, capacity, 0, 0)
        _lib.call("dr_raster_visibility_bin", _lib.ref(geo.struct), _lib.ptr(workspace),
                  size.value, _lib.ptr(entries), spec, stream)
        _lib.call("dr_raster_visibility_tiles", _lib.ref(geo.struct), _lib.ptr(prev),
                  _lib.ptr(keys), _lib.ptr(workspace), size.value, _lib.ptr(entries), spec,
                  stream)
    arrived.synchronize()
    counts = (ctypes.c_uint32 * 4)(*[v & 0xFFFFFFFF for v in host.tolist()])
    if counts[1] > capacity:
        entries = torch.empty(counts[1], dtype=torch.int64, device=pos.device)
        _lib.call("dr_raster_visibility_bin", _lib.ref(geo.struct), _lib.ptr(workspace),
                  size.value, _lib.ptr(entries), counts, stream)
        _lib.call("dr_raster_visibility_tiles", _lib.ref(geo.struct), _lib.ptr(prev),
                  _lib.ptr(keys), _lib.ptr(workspace), size.value, _lib.ptr(entries), counts,
                  stream)
    torch.cuda.synchronize()
    return keys, list(counts)


def _keys_one_call(pos, tri, res, capacity, groups, prev=None):
    """Keys from dr_raster_visibility (no wait: an entry buffer of ``capacity``, a tile pass of
    ``groups`` workgroups, the overflow pass when the lists do not fit) and its counts."""
    import ctypes

    from diffrast_amd.backends import _lib

    geo = hip._Geometry(pos, tri, res)
    keys = torch.empty(geo.shape, dtype=torch.int64, device=pos.device)
    size = ctypes.c_size_t()
    _lib.call("dr_raster_workspace_size", _lib.ref(geo.struct), ctypes.byref(size))
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=pos.device)
    host = torch.full((4,), -1, dtype=torch.int32, pin_memory=True)
    entries = torch.empty(max(capacity, 1), dtype=torch.int64, device=pos.device)
    _lib.call("dr_raster_visibility", _lib.ref(geo.struct), _lib.ptr(prev), _lib.ptr(keys),
              _lib.ptr(workspace), size.value, _lib.ptr(entries) if capacity else None,
              capacity, groups, host.data_ptr(), _lib.stream(pos.device))
    torch.cuda.synchronize()
    return keys, [v & 0xFFFFFFFF for v in host.tolist()]


def _keys_waiting(pos, tri, res, prev=None, groups=None):
    """Keys from dr_raster_visibility_begin (which waits for the counts), bin and tiles (with
    a tile pass of ``groups`` workgroups instead of the counted grid, if given)."""
    import ctypes

    from diffrast_amd.backends import _lib

    geo = hip._Geometry(pos, tri, res)
    keys = torch.empty(geo.shape, dtype=torch.int64, device=pos.device)
    size = ctypes.c_size_t()
    _lib.call("dr_raster_workspace_size", _lib.ref(geo.struct), ctypes.byref(size))
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=pos.device)
    counts = (ctypes.c_uint32 * 4)()
    stream = _lib.stream(pos.device)
    _lib.call("dr_raster_visibility_begin", _lib.ref(geo.struct), _lib.ptr(prev),
              _lib.ptr(keys), _lib.ptr(workspace), size.value, counts, stream)
    if counts[1]:
        entries = torch.empty(counts[1], dtype=torch.int64, device=pos.device)
        _lib.call("dr_raster_visibility_bin", _lib.ref(geo.struct), _lib.ptr(workspace),
                  size.value, _lib.ptr(entries), counts, stream)
        grid = counts if groups is None else (ctypes.c_uint32 * 4)(
            counts[0], counts[1], groups, counts[3])
        _lib.call("dr_raster_visibility_tiles", _lib.ref(geo.struct), _lib.ptr(prev),
                  _lib.ptr(keys), _lib.ptr(workspace), size.value, _lib.ptr(entries), grid,
                  stream)
    torch.cuda.synchronize()
    return keys, list(counts)


def _ids_of(keys):
    """Triangle ids (-1: none) of visibility keys."""
    return torch.where(keys == -1, torch.full_like(keys, -1), keys & 0xFFFFFFFF)


def _native_layers(pos, tri, res, count):
    """Ids of ``count`` peel layers from the oracle's brute force at every pixel."""
    from oracle import native
    h, w = res
    batch = pos.shape[0]
    b, row, col = (t.reshape(-1) for t in torch.meshgrid(
        torch.arange(batch), torch.arange(h), torch.arange(w), indexing="ij"))
    previous, out = None, []
    for _ in range(count):
        previous = native.visible_at(pos, tri, h, w, b, row, col, previous)
        out.append(previous[1].view(batch, h, w))
    return out


@pytest.mark.parametrize("groups", [8, 24])
def test_tile_pass_with_a_short_grid_covers_every_tile(groups):
    # dr_raster_visibility_tiles with the call's own counts but a grid smaller than one
    # workgroup per busy tile: every tile must still be rasterized (every pixel against the
    # oracle, two layers).
    pos, tri = mixed_mesh(torch.Generator().manual_seed(12), batch=3)
    res = (96, 80)
    expect = _native_layers(pos, tri, res, 2)
    pos, tri = pos.cuda().contiguous(), tri.cuda().int().contiguous()
    prev = None
    for layer in range(2):
        keys, counts = _keys_waiting(pos, tri, res, prev, groups=groups)
        assert counts[3] > 0 and counts[2] > groups
        assert torch.equal(_ids_of(keys).cpu(), expect[layer]), layer
        prev = keys


def test_looping_tile_pass_beyond_the_plain_grid():
    # 1040 images of 128 x 128 are 66,560 tiles, more than the tile pass launches one
    # workgroup each for: the backend and the one-call entry point with grids of 8 and 24
    # run the looping kernel. Every pixel of two layers against the oracle.
    gen = torch.Generator().manual_seed(13)
    pos, tri = random_mesh(6, gen, batch=1040)
    res = (128, 128)
    expect = _native_layers(pos, tri, res, 2)
    assert (expect[1] >= 0).any()
    pos_dev, tri_dev = pos.cuda().contiguous(), tri.cuda().contiguous()
    hip._SIZES.clear()
    for repeat in range(2):  # the first call learns the sizes, the second queues at once
        state = None
        for layer in range(2):
            rast, _, state = hip.rasterize_layer(pos_dev, tri_dev, res, False, state)
            assert torch.equal(rast[..., 3].long().cpu() - 1, expect[layer]), (repeat, layer)
    for groups in (8, 24):
        prev = None
        for layer in range(2):
            keys, _ = _keys_one_call(pos_dev, tri_dev, res, 1 << 22, groups, prev)
            assert torch.equal(_ids_of(keys).cpu(), expect[layer]), (groups, layer)
            prev = keys


def test_processing_order_of_a_freed_tri_is_not_taken_by_a_new_one():
    # A tri freed and a different tri of the same shape allocated at its address, with a
    # fresh version counter: the new one must get its own processing order (the old one
    # carries the old triangles' vertex rows and ids).
    from diffrast_amd import workloads as W
    gen = torch.Generator().manual_seed(24)
    verts, tri = W.icosphere(5)
    pos = W.clip_positions(verts, W.random_eyes(2, 3.0, gen), 1.0)
    res = (64, 80)
    hip._ORDERS.clear()
    first = tri.cuda()
    address = first.data_ptr()
    hip.rasterize_layer(pos.cuda(), first, res, True, None)
    assert len(hip._ORDERS) == 1
    del first
    torch.cuda.synchronize()
    other_cpu = tri[torch.randperm(tri.shape[0], generator=gen)].contiguous()
    held = []
    other = other_cpu.cuda()
    while other.data_ptr() != address and len(held) < 64:
        held.append(other)
        other = other_cpu.cuda()
    assert other.data_ptr() == address and other._version == 0
    rast, db, _ = hip.rasterize_layer(pos.cuda(), other, res, True, None)
    (er, ed), = oracle_layers(pos, other_cpu, res, 1)
    assert torch.equal(rast[..., 3].cpu(), er[..., 3])
    assert rel_error(db.cpu(), ed) < VALUE_TOL
    del held


@pytest.mark.parametrize("resolution", [(96, 80), (40, 24), (300, 17)])
def test_visibility_with_entry_buffer_queued_before_the_counts(resolution):
    # Binning and the tile pass queued with an entry buffer that is large enough, exactly large
    # enough, one entry short or far too small must give the keys and counts of the calls that
    # wait for the counts, for the first layer and for a peeled one.
    pos, tri = mixed_mesh(torch.Generator().manual_seed(11), batch=3)
    pos, tri = pos.cuda().contiguous(), tri.cuda().int().contiguous()
    prev = None
    for layer in range(2):
        expected, counts = _keys_waiting(pos, tri, resolution, prev)
        n = counts[1]
        assert n > 0 and counts[2] > 0 and counts[0] > 0
        for capacity in (0, n + 5000, n, n - 1, 1):
            keys, got = _keys_through_abi(pos, tri, resolution, capacity, prev)
            assert got == counts, (layer, capacity)
            assert torch.equal(keys, expected), (layer, capacity)
            # The one-call form: lists that do not fit go through the overflow pass; a tile
            # pass of fewer workgroups than busy tiles loops over them.
            for groups in (0, 8, 24, counts[2]):
                keys, got = _keys_one_call(pos, tri, resolution, capacity, groups, prev)
                assert got == counts, (layer, capacity, groups)
                assert torch.equal(keys, expected), (layer, capacity, groups)
        prev = expected
    ours = [hip.rasterize_layer(pos, tri, resolution, True, None)[0] for _ in range(3)]
    assert torch.equal(ours[0], ours[1]) and torch.equal(ours[0], ours[2])


def test_tile_lists_outgrowing_the_remembered_size_through_public_path():
    # The same mesh shape drawn at a quarter of its size, then whole, alternately: the first
    # call learns its list sizes from the device; each whole-size call outgrows the buffer sized
    # from the call before and goes through the overflow pass; each small call fits. Every
    # layer must match the oracle, and the sizes remembered must follow the calls.
    gen = torch.Generator().manual_seed(5)
    pos, tri = random_mesh(2000, gen, batch=2)
    small = pos.clone()
    small[..., :2] *= 0.25
    res = (128, 128)
    hip._SIZES.clear()
    seen = []
    for p in (small, pos, small, pos):
        assert_layers_match(p, tri, res, count=2)
        torch.cuda.synchronize()
        first_layer = [v for k, v in hip._SIZES.items() if k[-1]]
        assert len(first_layer) == 1
        first_layer[0].refresh()
        seen.append(first_layer[0].entries)
    assert seen[0] > 0 and seen[1] > hip._entry_capacity(seen[0]), seen
    assert seen[2] == seen[0] and seen[3] == seen[1], seen