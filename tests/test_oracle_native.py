"""The oracle's C visibility (oracle/visible.c) against the oracle's PyTorch restatement and the
reference's golden vectors, on the CPU.

The C version exists to brute-force every triangle of the full-size workloads at thousands of
pixels (the GPU tests' id checks); it must decide exactly as oracle/reference.py does: the same
ids and the same depth bits at every pixel, over several peel layers, including exact edge
ties on pixel centres, triangles crossing the camera plane, degenerate and non-finite ones.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import mixed_mesh, random_mesh, tiny_mesh
from oracle import native
from oracle import reference as R

GOLDEN = Path(__file__).parent / "golden"


def every_pixel(batch, height, width):
    b, row, col = torch.meshgrid(torch.arange(batch), torch.arange(height), torch.arange(width),
                                 indexing="ij")
    return b.reshape(-1), row.reshape(-1), col.reshape(-1)


def native_layers(pos, tri, res, count):
    """(depth, id) images of ``count`` peel layers from the C oracle, every pixel."""
    h, w = res
    batch = pos.shape[0] if pos.ndim == 3 else 1
    b, row, col = every_pixel(batch, h, w)
    previous, out = None, []
    for _ in range(count):
        depth, ids = native.visible_at(pos, tri, h, w, b, row, col, previous)
        previous = (depth, ids)
        out.append((depth.view(batch, h, w), ids.view(batch, h, w)))
    return out


def torch_layers(pos, tri, res, count):
    pos = pos if pos.ndim == 3 else pos[None]
    px, py = R.pixel_centres(res[0], res[1], pos)
    previous, out = None, []
    for _ in range(count):
        previous = R.visible_triangles(pos, tri, px, py, previous)
        out.append(previous)
    return out


def assert_same(pos, tri, res, count=3):
    ours = native_layers(pos, tri, res, count)
    ref = torch_layers(pos, tri, res, count)
    for layer, ((d, i), (ed, ei)) in enumerate(zip(ours, ref)):
        assert torch.equal(i, ei), f"layer {layer}: ids differ at {(i != ei).sum()} pixels"
        assert torch.equal(d, ed), f"layer {layer}: depths differ"
    return ref


@pytest.mark.parametrize("scene", ["random", "crossing", "clipped", "tiny"])
def test_golden_ids_over_four_layers(scene):
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "raster.npz").items()}
    pos, tri = g[f"{scene}/pos"], g[f"{scene}/tri"]
    res = tuple(int(v) for v in g[f"{scene}/res"])
    for layer, (_, ids) in enumerate(native_layers(pos, tri, res, 4)):
        assert torch.equal(ids + 1, g[f"{scene}/rast{layer}"][..., 3].long()), (scene, layer)


@pytest.mark.parametrize("w_range", [(1.0, 2.0), (-1.0, 2.0)])
def test_random_triangles_per_view(w_range):
    pos, tri = random_mesh(150, torch.Generator().manual_seed(40), batch=3, w_range=w_range)
    ref = assert_same(pos, tri, (29, 37))
    assert (ref[0][1] >= 0).any() and (ref[1][1] >= 0).any()


def test_shared_positions_and_tiny_triangles():
    pos, tri = tiny_mesh(800, torch.Generator().manual_seed(41), 0.05, batch=1)
    assert_same(pos[0], tri, (48, 40))
    pos, tri = mixed_mesh(torch.Generator().manual_seed(42), batch=2)
    assert_same(pos, tri, (33, 50), count=2)


def test_lattice_triangles_with_exact_edge_ties():
    # Vertices on pixel centres of an 8x8 image at w = 1 (centres are k/8 - 15/16 ... exact
    # in float32), so edge functions are exactly zero along shared edges and the fill rule's
    # tie-breaks decide; equal depths everywhere, so the index order decides the layers.
    gen = torch.Generator().manual_seed(43)
    n = 120
    ij = torch.randint(0, 8, (1, 3 * n, 2), generator=gen).float()
    xy = (ij * 2 + 1) / 8 - 1
    z = torch.full((1, 3 * n, 1), 0.25)
    pos = torch.cat([xy, z, torch.ones(1, 3 * n, 1)], -1)
    tri = torch.arange(3 * n, dtype=torch.int32).view(n, 3)
    ref = assert_same(pos, tri, (8, 8), count=4)
    assert (ref[3][1] >= 0).any()


def test_degenerate_and_non_finite_triangles():
    pos, tri = random_mesh(60, torch.Generator().manual_seed(44), batch=1)
    pos = pos.clone()
    pos[0, 3:6] = pos[0, 3]                      # a point
    pos[0, 7] = (pos[0, 6] + pos[0, 8]) / 2      # collinear
    pos[0, 9, 0] = float("nan")
    pos[0, 13, 3] = float("inf")
    pos[0, 17, 1] = 1e30                          # edge products overflow
    tri = torch.cat([tri, torch.tensor([[0, 0, 1], [2, 2, 2]], dtype=torch.int32)])
    assert_same(pos, tri, (40, 40))


def test_list_of_pixels_matches_the_torch_list_version():
    pos, tri = random_mesh(400, torch.Generator().manual_seed(45), batch=2)
    gen = torch.Generator().manual_seed(46)
    b = torch.randint(0, 2, (300,), generator=gen)
    row = torch.randint(0, 70, (300,), generator=gen)
    col = torch.randint(0, 90, (300,), generator=gen)
    d, i = native.visible_at(pos, tri, 70, 90, b, row, col)
    ed, ei = R.visible_at(pos, tri, 70, 90, b, row, col)
    assert torch.equal(i, ei) and torch.equal(d, ed)
    d2, i2 = native.visible_at(pos, tri, 70, 90, b, row, col, (d, i))
    ed2, ei2 = R.visible_at(pos, tri, 70, 90, b, row, col, (ed, ei))
    assert torch.equal(i2, ei2) and torch.equal(d2, ed2)
    assert (i2 >= 0).any()


@pytest.mark.parametrize("half_width", [2.0 ** -5, 0.5])
@pytest.mark.parametrize(("steps", "drawn"), [(4, False), (16, False), (18, True), (64, True)])
def test_slivers_at_the_area_tolerance(half_width, steps, drawn):
    # The reference's sliver rule (tests/test_coverage.py:581-589): a sliver around the centre
    # of pixel (8, 8) of 16x16 whose area there is 2 * steps / 17 epsilons of its terms (every
    # value computed is exact) is drawn from 18 steps on, not at 16 or fewer.
    centre, step = 0.0625, 2.0 ** -27
    xy = [[-half_width, -steps * step], [half_width, -steps * step], [0.0, steps * step]]
    pos = torch.tensor([[[centre + x, centre + y, 0.0, 1.0] for x, y in xy]])
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    (_, ids), = native_layers(pos, tri, (16, 16), 1)
    assert (ids[0, 8, 8] == 0).item() == drawn
    assert drawn or (ids == -1).all()
    assert_same(pos, tri, (16, 16), count=1)


@pytest.mark.parametrize("shape", ["along_x", "along_y", "diagonal"])
def test_sliver_sweep_equals_the_torch_oracle(shape):
    # Slivers from 1 to 99 steps thick, lying along x, along y or along the diagonal: the
    # drawn/not-drawn boundary moves with every term of the area tolerance (along the diagonal
    # span_x and span_y are both of the order of the reaches), so the C test must place it
    # where the PyTorch oracle does.
    centre, step = 0.0625, 2.0 ** -27
    verts = []
    for steps in range(1, 100):
        d = steps * step
        if shape == "diagonal":
            xy = [[-0.5 + d, -0.5 - d], [0.5 + d, 0.5 - d], [-d, d]]
        else:
            xy = [[-0.5, -d], [0.5, -d], [0.0, d]]
            if shape == "along_y":
                xy = [[y, x] for x, y in xy]
        verts += [[centre + x, centre + y, 0.0, 1.0] for x, y in xy]
    pos = torch.tensor(verts)
    drawn = []
    for k in range(99):
        tri = torch.tensor([[3 * k, 3 * k + 1, 3 * k + 2]], dtype=torch.int32)
        ref = assert_same(pos, tri, (16, 16), count=1)
        drawn.append(bool(ref[0][1][0, 8, 8] == 0))
    assert not drawn[0] and drawn[-1]  # the boundary lies inside the sweep
