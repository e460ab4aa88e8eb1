"""Interpolate, texture and antialias on the GPU against the CPU oracle.

Forward values within 1e-5 relative (normalised by max(|value|, 1)), gradients within 1e-4
(normalised by the largest reference gradient), both stated per test.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

import diffrast_amd as dr
from diffrast_amd.backends import hip
from helpers import random_mesh, rel_error, tiny_mesh
from oracle import reference as R

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden"
VALUE_TOL = 1e-5
GRAD_TOL = 1e-4


def grads_of(fn, inputs, weights, device):
    ins = [t.clone().to(device).requires_grad_(True) if t is not None and t.is_floating_point()
           else (None if t is None else t.to(device)) for t in inputs]
    out = fn(*ins)
    outs = out if isinstance(out, tuple) else (out,)
    loss = sum((o * w.to(device)).nansum() for o, w in zip(outs, weights) if o.numel())
    loss.backward()
    grads = [None if t is None or not t.is_floating_point() else
             (t.grad.cpu() if t.grad is not None else torch.zeros_like(t).cpu()) for t in ins]
    return [o.detach().cpu() for o in outs], grads


def assert_grads_close(ours, ref, tol=GRAD_TOL):
    for g, e in zip(ours, ref):
        if g is None or e is None:
            continue
        scale = max(e.abs().max().item(), 1e-12)
        torch.testing.assert_close(g, e, atol=tol * scale, rtol=tol)


# ---- interpolate -----------------------------------------------------------------------------


def interp_scene(channels, layout, seed=0):
    gen = torch.Generator().manual_seed(seed)
    pos, tri = random_mesh(80, gen, batch=2)
    rast, rast_db = R.rasterize(pos, tri, (40, 56), True)
    v = pos.shape[1]
    shape = {"shared": (v, channels), "single": (1, v, channels)}.get(layout, (2, v, channels))
    attr = torch.randn(*shape, generator=gen)
    return attr, rast.detach(), rast_db.detach(), tri


@pytest.mark.parametrize("channels", [1, 2, 3, 4, 5, 8, 33])
@pytest.mark.parametrize("layout", ["shared", "single", "per_view"])
def test_interpolate_forward_is_bit_exact(channels, layout):
    attr, rast, db, tri = interp_scene(channels, layout)
    for diff in ([], list(range(channels)), [channels - 1, 0]):
        ref = R.interpolate(attr, rast, tri, db if diff else None, diff)
        out = hip.interpolate(attr.cuda(), rast.cuda(), tri.cuda(), db.cuda() if diff else None,
                              diff)
        assert torch.equal(out[0].cpu(), ref[0])
        assert torch.equal(out[1].cpu(), ref[1])


@pytest.mark.parametrize("layout", ["shared", "per_view"])
@pytest.mark.parametrize("diff", [[], [0, 2, 3], [1, 1]])
def test_interpolate_gradients(layout, diff):
    attr, rast, db, tri = interp_scene(20, layout, seed=1)
    gen = torch.Generator().manual_seed(2)
    w_out = torch.randn(*rast.shape[:3], 20, generator=gen)
    w_da = torch.randn(*rast.shape[:3], 2 * len(diff), generator=gen)
    ref = grads_of(lambda a, r, d: R.interpolate(a, r, tri, d, diff), [attr, rast, db],
                   [w_out, w_da], "cpu")
    ours = grads_of(lambda a, r, d: hip.interpolate(a, r, tri.cuda(), d, diff),
                    [attr, rast, db], [w_out, w_da], "cuda")
    assert_grads_close(ours[1], ref[1])


@pytest.mark.parametrize("channels", [1, 2, 3, 5, 8, 33])
@pytest.mark.parametrize("layout", ["shared", "per_view"])
def test_interpolate_gradients_of_constant_attributes(channels, layout):
    # Without an attribute gradient the backward pass has a kernel of its own (grad_rast and
    # grad_rast_db only); its sums run in the order of the pass that also scatters the attribute
    # gradient, so the two agree bit for bit, and both agree with the oracle.
    attr, rast, db, tri = interp_scene(channels, layout, seed=3)
    gen = torch.Generator().manual_seed(4)
    a, t = attr.cuda(), tri.cuda()
    for diff in ([], list(range(channels)), [channels - 1, 0], [0, 0]):
        w_out = torch.randn(*rast.shape[:3], channels, generator=gen)
        w_da = torch.randn(*rast.shape[:3], 2 * len(diff), generator=gen)
        ref = grads_of(lambda r, d: R.interpolate(attr, r, tri, d, diff), [rast, db],
                       [w_out, w_da], "cpu")
        ours = grads_of(lambda r, d: hip.interpolate(a, r, t, d, diff), [rast, db],
                        [w_out, w_da], "cuda")
        assert_grads_close(ours[1], ref[1])
        both = grads_of(lambda x, r, d: hip.interpolate(x, r, t, d, diff), [attr, rast, db],
                        [w_out, w_da], "cuda")
        assert torch.equal(ours[1][0], both[1][1]), diff
        assert torch.equal(ours[1][1], both[1][2]), diff


@pytest.mark.parametrize("channels", [2, 8])
def test_interpolate_gather_tiles_on_partial_tiles(channels):
    # Index rows of 400,000 triangles outgrow an L2, so the forward pass and the backward pass
    # of constant attributes take the tiled gather layout; 2 x 45 x 70 pixels leave partial tiles
    # at the right and lower edges. rast is synthetic (any barycentrics, ids, background).
    gen = torch.Generator().manual_seed(9)
    num_tri, num_vertices = 400_000, 150_000
    tri = torch.randint(0, num_vertices, (num_tri, 3), generator=gen, dtype=torch.int32)
    attr = torch.randn(num_vertices, channels, generator=gen)
    shape = (2, 45, 70)
    ids = torch.randint(0, num_tri + 1, shape, generator=gen).float()  # 0: background
    rast = torch.cat([torch.rand(*shape, 3, generator=gen), ids[..., None]], -1)
    db = torch.randn(*shape, 4, generator=gen)
    diff = list(range(channels))
    a, t = attr.cuda(), tri.cuda()
    ref = R.interpolate(attr, rast, tri, db, diff)
    out = hip.interpolate(a, rast.cuda(), t, db.cuda(), diff)
    assert torch.equal(out[0].cpu(), ref[0]) and torch.equal(out[1].cpu(), ref[1])
    w_out = torch.randn(*shape, channels, generator=gen)
    w_da = torch.randn(*shape, 2 * channels, generator=gen)
    expect = grads_of(lambda r, d: R.interpolate(attr, r, tri, d, diff), [rast, db],
                      [w_out, w_da], "cpu")
    ours = grads_of(lambda r, d: hip.interpolate(a, r, t, d, diff), [rast, db], [w_out, w_da],
                    "cuda")
    assert_grads_close(ours[1], expect[1])
    both = grads_of(lambda x, r, d: hip.interpolate(x, r, t, d, diff), [attr, rast, db],
                    [w_out, w_da], "cuda")
    assert torch.equal(ours[1][0], both[1][1]) and torch.equal(ours[1][1], both[1][2])


def test_interpolate_golden_fixture():
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "interpolate.npz").items()}
    outs, grads = grads_of(lambda a, r, d: hip.interpolate(a, r, g["tri"].cuda(), d, [3, 0]),
                           [g["attr"], g["rast"], g["rast_db"]],
                           [g["weights"], g["weights_da"]], "cuda")
    assert torch.equal(outs[0], g["out"]) and torch.equal(outs[1], g["out_da"])
    assert_grads_close(grads, [g["grad_attr"], g["grad_rast"], g["grad_rast_db"]])


def test_interpolate_ids_past_the_end_are_background():
    attr, rast, db, tri = interp_scene(3, "shared")
    rast = rast.clone()
    rast[0, :5, :5, 3] = tri.shape[0] + 7
    out, _ = hip.interpolate(attr.cuda(), rast.cuda(), tri.cuda(), None, [])
    assert (out[0, :5, :5] == 0).all()


# ---- texture ---------------------------------------------------------------------------------

FILTERS = ("nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear")
BOUNDARIES = ("wrap", "clamp", "zero")


def tex_scene(tex_batch=2, channels=3, size=(37, 50), seed=0):
    gen = torch.Generator().manual_seed(seed)
    tex = torch.randn(tex_batch, *size, channels, generator=gen)
    uv = torch.rand(2, 20, 24, 2, generator=gen) * 1.6 - 0.3
    uv_da = torch.rand(2, 20, 24, 4, generator=gen) * 0.2 - 0.1
    return tex, uv, uv_da


@pytest.mark.parametrize("boundary", BOUNDARIES)
@pytest.mark.parametrize("filter_mode", FILTERS)
@pytest.mark.parametrize("tex_batch, channels", [(1, 1), (2, 3), (2, 4), (2, 20)])
def test_texture_forward(filter_mode, boundary, tex_batch, channels):
    tex, uv, uv_da = tex_scene(tex_batch, channels)
    da = uv_da if "mipmap" in filter_mode else None
    ref = R.texture(tex, uv, da, filter_mode, boundary, None)
    out = hip.texture(tex.cuda(), uv.cuda(), None if da is None else da.cuda(), filter_mode,
                      boundary, None).cpu()
    assert torch.equal(out.isnan(), ref.isnan())
    assert rel_error(out.nan_to_num(), ref.nan_to_num()) < VALUE_TOL


@pytest.mark.parametrize("boundary", BOUNDARIES)
@pytest.mark.parametrize("filter_mode", FILTERS)
def test_texture_golden_fixture(filter_mode, boundary):
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "texture.npz").items()}
    mip = "mipmap" in filter_mode
    key = f"{filter_mode}/{boundary}"

    def fn(t, c, d, b):
        return hip.texture(t, c, d if mip else None, filter_mode, boundary, None,
                           mip_level_bias=b if mip else None)

    outs, grads = grads_of(fn, [g["tex"], g["uv"], g["uv_da"], g["bias"]], [g["weights"]],
                           "cuda")
    assert rel_error(outs[0], g[f"{key}/out"]) < VALUE_TOL
    names = ("tex", "uv", "uv_da", "bias")
    assert_grads_close(grads, [g[f"{key}/grad_{n}"] for n in names])


@pytest.mark.parametrize("boundary", BOUNDARIES)
@pytest.mark.parametrize("filter_mode", FILTERS)
def test_texture_gradients(filter_mode, boundary):
    tex, uv, uv_da = tex_scene(channels=4, seed=1)
    weights = torch.randn(2, 20, 24, 4, generator=torch.Generator().manual_seed(2))
    mip = "mipmap" in filter_mode
    ref = grads_of(lambda t, c, d: R.texture(t, c, d if mip else None, filter_mode, boundary,
                                             None), [tex, uv, uv_da], [weights], "cpu")
    ours = grads_of(lambda t, c, d: hip.texture(t, c, d if mip else None, filter_mode, boundary,
                                                None), [tex, uv, uv_da], [weights], "cuda")
    assert rel_error(ours[0][0], ref[0][0]) < VALUE_TOL
    assert_grads_close(ours[1], ref[1])


@pytest.mark.parametrize("boundary", ["wrap", "clamp", "zero"])
@pytest.mark.parametrize("filter_mode", FILTERS)
@pytest.mark.parametrize("channels", [1, 3, 4, 6])
def test_texture_gradients_smooth_mapping(filter_mode, boundary, channels):
    # uv varies smoothly over the image, so a workgroup's taps stay within small windows of the
    # texture that it accumulates in LDS; the mapping crosses the wrap seam and the texture's
    # edges (windows that do not fit, taps added to global memory directly), and the footprint
    # (hence the level) grows across the image. Six channels take two passes.
    gen = torch.Generator().manual_seed(11)
    H, W = 72, 88
    tex = torch.randn(1, 64, 48, channels, generator=gen)
    yy, xx = torch.meshgrid(torch.arange(H, dtype=torch.float32),
                            torch.arange(W, dtype=torch.float32), indexing="ij")
    scale = 0.6 + 2.5 * xx / W  # texels per pixel grows left to right
    u = -0.15 + xx * scale / 48 + 0.02 * torch.sin(yy / 5)
    v = -0.1 + yy * 0.9 / 64 + 0.01 * torch.cos(xx / 7)
    uv = torch.stack([u, v], -1)[None].repeat(2, 1, 1, 1)
    uv[1] = uv[1].flip(1) * 0.7 + 0.2
    da = torch.stack([scale / 48, 0.002 * torch.ones_like(u), 0.001 * torch.ones_like(u),
                      0.9 / 64 * torch.ones_like(u)], -1)[None].repeat(2, 1, 1, 1)
    mip = "mipmap" in filter_mode
    weights = torch.randn(2, H, W, channels, generator=gen)
    ref = grads_of(lambda t, c, d: R.texture(t, c, d if mip else None, filter_mode, boundary,
                                             None), [tex, uv, da], [weights], "cpu")
    ours = grads_of(lambda t, c, d: hip.texture(t, c, d if mip else None, filter_mode,
                                                boundary, None), [tex, uv, da], [weights], "cuda")
    assert rel_error(ours[0][0], ref[0][0]) < VALUE_TOL
    assert_grads_close(ours[1], ref[1])


@pytest.mark.parametrize("pattern", ["constant", "magnified", "mixed"])
@pytest.mark.parametrize("filter_mode", FILTERS)
def test_texture_gradients_where_pixels_share_texels(filter_mode, pattern):
    tex, uv, uv_da = tex_scene(channels=3, seed=5)
    if pattern == "constant":
        uv = torch.full_like(uv, 0.3)
    elif pattern == "magnified":
        uv = uv / 16 + 0.4
    else:
        uv[:, ::2] = 0.0
    mip = "mipmap" in filter_mode
    grads = []
    for fn, device in ((hip.texture, "cuda"), (R.texture, "cpu")):
        t = tex.clone().to(device).requires_grad_(True)
        fn(t, uv.to(device), uv_da.to(device) if mip else None, filter_mode, "clamp",
           None).sum().backward()
        grads.append(t.grad.cpu())
    assert_grads_close(grads[:1], grads[1:])


@pytest.mark.parametrize("max_mip_level", [0, 2])
def test_texture_max_mip_level(max_mip_level):
    tex, uv, uv_da = tex_scene()
    ref = R.texture(tex, uv, uv_da * 4, "linear-mipmap-linear", "wrap", max_mip_level)
    out = hip.texture(tex.cuda(), uv.cuda(), (uv_da * 4).cuda(), "linear-mipmap-linear",
                      "wrap", max_mip_level).cpu()
    assert rel_error(out, ref) < VALUE_TOL


@pytest.mark.parametrize("max_mip_level", [0, 1, 2, 9])
@pytest.mark.parametrize("filter_mode", ["linear-mipmap-linear", "linear-mipmap-nearest"])
def test_cube_texture_max_mip_level(max_mip_level, filter_mode):
    # A limited chain on a cube map (each face 16x16, so 9 is past the 1x1 level), with a bias:
    # values and every gradient against the oracle.
    gen = torch.Generator().manual_seed(11 + max_mip_level)
    tex = torch.rand(1, 6, 16, 16, 3, generator=gen)
    dirs = torch.randn(2, 9, 11, 3, generator=gen)
    dirs_da = torch.randn(2, 9, 11, 6, generator=gen) * 0.3
    bias = torch.rand(2, 9, 11, generator=gen) * 2.5
    weights = torch.randn(2, 9, 11, 3, generator=gen)

    def run(fn):
        return lambda t, d, dd, b: fn(t, d, dd, filter_mode, "cube", max_mip_level,
                                      mip_level_bias=b)

    outs, grads = grads_of(run(hip.texture), [tex, dirs, dirs_da, bias], [weights], "cuda")
    e_outs, e_grads = grads_of(run(R.texture), [tex, dirs, dirs_da, bias], [weights], "cpu")
    assert rel_error(outs[0], e_outs[0]) < VALUE_TOL
    assert_grads_close(grads, e_grads)


@pytest.mark.parametrize("size", [(16, 16), (5, 7), (1, 13), (37, 50)])
def test_mip_chain_matches_oracle(size):
    tex = torch.randn(2, *size, 3, generator=torch.Generator().manual_seed(3))
    ref = R.texture_construct_mip(tex, None)
    ours = hip.texture_construct_mip(tex.cuda(), None)
    assert len(ours) == len(ref)
    for a, b in zip(ours, ref):
        assert a.shape == b.shape
        assert rel_error(a.cpu(), b) < VALUE_TOL
    # Adjoint: gradient of a weighted sum of every level.
    weights = [torch.randn(l.shape, generator=torch.Generator().manual_seed(i))
               for i, l in enumerate(ref)]
    grads = []
    for fn, device in ((hip.texture_construct_mip, "cuda"), (R.texture_construct_mip, "cpu")):
        t = tex.clone().to(device).requires_grad_(True)
        sum((l * w.to(device)).sum() for l, w in zip(fn(t, None), weights)).backward()
        grads.append(t.grad.cpu())
    torch.testing.assert_close(grads[0], grads[1], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("shape", [(2, 64, 128, 4), (1, 96, 160, 8), (1, 6, 32, 32, 3),
                                   (1, 256, 256, 4)])
def test_mip_chain_tile_stages(shape):
    """Sizes divisible by 2^G go through tile stages of up to six levels, the rest level by
    level: 64x128 ends in 1x2 -> 1x1, 96x160 leaves 3x5 after five halvings, a cube map
    stages each face, 256x256 runs a full six-level stage then two more."""
    tex = torch.randn(*shape, generator=torch.Generator().manual_seed(5))
    ref = R.texture_construct_mip(tex, None)
    ours = hip.texture_construct_mip(tex.cuda(), None)
    assert len(ours) == len(ref)
    for a, b in zip(ours, ref):
        assert a.shape == b.shape
        assert rel_error(a.cpu(), b) < VALUE_TOL
    weights = [torch.randn(l.shape, generator=torch.Generator().manual_seed(i))
               for i, l in enumerate(ref)]
    grads = []
    for fn, device in ((hip.texture_construct_mip, "cuda"), (R.texture_construct_mip, "cpu")):
        t = tex.clone().to(device).requires_grad_(True)
        sum((l * w.to(device)).sum() for l, w in zip(fn(t, None), weights)).backward()
        grads.append(t.grad.cpu())
    torch.testing.assert_close(grads[0], grads[1], atol=1e-5, rtol=1e-5)


def test_texture_through_public_api_with_mip_stack():
    tex, uv, uv_da = tex_scene(tex_batch=1, channels=3, seed=7)
    stack = dr.texture_construct_mip(tex.cuda())
    out = dr.texture(tex.cuda(), uv.cuda(), uv_da.cuda(), mip=stack)
    ref = R.texture(tex, uv, uv_da, "linear-mipmap-linear", "wrap", None)
    assert rel_error(out.cpu(), ref) < VALUE_TOL
    again = dr.texture(tex.cuda(), uv.cuda(), uv_da.cuda(), mip=stack)
    assert torch.equal(again, out)


def test_texture_special_coordinates_golden():
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "texture.npz").items()}
    for boundary in BOUNDARIES:
        for filter_mode in ("nearest", "linear"):
            out = hip.texture(g["tex"][:1].cuda(), g["special/uv"].cuda(), None, filter_mode,
                              boundary, None).cpu()
            expected = g[f"special/{filter_mode}/{boundary}"]
            assert torch.equal(out.isnan(), expected.isnan()), (filter_mode, boundary)
            assert rel_error(out.nan_to_num(), expected.nan_to_num()) < VALUE_TOL


@pytest.mark.parametrize("filter_mode", ["nearest", "linear", "linear-mipmap-linear"])
def test_cube_map_golden_fixture(filter_mode):
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "texture.npz").items()}
    mip = "mipmap" in filter_mode

    def fn(t, d, dd):
        return hip.texture(t, d, dd if mip else None, filter_mode, "cube", None)

    outs, grads = grads_of(fn, [g["cube/tex"], g["cube/dirs"], g["cube/dirs_da"]],
                           [g["cube/weights"]], "cuda")
    assert rel_error(outs[0], g[f"cube/{filter_mode}/out"]) < VALUE_TOL
    assert_grads_close(grads, [g[f"cube/{filter_mode}/grad_{n}"] for n in ("tex", "dirs",
                                                                           "dirs_da")])


# ---- antialias -------------------------------------------------------------------------------


def aa_scene(seed=0, channels=3, batch=2, **mesh):
    pos, tri = random_mesh(60, torch.Generator().manual_seed(seed), batch=batch, **mesh)
    rast, _ = R.rasterize(pos, tri, (48, 64), True)
    gen = torch.Generator().manual_seed(seed + 1)
    color = torch.rand(batch, 48, 64, channels, generator=gen)
    weights = torch.randn(batch, 48, 64, channels, generator=gen)
    return pos, tri, rast, color, weights


def test_edge_neighbours_and_silhouettes_golden():
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "antialias.npz").items()}
    nbr = hip.edge_neighbours(g["sil/tri"].cuda()).cpu()
    assert torch.equal(nbr.long(), g["sil/neighbours"])
    mask = hip.silhouette_mask(g["sil/pos"].cuda(), g["sil/tri"].cuda(), nbr.cuda()).cpu()
    bits = torch.stack([(mask >> k) & 1 for k in range(3)], -1).bool()
    assert torch.equal(bits, g["sil/silhouette"])


def test_edge_neighbours_of_a_closed_mesh():
    from diffrast_amd.workloads import icosphere

    _, tri = icosphere(3)
    nbr = hip.edge_neighbours(tri.cuda()).cpu()
    assert torch.equal(nbr.long(), R.edge_neighbours(tri))


@pytest.mark.parametrize("channels", [1, 3, 4, 20])
@pytest.mark.parametrize("mesh", [{}, {"w_range": (-1.0, 2.0)}, {"z_range": 2.0, "xy_range": 3.0}])
def test_antialias_matches_oracle(channels, mesh):
    pos, tri, rast, color, weights = aa_scene(channels=channels, **mesh)
    ref = grads_of(lambda c, p: R.antialias(c, rast, p, tri, 1.0), [color, pos], [weights], "cpu")
    ours = grads_of(lambda c, p: hip.antialias(c, rast.cuda(), p, tri.cuda(), 1.0),
                    [color, pos], [weights], "cuda")
    assert (ref[0][0] != color).any(), "the scene should have silhouettes to blend"
    assert rel_error(ours[0][0], ref[0][0]) < VALUE_TOL
    assert rel_error(ours[1][0], ref[1][0]) < VALUE_TOL
    # Position gradients: vertices near the camera plane have huge gradients whose float32
    # rounding differs between implementations; 1e-4 of the largest one.
    assert_grads_close([ours[1][1]], [ref[1][1]])


@pytest.mark.parametrize("channels,size", [(3, (100, 120)), (4, (100, 120)), (3, (75, 101))])
def test_antialias_small_objects_in_large_images(channels, size):
    # A few small triangles in 100 x 120 images: most 16 x 16 tiles hold no active pair and copy
    # colour and gradient as whole tiles without reading pair records; the active ones sit next
    # to them, with pairs across tile borders (a tile's left and upper neighbours' records). At
    # 75 x 101 with 3 channels the tiles' rows are not 16-byte aligned (the per-float copy).
    gen = torch.Generator().manual_seed(41)
    pos, tri = tiny_mesh(12, gen, 0.18, batch=3)
    rast, _ = R.rasterize(pos, tri, size, True)
    color = torch.rand(3, *size, channels, generator=gen)
    weights = torch.randn(3, *size, channels, generator=gen)
    ref = grads_of(lambda c, p: R.antialias(c, rast, p, tri, 1.0), [color, pos], [weights], "cpu")
    ours = grads_of(lambda c, p: hip.antialias(c, rast.cuda(), p, tri.cuda(), 1.0),
                    [color, pos], [weights], "cuda")
    assert (ref[0][0] != color).any() and (rast[..., 3] == 0).float().mean() > 0.5
    assert rel_error(ours[0][0], ref[0][0]) < VALUE_TOL
    assert rel_error(ours[1][0], ref[1][0]) < VALUE_TOL
    assert_grads_close([ours[1][1]], [ref[1][1]])


def test_antialias_golden_fixtures():
    g = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "antialias.npz").items()}
    for name in ("plain", "crossing", "boost"):
        boost = float(g[f"{name}/boost"])
        rast, tri = g[f"{name}/rast"], g[f"{name}/tri"]
        outs, grads = grads_of(lambda c, p: hip.antialias(c, rast.cuda(), p, tri.cuda(), boost),
                               [g[f"{name}/color"], g[f"{name}/pos"]], [g[f"{name}/weights"]],
                               "cuda")
        assert rel_error(outs[0], g[f"{name}/out"]) < VALUE_TOL, name
        assert_grads_close(grads, [g[f"{name}/grad_color"], g[f"{name}/grad_pos"]])


def test_antialias_shared_pos_and_straight_edge_area():
    edge = 0.3
    pos = torch.tensor([[-2.0, -2.0, 0.0, 1.0], [edge, -2.0, 0.0, 1.0], [edge, 2.0, 0.0, 1.0],
                        [-2.0, 2.0, 0.0, 1.0]])
    tri = torch.tensor([[0, 1, 2], [0, 2, 3]], dtype=torch.int32)
    ctx = dr.RasterizeContext("cuda")
    rast, _ = dr.rasterize(ctx, pos[None].cuda(), tri.cuda(), (16, 24))
    cov = (rast[..., 3:] > 0).float()
    out = dr.antialias(cov, rast, pos.cuda(), tri.cuda())
    torch.testing.assert_close(out.sum().cpu(), torch.tensor(16 * (edge + 1) * 24 / 2))


def test_topology_hash_through_public_api():
    pos, tri, rast, color, _ = aa_scene(seed=3)
    tri_gpu = tri.cuda()
    topo = dr.antialias_construct_topology_hash(tri_gpu)
    a = dr.antialias(color.cuda(), rast.cuda(), pos.cuda(), tri_gpu, topology_hash=topo)
    b = dr.antialias(color.cuda(), rast.cuda(), pos.cuda(), tri_gpu)
    assert torch.equal(a, b)


# ---- argument types at the backend boundary --------------------------------------------------


def test_backend_refuses_types_its_kernels_do_not_compute_in():
    attr, rast, db, tri = interp_scene(3, "shared")
    with pytest.raises(TypeError, match="tri"):
        hip.interpolate(attr.cuda(), rast.cuda(), tri.long().cuda(), None, [])
    with pytest.raises(TypeError, match="attr"):
        hip.interpolate(attr.half().cuda(), rast.cuda(), tri.cuda(), None, [])
    pos, tri2 = random_mesh(4, torch.Generator().manual_seed(0))
    with pytest.raises(TypeError, match="tri"):
        hip.rasterize(pos.cuda(), tri2.long().cuda(), (8, 8), True)
    with pytest.raises(TypeError, match="pos"):
        hip.rasterize(pos.half().cuda(), tri2.cuda(), (8, 8), True)
    tex, uv, uv_da = tex_scene()
    with pytest.raises(TypeError, match="uv"):
        hip.texture(tex.cuda(), uv.half().cuda(), None, "linear", "wrap", None)
