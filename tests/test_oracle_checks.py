"""The oracle against checks that do not come from the reference's code.

Integer-exact coverage of lattice meshes, slivers of known area, float64 screen-space
rasterization, closed forms of interpolation and filtering, Fraction-exact mip weights, a
brute-force cube sampler that finds neighbouring texels by projection, exact antialiased areas
and finite differences. Each is chosen so that a plausible mistake in the oracle (a swapped
operand, a dropped term, a wrong tie rule) fails it.
"""

import itertools
import math
from fractions import Fraction

import pytest
import torch

from helpers import tiny_mesh
from oracle import cube as Q
from oracle import reference as R

QUAD = torch.tensor([[0, 1, 2], [0, 2, 3]], dtype=torch.int32)


def ids(pos, tri, res, layers=1):
    state, out = None, []
    for _ in range(layers):
        rast, _, state = R.rasterize_layer(pos, tri, res, True, state)
        out.append(rast[..., 3].long() - 1)
    return out if layers > 1 else out[0]


def lattice(cols, rows, res, w=1.0, z=0.0, dtype=torch.float32):
    height, width = res
    x = (cols.to(dtype) * 2 + 1) / width - 1
    y = (rows.to(dtype) * 2 + 1) / height - 1
    w = torch.as_tensor(w, dtype=dtype).expand(x.shape)
    return torch.stack([x * w, y * w, z * w, w], -1)[None]


def integer_owner(cols, rows, tri, res):
    """Coverage of lattice triangles in integer arithmetic with the fill rule as an
    infinitesimal shift of the sample towards +x, then (much smaller) +y."""
    height, width = res
    v = torch.stack([cols, rows], -1).long()[tri.long()]  # [T, 3, 2]
    px = torch.arange(width).view(1, 1, width)
    py = torch.arange(height).view(1, height, 1)
    big = 1 << 13
    inside, area = [], 0
    for k in range(3):
        a, b = v[:, (k + 1) % 3], v[:, (k + 2) % 3]
        ax, ay = a[:, 0, None, None], a[:, 1, None, None]
        bx, by = b[:, 0, None, None], b[:, 1, None, None]
        e = (ax - px) * (by - py) - (bx - px) * (ay - py)
        area = area + e
        # d e / d px = ay - by, d e / d py = bx - ax
        inside.append((e * big + (ay - by)) * big + (bx - ax))
    sign = area.sign()
    cover = torch.stack([s * sign > 0 for s in inside]).all(0)
    count = cover.sum(0)
    return torch.where(count > 0, cover.long().argmax(0), -1), count


# ---- rasterize -------------------------------------------------------------------------------


@pytest.mark.parametrize("size", [8, 100, 255])
def test_quad_diagonal_belongs_to_the_triangle_on_its_right(size):
    pos = torch.tensor([[[-1.0, -1.0, 0.0, 1.0], [1.0, -1.0, 0.0, 1.0], [1.0, 1.0, 0.0, 1.0],
                         [-1.0, 1.0, 0.0, 1.0]]])
    row, col = torch.meshgrid(torch.arange(size), torch.arange(size), indexing="ij")
    assert torch.equal(ids(pos, QUAD, (size, size))[0], torch.where(col >= row, 0, 1))


@pytest.mark.parametrize("order", [[0, 1, 2, 3], [3, 2, 1, 0], [1, 2, 3, 0]])
def test_rectangle_owns_left_and_top_edges(order):
    cols = torch.tensor([5, 17, 17, 5])[order]
    rows = torch.tensor([3, 3, 14, 14])[order]
    got = ids(lattice(cols, rows, (20, 24), w=2.5), QUAD, (20, 24))[0] >= 0
    expected = torch.zeros(20, 24, dtype=torch.bool)
    expected[3:14, 5:17] = True
    assert torch.equal(got, expected)


def test_fill_rule_matches_integer_coverage():
    res = (40, 48)
    gen = torch.Generator().manual_seed(0)
    for _ in range(30):
        col, row = torch.randint(18, 24, (2,), generator=gen).tolist()
        dx = (3, 5, 7, 9, 11)[int(torch.randint(5, (1,), generator=gen))]
        dy = (2, 4, 8, 16)[int(torch.randint(4, (1,), generator=gen))]
        sx, sy = (torch.randint(0, 2, (2,), generator=gen) * 2 - 1).tolist()
        cols = torch.tensor([col, col + sx * dx, col])
        rows = torch.tensor([row, row, row + sy * dy])
        tri = torch.tensor([torch.randperm(3, generator=gen).tolist()], dtype=torch.int32)
        w = torch.rand(3, generator=gen) + 0.5
        expected, _ = integer_owner(cols, rows, tri, res)
        assert torch.equal(ids(lattice(cols, rows, res, w=w), tri, res)[0], expected)


def test_shared_edges_cover_their_union_once():
    res = (36, 40)
    gen = torch.Generator().manual_seed(3)
    for _ in range(20):
        a, b = torch.randint(8, 28, (2, 2), generator=gen) // 4 * 4 + 2
        along = b - a
        if not along.any():
            continue
        normal = torch.stack([-along[1], along[0]])
        c = a + normal + torch.randint(-3, 4, (2,), generator=gen)
        d = b - normal + torch.randint(-3, 4, (2,), generator=gen)
        cols, rows = torch.stack([a, b, c, d]).unbind(-1)
        tri = torch.tensor([[0, 1, 2], [1, 0, 3]], dtype=torch.int32)
        pos = lattice(cols, rows, res, w=torch.rand(4, generator=gen) + 0.5)
        first, second = ids(pos, tri, res, layers=2)
        alone = [ids(pos, tri[k:k + 1], res) >= 0 for k in (0, 1)]
        assert not (alone[0] & alone[1]).any()
        assert torch.equal(alone[0] | alone[1], first >= 0)
        assert (second == -1).all()


@pytest.mark.parametrize("half_width", [2.0 ** -5, 0.5])
@pytest.mark.parametrize(("steps", "drawn"), [(4, False), (16, False), (18, True), (64, True)])
def test_area_tolerance_is_two_epsilons(half_width, steps, drawn):
    # A sliver around the centre of pixel (8, 8) of 16x16 whose area there is 2 * steps / 17
    # epsilons of its terms; every value the test computes is exact.
    centre, step = 0.0625, 2.0 ** -27
    xy = [[-half_width, -steps * step], [half_width, -steps * step], [0.0, steps * step]]
    pos = torch.tensor([[[centre + x, centre + y, 0.0, 1.0] for x, y in xy]])
    got = ids(pos, torch.tensor([[0, 1, 2]], dtype=torch.int32), (16, 16))
    assert (got[0, 8, 8] == 0) == drawn
    assert drawn or (got == -1).all()


def test_degenerate_triangles_are_not_drawn():
    gen = torch.Generator().manual_seed(0)
    ends = torch.randint(-9, 10, (3000, 2, 2), generator=gen).float() / 10
    xy = torch.cat([ends, ends.mean(1, keepdim=True)], 1).reshape(1, -1, 2)
    w = 1 + torch.rand(1, xy.shape[1], 1, generator=gen)
    pos = torch.cat([xy * w, torch.zeros_like(w), w], -1)
    tri = torch.arange(pos.shape[1], dtype=torch.int32).view(-1, 3)
    assert (ids(pos, tri, (50, 50)) == -1).all()
    i, j = torch.randint(0, pos.shape[1], (2, 500), generator=gen)
    rep = torch.cat([torch.stack([i, i, j], -1), torch.stack([i, j, i], -1)]).int()
    assert (ids(pos, rep, (50, 50)) == -1).all()


@pytest.mark.parametrize("exponent", [-40, -10, 10, 40])
def test_coverage_is_invariant_to_clip_space_scale(exponent):
    pos, tri = tiny_mesh(80, torch.Generator().manual_seed(5), 0.3)
    assert torch.equal(ids(pos * 2.0 ** exponent, tri, (48, 48)), ids(pos, tri, (48, 48)))


@pytest.mark.parametrize("value", [float("nan"), float("inf"), -float("inf")])
def test_non_finite_vertices_are_culled(value):
    pos = torch.tensor([[[-0.8, -0.8, 0.5, 1.0], [0.8, -0.8, 0.5, 1.0], [0.8, 0.8, 0.5, 1.0],
                         [-0.8, 0.8, 0.5, 1.0], [-0.5, -0.5, -0.5, 1.0], [0.5, -0.5, -0.5, 1.0],
                         [0.5, 0.5, -0.5, 1.0], [-0.5, 0.5, -0.5, 1.0]]])
    tri = torch.cat([QUAD, QUAD + 4])
    behind = ids(pos, tri[:2], (24, 24))
    broken = pos.clone()
    broken[0, 6, 1] = value  # vertex 6 is in both front triangles
    got = ids(broken, tri, (24, 24))
    assert torch.equal(got, behind)


def screen_space(pos, tri, res, margin=1e-4):
    """Float64 rasterizer in screen space for triangles in front: ids and ambiguous pixels."""
    height, width = res
    p = pos.double()
    ndc = p[..., :3] / p[..., 3:]
    v = ndc[:, tri.long()][:, :, None, None]  # [B, T, 1, 1, 3, 3]
    px = ((torch.arange(width, dtype=torch.float64) * 2 + 1) / width - 1).view(1, width)
    py = ((torch.arange(height, dtype=torch.float64) * 2 + 1) / height - 1).view(height, 1)

    def edge(i, j):
        return (v[..., j, 0] - v[..., i, 0]) * (py - v[..., i, 1]) - (
            v[..., j, 1] - v[..., i, 1]) * (px - v[..., i, 0])

    lam = torch.stack([edge(1, 2), edge(2, 0), edge(0, 1)], -1)
    lam = lam / lam.sum(-1, keepdim=True)
    inside = (lam >= 0).all(-1)
    depth = torch.where(inside, (lam * v[..., 2]).sum(-1), torch.inf)
    best, which = depth.min(1)
    got = torch.where(best.isinf(), -1, which)
    near = (lam.abs().min(-1).values < margin).any(1)
    sorted_depth = depth.sort(1).values
    tie = (sorted_depth[:, 1] - sorted_depth[:, 0]) < margin
    return got, near | tie


@pytest.mark.parametrize("size", [0.3, 0.03])
def test_small_triangles_match_a_float64_screen_space_rasterizer(size):
    pos, tri = tiny_mesh(400, torch.Generator().manual_seed(3), size)
    expected, ambiguous = screen_space(pos, tri, (56, 64))
    got = ids(pos, tri, (56, 64))
    assert (~ambiguous).float().mean() > 0.9 and (expected[~ambiguous] >= 0).sum() > 20
    assert torch.equal(got[~ambiguous], expected[~ambiguous])


def test_depth_layers_are_ordered_and_equal_depths_go_by_index():
    tri = torch.tensor([[6, 7, 8], [0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    flat = [[-0.2, -0.2, 0.25, 1.0], [0.2, -0.2, 0.25, 1.0], [0.0, 0.2, 0.25, 1.0]]
    layers = ids(torch.tensor([flat * 3]), tri, (8, 8), layers=4)
    covered = layers[0] >= 0
    assert covered.any()
    for layer, expected in zip(layers, [0, 1, 2, -1]):
        assert (layer[covered] == expected).all()
    gen = torch.Generator().manual_seed(1)
    pos, tri = tiny_mesh(60, gen, 0.8)
    state = None
    previous = None
    for _ in range(3):
        rast, _, state = R.rasterize_layer(pos, tri, (24, 24), True, state)
        if previous is not None:
            both = (rast[..., 3] > 0) & (previous[..., 3] > 0)
            assert (rast[..., 2][both] >= previous[..., 2][both]).all()
        previous = rast


def test_visibility_at_listed_pixels_equals_the_full_grid():
    # visible_at is the brute force behind the full-size checks: every pixel of a batched
    # mesh, over three depth layers, must equal visible_triangles there.
    gen = torch.Generator().manual_seed(4)
    pos, tri = tiny_mesh(80, gen, 0.6, batch=2)
    height, width = 20, 28
    b, row, col = (t.reshape(-1) for t in torch.meshgrid(
        torch.arange(2), torch.arange(height), torch.arange(width), indexing="ij"))
    px, py = R.pixel_centres(height, width, pos)
    full, listed = None, None
    for _ in range(3):
        full = R.visible_triangles(pos, tri, px, py, full)
        listed = R.visible_at(pos, tri, height, width, b, row, col, listed)
        assert torch.equal(listed[1], full[1].reshape(-1))
        assert torch.equal(listed[0], full[0].reshape(-1))
    assert (full[1] >= 0).any()


def test_resolve_closed_forms_and_rast_db_finite_differences():
    pos = torch.tensor([[[-0.8, -0.6, 0.2, 1.0], [1.2, -0.9, 0.5, 2.0], [0.1, 1.5, -0.3, 1.5]]],
                       dtype=torch.float64)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    res = (16, 24)
    rast, rast_db = R.rasterize(pos, tri, res)
    b = rast[..., :2]
    covered = rast[..., 3] > 0
    bary = torch.cat([b, 1 - b.sum(-1, keepdim=True)], -1)  # perspective-correct weights
    p = pos[0]
    xw = (bary[..., :, None] * p[None, None, None]).sum(-2)
    px = ((torch.arange(res[1], dtype=torch.float64) * 2 + 1) / res[1] - 1)
    py = ((torch.arange(res[0], dtype=torch.float64) * 2 + 1) / res[0] - 1)
    # The homogeneous point interpolated with b projects onto the pixel centre.
    torch.testing.assert_close((xw[..., 0] / xw[..., 3])[covered],
                               px.expand(1, res[0], -1)[covered])
    torch.testing.assert_close((xw[..., 1] / xw[..., 3])[covered],
                               py[:, None].expand(1, -1, res[1])[covered])
    torch.testing.assert_close(rast[..., 2][covered], (xw[..., 2] / xw[..., 3])[covered])
    # rast_db against a sub-pixel finite difference of the same formulas.
    tri_id = rast[..., 3].long() - 1
    h = 1e-6
    for axis, chans in ((0, (0, 2)), (1, (1, 3))):
        shift = torch.zeros(4, dtype=torch.float64)
        shift[axis] = h * (2 / res[1 - axis])
        plus, _ = R.rasterize_from_ids(pos - shift * pos[..., 3:], tri, tri_id, True)
        minus, _ = R.rasterize_from_ids(pos + shift * pos[..., 3:], tri, tri_id, True)
        fd = (plus[..., :2] - minus[..., :2]) / (2 * h)
        torch.testing.assert_close(rast_db[..., list(chans)][covered], fd[covered],
                                   rtol=1e-5, atol=1e-7)


def test_resolve_gradcheck():
    pos = torch.tensor([[[-0.8, -0.6, 0.2, 1.0], [1.2, -0.9, 0.5, 2.0], [0.1, 1.5, -0.3, 1.5]]],
                       dtype=torch.float64, requires_grad=True)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    rast, _ = R.rasterize(pos.detach(), tri, (6, 6))
    tri_id = rast[..., 3].long() - 1
    assert torch.autograd.gradcheck(lambda p: R.rasterize_from_ids(p, tri, tri_id, True), (pos,))


# ---- interpolate -----------------------------------------------------------------------------


def test_interpolate_identity_and_exact_affine_derivatives():
    pos = torch.tensor([[[-1.0, -1.0, 0.0, 1.0], [3.0, -1.0, 0.0, 1.0], [-1.0, 3.0, 0.0, 1.0]]])
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    rast, rast_db = R.rasterize(pos, tri, (8, 8))
    out, _ = R.interpolate(torch.eye(3), rast, tri, None, [])
    torch.testing.assert_close(out.sum(-1), torch.ones(1, 8, 8))
    torch.testing.assert_close(out[..., 0], rast[..., 0])
    attr = torch.tensor([[0.0, 1.0], [4.0, -2.0], [1.0, 3.0]])
    out, out_da = R.interpolate(attr, rast, tri, rast_db, [0, 1])
    for c in range(2):
        torch.testing.assert_close(out_da[0, :, :-1, 2 * c], out[0, :, 1:, c] - out[0, :, :-1, c])
        torch.testing.assert_close(out_da[0, :-1, :, 2 * c + 1], out[0, 1:, :, c] - out[0, :-1, :, c])
    _, some = R.interpolate(torch.randn(3, 4), rast, tri, rast_db, [3, 1])
    assert some.shape == (1, 8, 8, 4)


# ---- texture ---------------------------------------------------------------------------------


def texel_centres(h, w):
    u = (torch.arange(w, dtype=torch.float32) + 0.5) / w
    v = (torch.arange(h, dtype=torch.float32) + 0.5) / h
    return torch.stack(torch.meshgrid(u, v, indexing="xy"), -1)[None]


def footprint(uv, texels, size):
    da = uv.new_zeros(*uv.shape[:3], 4)
    da[..., 0] = texels / size
    da[..., 3] = texels / size
    return da


TEX = torch.randn(1, 6, 8, 3, generator=torch.Generator().manual_seed(0))


@pytest.mark.parametrize("boundary", ["wrap", "clamp", "zero"])
@pytest.mark.parametrize("filter_mode", ["nearest", "linear"])
def test_texel_centres_return_texels(filter_mode, boundary):
    out = R.texture(TEX, texel_centres(6, 8), None, filter_mode, boundary, None)
    torch.testing.assert_close(out, TEX)


def test_boundaries_and_affine_reproduction():
    uv = torch.tensor([[[[0.0, 0.5 / 6]]]])
    torch.testing.assert_close(R.texture(TEX, uv, None, "linear", "wrap", None)[0, 0, 0],
                               (TEX[0, 0, 0] + TEX[0, 0, -1]) / 2)
    uv = torch.tensor([[[[-3.0, 0.5 / 6], [0.5 / 8, 7.0]]]])
    torch.testing.assert_close(R.texture(TEX, uv, None, "linear", "clamp", None)[0, 0],
                               torch.stack([TEX[0, 0, 0], TEX[0, -1, 0]]))
    uv = torch.tensor([[[[-3.0, 0.5], [0.0, 0.5 / 6]]]])
    out = R.texture(TEX, uv, None, "linear", "zero", None)
    torch.testing.assert_close(out[0, 0, 0], torch.zeros(3))
    torch.testing.assert_close(out[0, 0, 1], TEX[0, 0, 0] / 2)
    c = texel_centres(5, 7)
    tex = (2 * c[..., :1] - 3 * c[..., 1:] + 0.5).expand(-1, -1, -1, 2).contiguous()
    uv = torch.rand(1, 10, 10, 2, generator=torch.Generator().manual_seed(1))
    uv[..., 0] = 0.5 / 7 + uv[..., 0] * (1 - 1 / 7)
    uv[..., 1] = 0.5 / 5 + uv[..., 1] * (1 - 1 / 5)
    out = R.texture(tex, uv, None, "linear", "clamp", None)
    torch.testing.assert_close(out[..., 0], 2 * uv[..., 0] - 3 * uv[..., 1] + 0.5)


def test_mip_levels_blend_and_bias():
    tex = torch.randn(1, 16, 16, 2, generator=torch.Generator().manual_seed(4))
    uv = torch.rand(1, 4, 4, 2, generator=torch.Generator().manual_seed(5))
    top = R.texture(tex, uv, footprint(uv, 64, 16), "linear-mipmap-linear", "wrap", None)
    torch.testing.assert_close(top, tex.mean((1, 2), keepdim=True).expand_as(top))

    def at_lod(lod):
        return R.texture(TEX, uv, footprint(uv, 2.0 ** lod, 8), "linear-mipmap-linear", "wrap",
                         None)

    torch.testing.assert_close(at_lod(1.25), 0.75 * at_lod(1) + 0.25 * at_lod(2))
    bias = torch.full((1, 4, 4), 1.3)
    shifted = R.texture(TEX, uv, footprint(uv, 1.2, 8), "linear-mipmap-linear", "wrap", None,
                        mip_level_bias=bias)
    scaled = R.texture(TEX, uv, footprint(uv, 1.2 * 2 ** 1.3, 8), "linear-mipmap-linear", "wrap",
                       None)
    torch.testing.assert_close(shifted, scaled)
    const = torch.full((1, 5, 7, 2), 0.25)
    for texels in (1.5, 3.0, 9.0):
        out = R.texture(const, uv, footprint(uv, texels, 7), "linear-mipmap-linear", "wrap", None)
        torch.testing.assert_close(out, torch.full_like(out, 0.25))


def area_weights(n):
    m = (n + 1) // 2
    w = torch.zeros(m, n, dtype=torch.float64)
    for j, i in itertools.product(range(m), range(n)):
        overlap = min(Fraction((j + 1) * n, m), i + 1) - max(Fraction(j * n, m), i)
        w[j, i] = float(max(overlap, 0) / Fraction(n, m))
    return w


@pytest.mark.parametrize("size", [(5, 7), (6, 9), (1, 13), (3, 3), (15, 2)])
def test_mip_chain_equals_exact_area_weights(size):
    tex = torch.randn(2, *size, 2, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    expected = tex
    for level in R.mip_chain(tex, None)[1:]:
        rows, cols = area_weights(expected.shape[1]), area_weights(expected.shape[2])
        if expected.shape[1] == 1:
            rows = torch.ones(1, 1, dtype=torch.float64)
        if expected.shape[2] == 1:
            cols = torch.ones(1, 1, dtype=torch.float64)
        expected = torch.einsum("ri,bijc,sj->brsc", rows, expected, cols)
        torch.testing.assert_close(level, expected, rtol=1e-12, atol=1e-12)


def box_chain(tex, count):
    """The first ``count`` levels of a power-of-two texture (``[..., h, w, c]``: 2D or cube),
    each the mean of 2x2 blocks of the one before, built here independently of the oracle."""
    levels = [tex]
    while len(levels) < count:
        t = levels[-1]
        levels.append((t[..., 0::2, 0::2, :] + t[..., 1::2, 0::2, :] + t[..., 0::2, 1::2, :]
                       + t[..., 1::2, 1::2, :]) / 4)
    return levels


def mip_scene(cube, seed):
    gen = torch.Generator().manual_seed(seed)
    shape = (1, 6, 16, 16, 3) if cube else (1, 16, 16, 3)
    tex = torch.rand(*shape, generator=gen, dtype=torch.float64)
    if cube:
        uv = torch.randn(1, 6, 7, 3, generator=gen, dtype=torch.float64)
        uv_da = torch.randn(1, 6, 7, 6, generator=gen, dtype=torch.float64) * 0.4
    else:
        uv = torch.rand(1, 6, 7, 2, generator=gen, dtype=torch.float64)
        uv_da = torch.randn(1, 6, 7, 4, generator=gen, dtype=torch.float64) * 0.3
    bias = torch.rand(1, 6, 7, generator=gen, dtype=torch.float64) * 3
    return tex, uv, uv_da, bias, "cube" if cube else "wrap"


@pytest.mark.parametrize("cube", [False, True])
def test_max_mip_level_zero_is_the_plain_linear_lookup(cube):
    # With the chain stopped at level 0 the level of detail is clamped to 0: both taps read
    # level 0 and the blend weight is 0, so the result is the non-mipmapped bilinear lookup,
    # whatever the footprint and the bias (reference tests/test_cube.py:354-368).
    tex, uv, uv_da, bias, boundary = mip_scene(cube, 20)
    linear = R.texture(tex, uv, None, "linear", boundary, None)
    for da, b in ((uv_da, None), (uv_da * 50, bias), (None, bias * 4)):
        out = R.texture(tex, uv, da, "linear-mipmap-linear", boundary, 0, mip_level_bias=b)
        assert torch.equal(out, linear)
        nearest_level = R.texture(tex, uv, da, "linear-mipmap-nearest", boundary, 0,
                                  mip_level_bias=b)
        assert torch.equal(nearest_level, linear)


@pytest.mark.parametrize("cube", [False, True])
@pytest.mark.parametrize("k", [1, 2, 3, 9])
def test_max_mip_level_limits_the_chain_to_its_first_levels(cube, k):
    # A chain limited to k holds levels 0..k (fewer when the texture runs out: 16x16 has five),
    # equal to an explicit list of the first k box-filtered levels; a bias far past the top
    # reads the top level alone (reference tests/test_mip.py:119-130, tests/test_cube.py:
    # 354-398).
    tex, uv, uv_da, bias, boundary = mip_scene(cube, 21 + k)
    full = 5
    count = min(k, full - 1) + 1
    chain = R.mip_chain(tex, k)
    explicit = box_chain(tex, count)
    assert len(chain) == count and len(R.texture_construct_mip(tex, k)) == count - 1
    for ours, expect in zip(chain, explicit):
        assert ours.shape == expect.shape
        torch.testing.assert_close(ours, expect, rtol=1e-13, atol=1e-13)
    for mode in ("linear-mipmap-linear", "linear-mipmap-nearest"):
        limited = R.texture(tex, uv, uv_da, mode, boundary, k, mip_level_bias=bias)
        listed = R.texture(tex, uv, uv_da, mode, boundary, None, mip_level_bias=bias,
                           mip=explicit[1:])
        torch.testing.assert_close(limited, listed, rtol=1e-12, atol=1e-12)
        cut = R.texture(tex, uv, uv_da, mode, boundary, k, mip_level_bias=bias,
                        mip=box_chain(tex, full)[1:])
        torch.testing.assert_close(cut, listed, rtol=1e-12, atol=1e-12)
        packed = R.texture(tex, uv, uv_da, mode, boundary, k, mip_level_bias=bias,
                           packed=R.pack(box_chain(tex, full)))
        torch.testing.assert_close(packed, listed, rtol=1e-12, atol=1e-12)
    far = torch.full_like(bias, 40.0)
    top = R.texture(tex, uv, uv_da, "linear-mipmap-linear", boundary, k, mip_level_bias=far)
    alone = R.texture(explicit[-1], uv, None, "linear", boundary, None)
    torch.testing.assert_close(top, alone, rtol=1e-13, atol=1e-13)


# ---- cube maps -------------------------------------------------------------------------------


def brute_force_cube(tex, dirs):
    """Bilinear cube lookup in float64 that finds texels across edges by projecting the 3D
    centre of each tap onto the cube (not by the integer fold); beyond a corner the missing
    tap is the mean of the other three."""
    major = torch.tensor(Q.MAJOR, dtype=torch.float64)
    s_axis = torch.tensor(Q.S_AXIS, dtype=torch.float64)
    t_axis = torch.tensor(Q.T_AXIS, dtype=torch.float64)
    size = tex.shape[2]
    t64 = tex.double()

    def face_of(d):
        a = d.abs()
        axis = 0 if a[0] >= a[1] and a[0] >= a[2] else (1 if a[1] >= a[2] else 2)
        return 2 * axis + int(d[axis] < 0)

    def texel(face, row, col):
        if (row < 0 or row >= size) and (col < 0 or col >= size):
            return None
        sc, tc = (2 * col + 1) / size - 1, (2 * row + 1) / size - 1
        d = major[face] + sc * s_axis[face] + tc * t_axis[face]
        f = face_of(d)
        m = (d * major[f]).sum()
        s = ((d * s_axis[f]).sum() / m + 1) / 2
        t = ((d * t_axis[f]).sum() / m + 1) / 2
        c = min(max(int(math.floor(float(s) * size)), 0), size - 1)
        r = min(max(int(math.floor(float(t) * size)), 0), size - 1)
        return t64[0, f, r, c]

    out = torch.zeros(*dirs.shape[:-1], tex.shape[-1], dtype=torch.float64)
    for index in itertools.product(*(range(n) for n in dirs.shape[:-1])):
        d = dirs[index].double()
        f = face_of(d)
        m = (d * major[f]).sum()
        s = ((d * s_axis[f]).sum() / m + 1) / 2
        t = ((d * t_axis[f]).sum() / m + 1) / 2
        x, y = float(s) * size - 0.5, float(t) * size - 0.5
        c0, r0 = math.floor(x), math.floor(y)
        fx, fy = x - c0, y - r0
        taps = [texel(f, r0 + dr, c0 + dc) for dr, dc in ((0, 0), (0, 1), (1, 0), (1, 1))]
        present = [tp for tp in taps if tp is not None]
        taps = [tp if tp is not None else sum(present) / 3 for tp in taps]
        out[index] = ((1 - fy) * ((1 - fx) * taps[0] + fx * taps[1]) +
                      fy * ((1 - fx) * taps[2] + fx * taps[3]))
    return out


def test_cube_lookup_matches_brute_force_projection():
    gen = torch.Generator().manual_seed(7)
    tex = torch.rand(1, 6, 5, 5, 2, generator=gen)
    dirs = torch.randn(1, 12, 12, 3, generator=gen)
    # Directions on and near face edges and corners.
    dirs[0, 0, :6] = torch.tensor([[1.0, 1.0, 1.0], [1.0, 1.0, 0.3], [1.0, -0.999, 0.2],
                                   [0.0, 1.0, 0.999], [-1.0, 0.5, -1.0], [0.2, -1.0, -1.0]])
    expected = brute_force_cube(tex, dirs)
    got = R.texture(tex, dirs, None, "linear", "cube", None)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-6)


def test_cube_invalid_directions_read_zero():
    tex = torch.rand(1, 6, 4, 4, 1, generator=torch.Generator().manual_seed(8))
    dirs = torch.tensor([[[[0.0, 0.0, 0.0], [float("nan"), 1.0, 0.0], [1e-40, 0.0, 0.0],
                           [0.0, 2.0, 0.0]]]])
    out = R.texture(tex, dirs, None, "linear", "cube", None)
    assert (out[0, 0, :3] == 0).all() and (out[0, 0, 3] != 0).all()


# ---- antialias and adjacency -----------------------------------------------------------------


def half_plane(edge, axis, dtype=torch.float32):
    corners = [[-2.0, -2.0], [edge, -2.0], [edge, 2.0], [-2.0, 2.0]]
    if axis == 1:
        corners = [[y, x] for x, y in corners][::-1]
    return torch.tensor([[[x, y, 0.0, 1.0] for x, y in corners]], dtype=dtype)


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("edge", [-0.5, 0.0625, 0.3, 0.71])
def test_straight_edge_area_is_exact(axis, edge):
    h, w = 16, 24
    pos = half_plane(edge, axis)
    rast, _ = R.rasterize(pos, QUAD, (h, w))
    out = R.antialias((rast[..., 3:] > 0).float(), rast, pos, QUAD)
    size, across = (w, h) if axis == 0 else (h, w)
    torch.testing.assert_close(out.sum(), torch.tensor(across * (edge + 1) * size / 2))


@pytest.mark.parametrize("top", [-0.2, 0.25, 0.9])
def test_slanted_edge_area_is_exact(top):
    h, w, bottom = 16, 24, 0.3
    pos = half_plane(0.0, 0)
    pos[0, 1, 0], pos[0, 2, 0] = bottom - (top - bottom) / 2, top + (top - bottom) / 2
    rast, _ = R.rasterize(pos, QUAD, (h, w))
    out = R.antialias((rast[..., 3:] > 0).float(), rast, pos, QUAD)
    torch.testing.assert_close(out.sum(), torch.tensor(h * ((bottom + top) / 2 + 1) * w / 2))


@pytest.mark.parametrize("axis", [0, 1])
def test_straight_edge_gradient_is_the_edge_length(axis):
    h, w = 16, 24
    pos = half_plane(0.3, axis, torch.float64).requires_grad_(True)
    rast, _ = R.rasterize(pos, QUAD, (h, w))
    R.antialias((rast[..., 3:] > 0).double(), rast, pos, QUAD).sum().backward()
    size, across = (w, h) if axis == 0 else (h, w)
    torch.testing.assert_close(pos.grad[0, [1, 2], axis].sum(),
                               torch.tensor(across * size / 2, dtype=torch.float64))


def test_interior_edges_are_left_alone_and_silhouette_cases():
    pos = half_plane(2.0, 0)
    rast, _ = R.rasterize(pos, QUAD, (12, 12))
    color = torch.stack([rast[..., 3] == 1, rast[..., 3] == 2], -1).float()
    torch.testing.assert_close(R.antialias(color, rast, pos, QUAD), color)
    flat = R.silhouette_edges(half_plane(0.3, 0).double(), QUAD.long())
    diagonal = torch.zeros(2, 3, dtype=torch.bool)
    diagonal[0, 1] = diagonal[1, 2] = True  # edge k is opposite vertex k
    assert torch.equal(flat[0], ~diagonal)
    folded = half_plane(0.3, 0).double()
    folded[0, 3, :2] = torch.tensor([0.5, -1.5])
    sil = R.silhouette_edges(folded, QUAD.long())
    assert sil[0, 0, 1] and sil[0, 1, 2]
    tri = torch.tensor([[0, 1, 2], [0, 2, 3], [0, 2, 4]])
    pos = torch.cat([half_plane(0.3, 0), torch.tensor([[[0.0, 1.0, 0.0, 1.0]]])], 1).double()
    sil = R.silhouette_edges(pos, tri)
    assert sil[0, 0, 1] and sil[0, 1, 2] and sil[0, 2, 2]
    nbr = R.edge_neighbours(QUAD)
    assert nbr.tolist() == [[-1, 5, -1], [-1, -1, 1]]


def test_antialias_gradient_matches_finite_differences():
    pos = torch.tensor([[[-0.8, -0.6, 0.2, 1.0], [1.2, -0.9, 0.5, 2.0], [0.1, 1.5, -0.3, 1.5]]],
                       dtype=torch.float64)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    weights = torch.rand(1, 16, 16, 3, generator=torch.Generator().manual_seed(0),
                         dtype=torch.float64)

    def loss(p):
        rast, _ = R.rasterize(p, tri, (16, 16))
        color = (rast[..., 3:] > 0).double().expand(-1, -1, -1, 3)
        return (R.antialias(color, rast, p, tri) * weights).sum()

    p = pos.clone().requires_grad_(True)
    loss(p).backward()
    eps = 1e-6
    for vertex in range(3):
        for axis in (0, 1, 3):
            step = torch.zeros_like(pos)
            step[0, vertex, axis] = eps
            numeric = (loss(pos + step) - loss(pos - step)) / (2 * eps)
            torch.testing.assert_close(p.grad[0, vertex, axis], numeric, rtol=1e-4, atol=1e-6)


def test_cross_product_rounding_the_silhouettes_rely_on():
    """The reference classifies folds with torch.linalg.cross, whose CPU kernel rounds each
    component as fma(u_i, v_j, -(u_j v_i)); the HIP silhouette pass computes exactly that. A host
    whose torch rounds otherwise would classify near-degenerate folds differently."""
    gen = torch.Generator().manual_seed(3)
    u, v = torch.randn(2, 1, 200_000, 3, generator=gen)
    got = torch.linalg.cross(u, v, dim=-1)
    U, V = u.double(), v.double()
    for k, (i, j) in enumerate(((1, 2), (2, 0), (0, 1))):
        fused = (U[..., i] * V[..., j] - (U[..., j] * V[..., i]).float().double()).float()
        assert torch.equal(got[..., k], fused), k
