"""Code written for the reference (``import diffrast``, ``import diffrast.torch``) or for
nvdiffrast (``install_as_nvdiffrast``) runs unchanged on the HIP backend.

The call patterns are the ones the reference's compatibility tests exercise
(tests/test_compat.py:412-614, README.md:102-131): resolutions as lists, tuples, tensors and
NumPy values, positional arguments, attributes shared across a batched rast, per-face
attributes, a separate uv index buffer, rast edited in place, triangles drawn in chunks, and
non-contiguous inputs to every op. Each is checked against the plain call on the GPU, and the
plain scene's ids and values against the oracle.
"""

import sys

import numpy as np
import pytest
import torch

import diffrast as dr
import diffrast.torch as drt
from helpers import rel_error
from oracle import reference as R

pytestmark = pytest.mark.gpu

RES = (28, 36)


def panel(n=7):
    """A wavy grid of n x n quads with shared vertices, seen from two sides in perspective:
    pos [2, V, 4], tri [2 n^2, 3], uv [V, 2]. No two triangles overlap on screen."""
    t = torch.linspace(-0.85, 0.8, n + 1)
    y, x = torch.meshgrid(t, t, indexing="ij")
    x, y = x.flatten(), y.flatten()
    w = 1.2 + 0.2 * x + 0.15 * y
    z = 0.3 * torch.sin(2.0 * x) * torch.cos(1.5 * y)
    front = torch.stack([x * w, y * w, z * w, w], -1)
    back = front * torch.tensor([-1.0, 1.0, -1.0, 1.0])
    rows = []
    for i in range(n):
        for j in range(n):
            a = i * (n + 1) + j
            rows += [[a, a + 1, a + n + 2], [a, a + n + 2, a + n + 1]]
    uv = torch.stack([(x + 1) / 2, (y + 1) / 2], -1)
    return torch.stack([front, back]), torch.tensor(rows, dtype=torch.int32), uv


def noisy(*shape, seed):
    return torch.rand(*shape, generator=torch.Generator().manual_seed(seed))


def strided(t):
    """The same values in memory that is not contiguous."""
    view = t.repeat_interleave(2, dim=-1)[..., ::2]
    assert not view.is_contiguous()
    return view


@pytest.fixture(scope="module")
def scene():
    pos, tri, uv = panel()
    dev = torch.device("cuda", 0)
    ctx = dr.RasterizeContext(dev)
    rast, rast_db = dr.rasterize(ctx, pos.to(dev), tri.to(dev), RES)
    return dict(ctx=ctx, pos=pos.to(dev), tri=tri.to(dev), uv=uv.to(dev), rast=rast,
                rast_db=rast_db, cpu=(pos, tri, uv))


def test_plain_scene_against_the_oracle(scene):
    pos, tri, uv = scene["cpu"]
    ref, ref_db = R.rasterize(pos, tri, RES)
    assert torch.equal(scene["rast"][..., 3].cpu(), ref[..., 3])
    assert (ref[..., 3] > 0).float().mean() > 0.5
    assert rel_error(scene["rast"].cpu(), ref) < 1e-5
    assert rel_error(scene["rast_db"].cpu(), ref_db) < 1e-5
    out, out_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"], scene["rast_db"],
                                 diff_attrs="all")
    e_out, e_da = R.interpolate(uv, ref, tri, ref_db, [0, 1])
    assert rel_error(out.cpu(), e_out) < 1e-5 and rel_error(out_da.cpu(), e_da) < 1e-5


def test_resolution_forms(scene):
    forms = ([28, 36], (28, 36), torch.tensor([28, 36]), np.array([28, 36]),
             (np.int64(28), np.int32(36)), [np.intp(28), 36], np.zeros(RES).shape)
    for res in forms:
        rast, rast_db = dr.rasterize(scene["ctx"], scene["pos"], scene["tri"], res)
        assert torch.equal(rast, scene["rast"]) and torch.equal(rast_db, scene["rast_db"]), res


def test_positional_arguments(scene):
    rast, rast_db = dr.rasterize(scene["ctx"], scene["pos"], scene["tri"], [28, 36], None, True)
    assert torch.equal(rast, scene["rast"]) and torch.equal(rast_db, scene["rast_db"])
    tex = noisy(1, 16, 16, 3, seed=1).cuda()
    uv, uv_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"], scene["rast_db"], "all")
    out = dr.texture(tex, uv, uv_da, None, None, "linear", "wrap", None)
    assert torch.equal(out, dr.texture(tex, uv, filter_mode="linear", boundary_mode="wrap"))


def test_attributes_shared_across_a_batched_rast(scene):
    attr = noisy(scene["pos"].shape[1], 5, seed=2).cuda()
    shared, _ = dr.interpolate(attr, scene["rast"], scene["tri"])
    single, _ = dr.interpolate(attr[None], scene["rast"], scene["tri"])
    batched, _ = dr.interpolate(attr[None].expand(2, -1, -1), scene["rast"], scene["tri"])
    assert shared.shape == (2, *RES, 5)
    assert torch.equal(shared, single) and torch.equal(shared, batched)


def test_per_face_attributes(scene):
    faces = scene["tri"].shape[0]
    face_tri = torch.arange(faces, dtype=torch.int32, device="cuda")[:, None].repeat(1, 3)
    attr = noisy(faces, 3, seed=3).cuda()
    out, _ = dr.interpolate(attr, scene["rast"], face_tri)
    ids = scene["rast"][..., 3].long()
    expect = attr[(ids - 1).clamp(min=0)] * (ids > 0)[..., None]
    # u a + v a + (1 - u - v) a rounds within a few ulp of a.
    torch.testing.assert_close(out, expect, atol=1e-6, rtol=1e-5)


def test_separate_uv_index_buffer(scene):
    # One uv per triangle corner, as in a mesh whose uv map has seams.
    corner_uv = scene["uv"][scene["tri"].long()].reshape(-1, 2)
    uv_tri = torch.arange(corner_uv.shape[0], dtype=torch.int32, device="cuda").view(-1, 3)
    out, out_da = dr.interpolate(corner_uv, scene["rast"], uv_tri, scene["rast_db"], "all")
    e_out, e_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"], scene["rast_db"],
                                 "all")
    assert torch.equal(out, e_out) and torch.equal(out_da, e_da)


def test_rast_db_without_diff_attrs(scene):
    expect, _ = dr.interpolate(scene["uv"], scene["rast"], scene["tri"])
    for out, out_da in (dr.interpolate(scene["uv"], scene["rast"], scene["tri"],
                                       rast_db=scene["rast_db"]),
                        dr.interpolate(scene["uv"], scene["rast"], scene["tri"],
                                       scene["rast_db"], None)):
        assert torch.equal(out, expect) and out_da.shape == (2, *RES, 0)


def test_rast_edited_in_place(scene):
    expect, _ = dr.interpolate(scene["uv"], scene["rast"], scene["tri"])
    rast = scene["rast"].clone()
    rast[..., :2].clamp_(0, 1)
    out, _ = dr.interpolate(scene["uv"], rast, scene["tri"])
    torch.testing.assert_close(out, expect)


def test_rast_edited_in_place_with_gradients(scene):
    weights = noisy(2, *RES, 2, seed=4).cuda()

    def render(edit):
        pos = scene["pos"].clone().requires_grad_(True)
        rast, rast_db = dr.rasterize(scene["ctx"], pos, scene["tri"], RES)
        rast = edit(rast)
        uv, uv_da = dr.interpolate(scene["uv"], rast, scene["tri"], rast_db, "all")
        out = dr.antialias(uv, rast, pos, scene["tri"])
        ((out * weights).sum() + uv_da.square().sum()).backward()
        return out.detach(), pos.grad

    def in_place(rast):
        rast[..., 3:4] += 0
        rast[..., :2].clamp_(0, 1)
        return rast

    def copied(rast):
        return torch.cat([rast[..., :2].clamp(0, 1), rast[..., 2:]], -1)

    out, grad = render(in_place)
    e_out, e_grad = render(copied)
    assert grad.isfinite().all() and (grad != 0).any()
    torch.testing.assert_close(out, e_out)
    scale = e_grad.abs().max().item()
    torch.testing.assert_close(grad, e_grad, atol=1e-5 * scale, rtol=1e-4)


def test_triangles_drawn_in_chunks(scene):
    # A few triangles at a time, ids shifted to their place in the whole buffer, the first
    # chunk that covers a pixel kept: the same picture (no two triangles overlap on screen).
    rast = torch.zeros_like(scene["rast"])
    tri = scene["tri"]
    for start in range(0, tri.shape[0], 20):
        chunk, _ = dr.rasterize(scene["ctx"], scene["pos"], tri[start:start + 20], RES)
        covered = chunk[..., 3:4] > 0
        chunk[..., 3:4] += start
        rast = torch.where(covered & (rast[..., 3:4] == 0), chunk, rast)
    assert torch.equal(rast[..., 3], scene["rast"][..., 3])
    assert rast[..., 3].max() > 60
    out, _ = dr.interpolate(scene["uv"], rast, tri)
    expect, _ = dr.interpolate(scene["uv"], scene["rast"], tri)
    torch.testing.assert_close(out, expect, atol=1e-5, rtol=1e-5)


def test_empty_and_unused_derivatives_to_texture(scene):
    tex = noisy(1, 8, 8, 3, seed=5).cuda()
    uv, uv_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"])
    assert uv_da.shape[-1] == 0
    for mode in ("auto", "linear", "nearest"):
        assert torch.equal(dr.texture(tex, uv, uv_da, filter_mode=mode),
                           dr.texture(tex, uv, filter_mode=mode))
    uv, uv_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"], scene["rast_db"], "all")
    assert torch.equal(dr.texture(tex, uv, uv_da, filter_mode="nearest"),
                       dr.texture(tex, uv, filter_mode="nearest"))


def test_constant_texture_with_mipmaps(scene):
    tex = torch.tensor([0.2, 0.5, 0.9], device="cuda").view(1, 1, 1, 3).requires_grad_(True)
    uv, uv_da = dr.interpolate(scene["uv"], scene["rast"], scene["tri"], scene["rast_db"], "all")
    out = dr.texture(tex, uv, uv_da, filter_mode="linear-mipmap-linear")
    out.sum().backward()
    torch.testing.assert_close(out, tex.detach().expand_as(out))
    pixels = float(out[..., 0].numel())
    torch.testing.assert_close(tex.grad.flatten(), torch.full((3,), pixels, device="cuda"))


def test_antialias_of_a_mask_and_without_grad_db(scene):
    pos = scene["pos"].clone().requires_grad_(True)
    mask = (scene["rast"][..., 3:] > 0).float()
    out = dr.antialias(mask, scene["rast"], pos, scene["tri"])
    out.sum().backward()
    assert ((out > 0) & (out < 1)).any() and pos.grad.isfinite().all() and (pos.grad != 0).any()
    pos = scene["pos"].clone().requires_grad_(True)
    rast, _ = dr.rasterize(scene["ctx"], pos, scene["tri"], RES, grad_db=False)
    dr.interpolate(scene["uv"], rast, scene["tri"])[0].sum().backward()
    assert torch.equal(rast, scene["rast"]) and (pos.grad != 0).any()


def test_non_contiguous_inputs_to_every_op(scene):
    tex = noisy(1, 16, 16, 3, seed=6).cuda()
    weights = noisy(2, *RES, 3, seed=7).cuda()
    feat = noisy(scene["pos"].shape[1], 4, seed=8).cuda()

    def render(convert):
        pos = scene["pos"].clone().requires_grad_(True)
        texture = tex.clone().requires_grad_(True)
        attr = feat.clone().requires_grad_(True)
        tri = convert(scene["tri"])
        rast, rast_db = dr.rasterize(scene["ctx"], convert(pos), tri, RES)
        uv, uv_da = dr.interpolate(convert(scene["uv"]), convert(rast), tri, convert(rast_db),
                                   "all")
        f, _ = dr.interpolate(convert(attr), rast, tri)
        color = dr.texture(convert(texture), convert(uv), convert(uv_da),
                           filter_mode="linear-mipmap-linear")
        color = color + 0.1 * f[..., :3]
        out = dr.antialias(convert(color), convert(rast), convert(pos), tri)
        (out * weights).sum().backward()
        return out.detach(), pos.grad, texture.grad, attr.grad

    expect = render(lambda t: t)
    for ours, theirs in zip(render(strided), expect, strict=True):
        scale = theirs.abs().max().item()
        assert scale > 0
        torch.testing.assert_close(ours, theirs, atol=1e-5 * scale, rtol=1e-4)


def test_depth_peeler_and_ranges_with_strided_inputs(scene):
    pos = scene["pos"][0]
    tri = scene["tri"]
    ranges = torch.tensor([[0, 40], [30, 50]], dtype=torch.int32)
    layers = []
    for convert in (lambda t: t, strided):
        with dr.DepthPeeler(scene["ctx"], convert(pos), convert(tri), RES,
                            ranges=ranges) as peeler:
            layers.append([peeler.rasterize_next_layer()[0] for _ in range(2)])
    for a, b in zip(*layers):
        assert torch.equal(a, b)


def test_nvdiffrast_and_diffrast_torch_names(scene):
    assert drt.rasterize is dr.rasterize
    dr.install_as_nvdiffrast()
    try:
        import nvdiffrast.torch as nv
        ctx = nv.RasterizeCudaContext(device="cuda")
        rast, rast_db = nv.rasterize(ctx, scene["pos"], scene["tri"], resolution=[28, 36])
        assert torch.equal(rast, scene["rast"]) and torch.equal(rast_db, scene["rast_db"])
        uv, uv_da = nv.interpolate(scene["uv"], rast, scene["tri"], rast_db=rast_db,
                                   diff_attrs="all")
        tex = noisy(1, 16, 16, 3, seed=9).cuda()
        col = nv.texture(tex, uv, uv_da, filter_mode="linear-mipmap-linear")
        out = nv.antialias(col, rast, scene["pos"], scene["tri"])
        expect = dr.antialias(dr.texture(tex, uv, uv_da, filter_mode="linear-mipmap-linear"),
                              scene["rast"], scene["pos"], scene["tri"])
        assert torch.equal(out, expect)
    finally:
        dr.uninstall_as_nvdiffrast()
    assert "nvdiffrast" not in sys.modules
