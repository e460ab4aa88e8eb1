"""The five benchmark workloads at their full sizes, checked at sampled pixels.

The oracle cannot rasterize a 1.3M-triangle mesh at 8 x 1024^2 in a test, but its brute-force
visibility at a list of pixels (``visible_at``) goes through the same arithmetic for every
(triangle, pixel) pair, so ids must be bit-exact there; rast values come from the oracle's
resolve of those ids. Interpolate and texture are per-pixel operations: the oracle runs on the
GPU's own inputs at the sampled pixels (packed into a one-row image) and must agree to the
stated tolerance (interpolate bit-exact). Gradients are checked at the small sizes of the other
test files.
"""

import pytest
import torch

import diffrast_amd as dr
from bench import reflect
from diffrast_amd import workloads
from helpers import rel_error
from oracle import reference as R

pytestmark = pytest.mark.gpu

VALUE_TOL = 1e-5
GRAD_TOL = 1e-4
SAMPLES = 48  # pixels per checked image: half covered (by the GPU result), half anywhere


def sample_pixels(ids, image, gen):
    """(row, col) of SAMPLES pixels of ``image``: half where ids shows a triangle."""
    covered = (ids[image] >= 0).nonzero()
    anywhere = torch.stack([torch.randint(0, ids.shape[1], (SAMPLES // 2,), generator=gen),
                            torch.randint(0, ids.shape[2], (SAMPLES // 2,), generator=gen)], 1)
    pick = covered[torch.randperm(covered.shape[0], generator=gen)[:SAMPLES // 2]]
    rc = torch.cat([pick, anywhere])
    return rc[:, 0], rc[:, 1]


def check_visibility(pos, tri, rast, images, gen, offset=0, previous=None):
    """Ids bit-exact and rast within VALUE_TOL at sampled pixels of ``images``; returns the
    sampled (b, row, col) and the oracle's (depth, id) there."""
    H, W = rast.shape[1:3]
    gpu_ids = rast[..., 3].long() - 1
    bs, rows, cols = [], [], []
    for b in images:
        r, c = sample_pixels(gpu_ids, b, gen)
        bs.append(torch.full_like(r, b))
        rows.append(r)
        cols.append(c)
    b, row, col = torch.cat(bs), torch.cat(rows), torch.cat(cols)
    depth, ids = R.visible_at(pos, tri, H, W, b if pos.shape[0] > 1 else torch.zeros_like(b),
                              row, col, previous)
    ids = torch.where(ids >= 0, ids + offset, ids)
    assert torch.equal(gpu_ids[b, row, col], ids), "ids differ at sampled pixels"
    # rast there, from the oracle's resolve of those ids (one image per checked pixel).
    full_tri = tri if offset == 0 else None
    if full_tri is not None:
        tri_id = torch.full((pos.shape[0],) + tuple(rast.shape[1:3]), -1, dtype=torch.long)
        tri_id[b if pos.shape[0] > 1 else torch.zeros_like(b), row, col] = ids
        ref, _ = R.rasterize_from_ids(pos, tri, tri_id, False)
        ours = rast[b, row, col]
        expect = ref[b if pos.shape[0] > 1 else torch.zeros_like(b), row, col]
        assert rel_error(ours[:, :3], expect[:, :3]) < VALUE_TOL
    return (b, row, col), (depth, ids)


def packed(t, where):
    """Values of ``t`` [B, H, W, C] at the sampled pixels as a one-row image [1, 1, n, C]."""
    b, row, col = where
    return t[b, row, col][None, None]


def test_sphere_workload_in_full_forward_and_backward():
    # Small enough for the oracle at full size: rasterize -> interpolate -> antialias -> MSE,
    # every output and the gradients to positions and colours.
    w = workloads.build("sphere")
    t = w.tensors
    dev = torch.device("cuda", 0)
    tri, target = t["tri"], t["target"]

    def run(ops, pos, attr, rast_fn):
        pos = pos.clone().requires_grad_()
        attr = attr.clone().requires_grad_()
        rast = rast_fn(pos)
        col, _ = ops.interpolate(attr, rast, tri.to(pos.device))
        out = ops.antialias(col, rast, pos, tri.to(pos.device))
        ((out - target.to(pos.device)) ** 2).mean().backward()
        return [x.detach().cpu() for x in (rast, col, out, pos.grad, attr.grad)]

    ctx = dr.RasterizeContext(dev)
    ours = run(dr, t["pos"].to(dev), t["attr"].to(dev),
               lambda p: dr.rasterize(ctx, p, tri.to(dev), w.resolution, grad_db=False)[0])
    ids = R.rasterize(t["pos"], tri, w.resolution, False)[0][..., 3].long() - 1

    class Oracle:
        interpolate = staticmethod(lambda a, r, tr: R.interpolate(a, r, tr, None, []))
        antialias = staticmethod(R.antialias)

    ref = run(Oracle, t["pos"], t["attr"], lambda p: R.rasterize_from_ids(p, tri, ids, False)[0])
    assert torch.equal(ours[0][..., 3], ref[0][..., 3])
    for got, expect in zip(ours[:3], ref[:3]):
        assert rel_error(got, expect) < VALUE_TOL
    for got, expect in zip(ours[3:], ref[3:]):
        scale = expect.abs().max().item()
        assert scale > 0
        torch.testing.assert_close(got, expect, atol=GRAD_TOL * scale, rtol=GRAD_TOL)


def test_large_workload_at_sampled_pixels():
    w = workloads.build("large")
    t = w.tensors
    dev = torch.device("cuda", 0)
    ctx = dr.RasterizeContext(dev)
    tri = t["tri"]
    rast, rast_db = dr.rasterize(ctx, t["pos"].to(dev), tri.to(dev), w.resolution)
    f, _ = dr.interpolate(t["feat"].to(dev), rast, tri.to(dev))
    st, st_da = dr.interpolate(t["uv"].to(dev), rast, tri.to(dev), rast_db, diff_attrs="all")
    col = dr.texture(t["tex"].to(dev), st, st_da, filter_mode="linear-mipmap-linear",
                     boundary_mode="wrap")
    rast, rast_db, f, st, st_da, col = (x.cpu() for x in (rast, rast_db, f, st, st_da, col))
    gen = torch.Generator().manual_seed(30)
    where, _ = check_visibility(t["pos"], tri, rast, [0, 5], gen)
    pr, pdb = packed(rast, where), packed(rast_db, where)
    ref_f, _ = R.interpolate(t["feat"], pr, tri, None, [])
    assert torch.equal(packed(f, where), ref_f)
    ref_st, ref_da = R.interpolate(t["uv"], pr, tri, pdb, [0, 1])
    assert torch.equal(packed(st, where), ref_st) and torch.equal(packed(st_da, where), ref_da)
    ref_col = R.texture(t["tex"], ref_st, ref_da, "linear-mipmap-linear", "wrap", None)
    assert rel_error(packed(col, where), ref_col) < VALUE_TOL


def test_textured_workload_at_sampled_pixels():
    w = workloads.build("textured")
    t = w.tensors
    dev = torch.device("cuda", 0)
    tri = t["tri"]
    rast, rast_db = dr.rasterize(dr.RasterizeContext(dev), t["pos"].to(dev), tri.to(dev),
                                 w.resolution)
    uv, uv_da = dr.interpolate(t["uv"].to(dev), rast, tri.to(dev), rast_db, diff_attrs="all")
    tex = t["tex"].to(dev)
    col = dr.texture(tex, uv, uv_da, mip=dr.texture_construct_mip(tex),
                     filter_mode="linear-mipmap-linear", boundary_mode="wrap")
    rast, rast_db, uv, uv_da, col = (x.cpu() for x in (rast, rast_db, uv, uv_da, col))
    gen = torch.Generator().manual_seed(31)
    where, _ = check_visibility(t["pos"], tri, rast, [0, 3], gen)
    ref_uv, ref_da = R.interpolate(t["uv"], packed(rast, where), tri, packed(rast_db, where),
                                   [0, 1])
    assert torch.equal(packed(uv, where), ref_uv) and torch.equal(packed(uv_da, where), ref_da)
    ref_col = R.texture(t["tex"], ref_uv, ref_da, "linear-mipmap-linear", "wrap", None)
    assert rel_error(packed(col, where), ref_col) < VALUE_TOL


def test_cubemap_workload_at_sampled_pixels():
    w = workloads.build("cubemap")
    t = w.tensors
    dev = torch.device("cuda", 0)
    tri = t["tri"]
    rast, rast_db = dr.rasterize(dr.RasterizeContext(dev), t["pos"].to(dev), tri.to(dev),
                                 w.resolution)
    n, n_da = dr.interpolate(t["normals"].to(dev), rast, tri.to(dev), rast_db, diff_attrs="all")
    dirs, dirs_da = reflect(t["view"].to(dev), n, n_da)
    col = dr.texture(t["cube"].to(dev), dirs, dirs_da, filter_mode="linear-mipmap-linear",
                     boundary_mode="cube")
    rast, rast_db, n, n_da, dirs, dirs_da, col = (
        x.cpu() for x in (rast, rast_db, n, n_da, dirs, dirs_da, col))
    gen = torch.Generator().manual_seed(32)
    where, _ = check_visibility(t["pos"], tri, rast, [1, 2], gen)
    ref_n, ref_nda = R.interpolate(t["normals"], packed(rast, where), tri,
                                   packed(rast_db, where), [0, 1, 2])
    assert torch.equal(packed(n, where), ref_n) and torch.equal(packed(n_da, where), ref_nda)
    ref_col = R.texture(t["cube"], packed(dirs, where), packed(dirs_da, where),
                        "linear-mipmap-linear", "cube", None)
    assert rel_error(packed(col, where), ref_col) < VALUE_TOL


def test_instances_workload_layers_at_sampled_pixels():
    # Range mode with depth peeling: item i draws triangles [start, start + count); every
    # layer must match the oracle's peel of that item alone.
    w = workloads.build("instances")
    t = w.tensors
    dev = torch.device("cuda", 0)
    pos, tri, ranges = t["pos"], t["tri"], t["ranges"]
    layers = []
    with dr.DepthPeeler(dr.RasterizeContext(dev), pos.to(dev), tri.to(dev), w.resolution,
                        ranges=ranges) as peeler:
        for _ in range(3):
            layers.append(peeler.rasterize_next_layer()[0].cpu())
    gen = torch.Generator().manual_seed(33)
    for item in (0, 97, 255):
        start, count = (int(v) for v in ranges[item])
        own = tri[start:start + count]
        previous = None
        where = None
        for rast in layers:
            one = rast[item:item + 1]
            gpu_ids = one[..., 3].long() - 1
            if where is None:
                r, c = sample_pixels(gpu_ids, 0, gen)
                where = (torch.zeros_like(r), r, c)
            b, row, col = where
            depth, ids = R.visible_at(pos[None], own, *w.resolution, b, row, col, previous)
            assert torch.equal(gpu_ids[b, row, col], torch.where(ids >= 0, ids + start, ids))
            previous = (depth, ids)
