"""float64 at the backend level: the reference's GPU backend accepts float64 tensors and computes
in double (its tests: resolve to 1e-12, tests/test_coverage.py:792-808; interpolate and texture
by gradcheck, tests/test_triton.py:234-240 and :303-319; antialias to 1e-9, :408-415). Here the
same checks run against the oracle evaluated in float64; visibility stays float32 on both
backends, so pixels on an outline may differ and are left out where stated."""

import pytest
import torch

from diffrast_amd.backends import hip
from helpers import random_mesh
from oracle import reference as R

pytestmark = pytest.mark.gpu


def perspective_triangle():
    pos = torch.tensor([[[-0.8, -0.6, 0.2, 1.0], [1.2, -0.9, 0.5, 2.0], [0.1, 1.5, -0.3, 1.5]]],
                       dtype=torch.float64)
    return pos, torch.tensor([[0, 1, 2]], dtype=torch.int32)


@pytest.mark.parametrize("resolution", [(64, 96), (100, 100)])
def test_resolve_is_accurate_to_float64(resolution):
    # Sizes whose pixel size 2 / size is inexact in float32.
    pos, tri = perspective_triangle()
    ref_pos, our_pos = pos.clone().requires_grad_(True), pos.cuda().requires_grad_(True)
    ref, ref_db = R.rasterize(ref_pos, tri, resolution, True)
    ours, our_db = hip.rasterize(our_pos, tri.cuda(), resolution, True)
    assert ours.dtype == torch.float64 and our_db.dtype == torch.float64
    same = ref[..., 3] == ours[..., 3].cpu()
    assert same.float().mean() > 0.999 and (ref[..., 3] > 0).sum() > 100
    ref_db[same].square().sum().backward()
    our_db[same.cuda()].square().sum().backward()
    for value, expected in ((ours, ref), (our_db, ref_db)):
        torch.testing.assert_close(value.detach().cpu()[same], expected.detach()[same],
                                   rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(our_pos.grad.cpu(), ref_pos.grad, rtol=1e-12, atol=1e-13)


def interp_scene(channels, layout, seed):
    gen = torch.Generator().manual_seed(seed)
    pos, tri = random_mesh(80, gen, batch=2)
    rast, rast_db = R.rasterize(pos.double(), tri, (40, 56), True)
    v = pos.shape[1]
    shape = {"shared": (v, channels)}.get(layout, (2, v, channels))
    attr = torch.randn(*shape, generator=gen, dtype=torch.float64)
    return attr, rast.detach(), rast_db.detach(), tri


def test_interpolate_gradcheck_float64():
    attr, rast, rast_db, tri = interp_scene(3, "per_view", seed=4)
    rast, rast_db = rast[:, :8, :8].contiguous(), rast_db[:, :8, :8].contiguous()
    assert (rast[..., 3] > 0).any()
    inputs = [t.cuda().requires_grad_(True) for t in (attr, rast, rast_db)]
    tri = tri.cuda()
    assert torch.autograd.gradcheck(lambda a, r, d: hip.interpolate(a, r, tri, d, [0, 2]), inputs)


def test_interpolate_float64_matches_oracle():
    attr, rast, rast_db, tri = interp_scene(5, "shared", seed=5)
    ref = R.interpolate(attr, rast, tri, rast_db, [4, 1])
    ours = hip.interpolate(attr.cuda(), rast.cuda(), tri.cuda(), rast_db.cuda(), [4, 1])
    for o, e in zip(ours, ref):
        assert o.dtype == torch.float64
        torch.testing.assert_close(o.cpu(), e, rtol=1e-13, atol=1e-14)


FILTERS = ("nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear")


@pytest.mark.parametrize("filter_mode", FILTERS)
def test_texture_gradcheck_float64(filter_mode):
    gen = torch.Generator().manual_seed(3)
    tex = torch.randn(2, 6, 7, 2, generator=gen, dtype=torch.float64)
    uv = torch.rand(2, 3, 3, 2, generator=gen, dtype=torch.float64) * 1.6 - 0.3
    # Footprints of 1.2 to 3.2 texels keep the level of detail away from integers and clamps.
    scale = (torch.rand(2, 3, 3, 1, generator=torch.Generator().manual_seed(4)) * 2 + 1.2) / 7
    uv_da = scale.double() * torch.tensor([1.0, 0.1, -0.2, 0.9], dtype=torch.float64)
    mip = "mipmap" in filter_mode
    inputs = [t.cuda().requires_grad_(True) for t in (tex, uv, uv_da)]
    if filter_mode == "nearest":
        inputs[1].requires_grad_(False)
    assert torch.autograd.gradcheck(
        lambda t, c, d: hip.texture(t, c, d if mip else None, filter_mode, "wrap", None), inputs)


@pytest.mark.parametrize("boundary", ["wrap", "clamp", "zero"])
@pytest.mark.parametrize("filter_mode", FILTERS)
def test_texture_float64_matches_oracle(filter_mode, boundary):
    gen = torch.Generator().manual_seed(6)
    tex = torch.randn(2, 37, 50, 3, generator=gen, dtype=torch.float64)
    uv = torch.rand(2, 20, 24, 2, generator=gen, dtype=torch.float64) * 1.6 - 0.3
    uv_da = torch.rand(2, 20, 24, 4, generator=gen, dtype=torch.float64) * 0.2 - 0.1
    weights = torch.randn(2, 20, 24, 3, generator=gen, dtype=torch.float64)
    mip = "mipmap" in filter_mode
    grads = []
    for fn, device in ((hip.texture, "cuda"), (R.texture, "cpu")):
        ins = [t.clone().to(device).requires_grad_(True) for t in (tex, uv, uv_da)]
        out = fn(ins[0], ins[1], ins[2] if mip else None, filter_mode, boundary, None)
        (out * weights.to(device)).sum().backward()
        grads.append([out.detach().cpu()] + [
            t.grad.cpu() if t.grad is not None else torch.zeros_like(t).cpu() for t in ins])
    for o, e in zip(*grads):
        torch.testing.assert_close(o, e, rtol=1e-11, atol=1e-11)


def test_cube_map_float64_matches_oracle():
    gen = torch.Generator().manual_seed(7)
    cube = torch.randn(1, 6, 9, 9, 2, generator=gen, dtype=torch.float64)
    dirs = torch.randn(2, 10, 12, 3, generator=gen, dtype=torch.float64)
    dirs_da = torch.randn(2, 10, 12, 6, generator=gen, dtype=torch.float64) * 0.05
    weights = torch.randn(2, 10, 12, 2, generator=gen, dtype=torch.float64)
    grads = []
    for fn, device in ((hip.texture, "cuda"), (R.texture, "cpu")):
        ins = [t.clone().to(device).requires_grad_(True) for t in (cube, dirs, dirs_da)]
        out = fn(ins[0], ins[1], ins[2], "linear-mipmap-linear", "cube", None)
        (out * weights.to(device)).sum().backward()
        grads.append([out.detach().cpu()] + [t.grad.cpu() for t in ins])
    for o, e in zip(*grads):
        torch.testing.assert_close(o, e, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("channels", [1, 3, 20])
@pytest.mark.parametrize("mesh", [{}, {"w_range": (-1.0, 2.0)}, {"z_range": 2.0, "xy_range": 3.0}])
def test_antialias_float64_matches_oracle(channels, mesh):
    pos, tri = random_mesh(60, torch.Generator().manual_seed(0), batch=2, **mesh)
    pos = pos.double()
    rast, _ = R.rasterize(pos, tri, (48, 64), True)
    gen = torch.Generator().manual_seed(1)
    color = torch.rand(2, 48, 64, channels, generator=gen, dtype=torch.float64)
    weights = torch.randn(2, 48, 64, channels, generator=gen, dtype=torch.float64)
    results = []
    for fn, device in ((hip.antialias, "cuda"), (R.antialias, "cpu")):
        c = color.clone().to(device).requires_grad_(True)
        p = pos.clone().to(device).requires_grad_(True)
        out = fn(c, rast.detach().to(device), p, tri.to(device), 1.0)
        (out * weights.to(device)).sum().backward()
        results.append((out.detach().cpu(), c.grad.cpu(), p.grad.cpu()))
    assert (results[1][0] != color).any(), "the scene should have silhouettes to blend"
    for o, e in zip(*results):
        torch.testing.assert_close(o, e, atol=1e-9, rtol=1e-9)


def test_float64_refuses_mixed_types():
    attr, rast, rast_db, tri = interp_scene(3, "shared", seed=8)
    with pytest.raises(TypeError, match="rast must be torch.float64"):
        hip.interpolate(attr.cuda(), rast.float().cuda(), tri.cuda(), None, [])
