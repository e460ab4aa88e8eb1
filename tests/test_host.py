"""Host logic on the CPU: validation, backend selection, range mode, depth peeling, caches,
compatibility shims. The ops run on the CPU oracle through a test-only backend (the product
itself refuses CPU tensors)."""

import pickle
import threading
import warnings

import pytest
import torch

import diffrast_amd as dr
import oracle_backend
from diffrast_amd import _cache, backends, compat, log, ops, peeling, topology
from diffrast_amd.backends._autograd import first_order
from oracle import reference as R


@pytest.fixture
def oracle_backend_installed(monkeypatch):
    def get(device, op):
        return oracle_backend

    for module in (ops, peeling, topology):
        monkeypatch.setattr(module, "get_backend", get)
    topology._neighbour_cache.clear()
    yield
    topology._neighbour_cache.clear()


@pytest.fixture
def ctx():
    return dr.RasterizeContext("cpu")


def scene(num_tri=24, seed=0):
    gen = torch.Generator().manual_seed(seed)
    xy = torch.rand(3 * num_tri, 2, generator=gen) * 2.4 - 1.2
    z = torch.rand(3 * num_tri, 1, generator=gen) * 1.8 - 0.9
    w = torch.rand(3 * num_tri, 1, generator=gen) + 1.0
    pos = torch.cat([xy * w, z * w, w], -1)
    return pos, torch.arange(3 * num_tri, dtype=torch.int32).view(num_tri, 3)


# ---- backend selection -----------------------------------------------------------------------


def test_product_refuses_cpu_tensors_and_the_reference_backend(ctx):
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        backends.get_backend("cpu", "rasterize")
    with pytest.raises(ValueError, match="not part of diffrast_amd"):
        dr.set_backend("reference")
    with pytest.raises(ValueError, match="Unknown backend"):
        dr.set_backend("opengl")
    with pytest.raises(ValueError, match="Unknown op"):
        backends.get_backend_name("cuda", "shade")
    for name in ("hip", "triton", "auto"):
        dr.set_backend(name)
    dr.set_backend("auto")
    pos, tri = scene()
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        dr.rasterize(ctx, pos[None], tri, (8, 8))


def test_first_order_guard():
    class Twice(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            return x * 2

        @staticmethod
        @first_order("twice")
        def backward(ctx, g):
            return g * 2

    x = torch.ones(3, requires_grad=True)
    (gx,) = torch.autograd.grad(Twice.apply(x).sum(), x)
    assert torch.equal(gx, torch.full((3,), 2.0))
    with pytest.raises(RuntimeError, match="no second-order gradients"):
        torch.autograd.grad(Twice.apply(x).sum(), x, create_graph=True)


# ---- validation ------------------------------------------------------------------------------


def test_rasterize_validation(ctx):
    pos, tri = scene()
    with pytest.raises(ValueError, match=r"pos must have shape \[batch, vertices, 4\]"):
        dr.rasterize(ctx, pos[None, :, :3], tri, (8, 8))
    with pytest.raises(TypeError, match="tri must be torch.int32"):
        dr.rasterize(ctx, pos[None], tri.long(), (8, 8))
    with pytest.raises(ValueError, match="refers to vertex"):
        dr.rasterize(ctx, pos[None], tri + 1000, (8, 8))
    with pytest.raises(ValueError, match="resolution must be"):
        dr.rasterize(ctx, pos[None], tri, (8,))
    with pytest.raises(ValueError, match="resolution must be positive"):
        dr.rasterize(ctx, pos[None], tri, (0, 8))
    with pytest.raises(ValueError, match="ranges is required"):
        dr.rasterize(ctx, pos, tri, (8, 8))
    with pytest.raises(ValueError, match="does not lie within"):
        dr.rasterize(ctx, pos, tri, (8, 8), ranges=torch.tensor([[20, 10]], dtype=torch.int32))
    with pytest.raises(ValueError, match=r"at most 2\*\*24"):
        dr.rasterize(ctx, pos[None], tri[:1].expand((1 << 24) + 1, 3), (4, 4))
    assert ops.check_rasterize_inputs(ctx, pos[None], tri[:1].expand(1 << 24, 3), (4, 4),
                                      None) == (4, 4)


def test_interpolate_and_texture_validation():
    rast = torch.zeros(1, 4, 4, 4)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    attr = torch.zeros(3, 2)
    with pytest.raises(ValueError, match="rast_db is required"):
        dr.interpolate(attr, rast, tri, diff_attrs="all")
    with pytest.raises(ValueError, match="the one given is empty"):
        dr.interpolate(attr, rast, tri, rast_db=torch.zeros(1, 4, 4, 0), diff_attrs=[0])
    with pytest.raises(ValueError, match="out of range"):
        dr.interpolate(attr, rast, tri, rast_db=rast, diff_attrs=[2])
    with pytest.raises(TypeError, match="diff_attrs must be"):
        dr.interpolate(attr, rast, tri, rast_db=rast, diff_attrs=[0.5])
    with pytest.raises(ValueError, match="attr batch size"):
        dr.interpolate(torch.zeros(3, 3, 2), rast, tri)
    tex = torch.zeros(1, 4, 4, 3)
    uv = torch.zeros(1, 4, 4, 2)
    with pytest.raises(ValueError, match="Unknown filter_mode"):
        dr.texture(tex, uv, filter_mode="cubic")
    with pytest.raises(ValueError, match="requires uv_da or mip_level_bias"):
        dr.texture(tex, uv, filter_mode="linear-mipmap-linear")
    with pytest.raises(ValueError, match="shape of a cube map"):
        dr.texture(torch.zeros(1, 6, 4, 4, 3), uv)
    with pytest.raises(ValueError, match="six square faces"):
        dr.texture(torch.zeros(1, 5, 4, 4, 3), torch.zeros(1, 4, 4, 3), boundary_mode="cube")
    with pytest.raises(TypeError, match="mip must be"):
        dr.texture(tex, uv, uv_da=torch.zeros(1, 4, 4, 4), mip=5)
    with pytest.raises(ValueError, match="max_mip_level must be non-negative"):
        dr.texture(tex, uv, max_mip_level=-1)
    with pytest.raises(ValueError, match="All inputs must be on the same device"):
        dr.texture(tex, uv.to("meta"))


def test_antialias_validation():
    color = torch.zeros(1, 4, 4, 3)
    rast = torch.zeros(1, 4, 4, 4)
    pos = torch.zeros(3, 4)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    with pytest.raises(ValueError, match="color must match rast"):
        dr.antialias(torch.zeros(1, 5, 4, 3), rast, pos, tri)
    with pytest.raises(ValueError, match="pos batch size"):
        dr.antialias(color, rast, torch.zeros(2, 3, 4), tri)
    with pytest.raises(TypeError, match="pos_gradient_boost must be a number"):
        dr.antialias(color, rast, pos, tri, pos_gradient_boost="big")
    with pytest.raises(TypeError, match="topology_hash must come from"):
        topology.neighbours_for(tri, object())


# ---- range mode, depth peeling, mip stacks (oracle backend) ----------------------------------


def test_range_mode_matches_instanced_calls(oracle_backend_installed, ctx):
    pos, tri = scene()
    ranges = torch.tensor([[0, 9], [10, 13], [4, 5], [23, 1], [7, 0]], dtype=torch.int32)
    rast, rast_db = dr.rasterize(ctx, pos, tri, (24, 32), ranges=ranges)
    assert rast.shape == rast_db.shape == (5, 24, 32, 4)
    for item, (start, count) in enumerate(ranges.tolist()):
        one, one_db = dr.rasterize(ctx, pos[None], tri[start:start + count], (24, 32))
        ids = torch.where(one[..., 3:] > 0, one[..., 3:] + start, 0)
        assert torch.equal(rast[item], torch.cat([one[..., :3], ids], -1)[0])
        assert torch.equal(rast_db[item], one_db[0])


def test_depth_peeler_layers_and_lifetime(oracle_backend_installed, ctx):
    pos, tri = scene(seed=1)
    pos = pos[None].requires_grad_(True)
    with dr.DepthPeeler(ctx, pos, tri, (16, 16)) as peeler:
        layers = [peeler.rasterize_next_layer()[0] for _ in range(3)]
    first, _ = dr.rasterize(ctx, pos, tri, (16, 16))
    assert torch.equal(layers[0], first)
    both = (layers[0][..., 3] > 0) & (layers[1][..., 3] > 0)
    assert both.any() and (layers[1][..., 2][both] >= layers[0][..., 2][both]).all()
    with pytest.raises(RuntimeError, match="closed"):
        peeler.rasterize_next_layer()
    layers[1][..., :3].sum().backward()
    assert pos.grad is not None and pos.grad.abs().sum() > 0


def test_depth_peeler_copies_its_geometry(oracle_backend_installed, ctx):
    pos, tri = scene(seed=2)
    pos = pos[None]
    peeler = dr.DepthPeeler(ctx, pos, tri, (16, 16))
    expected = R.rasterize_layer(pos.clone(), tri, (16, 16), True, None)[0]
    pos.mul_(0.0)
    assert torch.equal(peeler.rasterize_next_layer()[0], expected)


def test_gl_context_without_derivatives(oracle_backend_installed):
    pos, tri = scene(seed=3)
    glctx = dr.RasterizeGLContext(output_db=False, device="cpu")
    rast, rast_db = dr.rasterize(glctx, pos[None], tri, (8, 8))
    assert rast_db.shape == (1, 8, 8, 0)
    with pytest.raises(TypeError, match="output_db must be a bool"):
        dr.RasterizeGLContext("cpu")


def test_mip_stack_packs_once_for_a_constant_texture(oracle_backend_installed):
    tex = torch.rand(1, 8, 8, 3)
    stack = dr.texture_construct_mip(tex)
    first = stack.pack(tex)
    assert stack.pack(tex) is first
    tex.add_(1.0)
    assert stack.pack(tex) is not first
    with pytest.raises(ValueError, match="constructed for a texture of shape"):
        dr.texture(torch.rand(1, 4, 4, 3), torch.rand(1, 2, 2, 2), uv_da=torch.rand(1, 2, 2, 4),
                   mip=stack)


def test_topology_cache_follows_the_tensor(oracle_backend_installed):
    pos, tri = scene(seed=4)
    rast = R.rasterize(pos[None], tri, (12, 12))[0]
    color = torch.rand(1, 12, 12, 3)
    dr.antialias(color, rast, pos, tri)
    assert len(topology._neighbour_cache) == 1
    dr.antialias(color, rast, pos, tri)
    assert len(topology._neighbour_cache) == 1
    topo = dr.antialias_construct_topology_hash(tri)
    clone = pickle.loads(pickle.dumps(topo))
    assert torch.equal(clone.neighbours(tri), topo.neighbours(tri))
    tri.add_(0)  # an in-place edit bumps the version
    with pytest.raises(ValueError, match="modified in place"):
        topo.neighbours(tri)
    with pytest.raises(ValueError, match="built for a tri of shape"):
        topo.neighbours(tri[:3])


# ---- caches, logging, compatibility ----------------------------------------------------------


def test_tensor_cache_semantics():
    calls = []
    cache = _cache.TensorCache(lambda t: calls.append(1) or t.sum().item(), max_entries=2)
    a = torch.ones(3)
    assert cache.get(a) == 3 and cache.get(a) == 3 and len(calls) == 1
    a.add_(1)
    assert cache.get(a) == 6 and len(calls) == 2
    b, c = torch.ones(1), torch.ones(2)
    cache.get(b), cache.get(c)
    assert len(cache) == 2
    del b, c
    assert len(cache) <= 2
    with torch.inference_mode():
        inf = torch.ones(2)
    cache.get(inf), cache.get(inf)
    errors = []

    def worker():
        try:
            for _ in range(200):
                cache.get(torch.ones(4))
        except Exception as e:  # pragma: no cover
            errors.append(e)

    threads = [threading.Thread(target=worker) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors


def test_log_levels_and_compat_aliases():
    assert log.get_log_level() == log.WARNING
    with pytest.raises(ValueError):
        dr.set_log_level(7)
    with pytest.raises(TypeError):
        dr.set_log_level("info")
    dr.set_log_level(2)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        log.warn("quiet at level 2")
    dr.set_log_level(1)
    import sys

    dr.install_as_nvdiffrast()
    import nvdiffrast.torch as nvdr

    assert nvdr.rasterize is dr.rasterize
    dr.uninstall_as_nvdiffrast()
    assert "nvdiffrast" not in sys.modules
    import diffrast
    import diffrast.torch as dt

    assert dt.rasterize is dr.rasterize and diffrast.ops is ops
    assert compat._displaced == {}


def test_range_tables_used_under_capture_are_never_evicted():
    # A captured graph keeps the device range tables' addresses, so a table used while a stream
    # is captured stays for good; beyond 16 tables the others are evicted, least recent first.
    from diffrast_amd.backends import hip

    cpu = torch.device("cpu")
    hip._RANGE_COPIES.clear()
    try:
        pinned = hip._range_tables([(0, 3), (3, 3)], [0, 3, 6], cpu, capturing=True)
        for i in range(40):
            hip._range_tables([(i, 1)], [0, 1], cpu, capturing=False)
        assert len(hip._RANGE_COPIES) == hip._RANGE_COPIES_KEPT
        again = hip._range_tables([(0, 3), (3, 3)], [0, 3, 6], cpu, capturing=False)
        assert again[0] is pinned[0] and again[1] is pinned[1]
        assert torch.equal(pinned[1], torch.tensor([0, 3, 6]))
        # A table first drawn eagerly and then under capture becomes pinned too.
        hip._range_tables([(7, 2)], [0, 2], cpu, capturing=False)
        hip._range_tables([(7, 2)], [0, 2], cpu, capturing=True)
        for i in range(40, 80):
            hip._range_tables([(i, 1)], [0, 1], cpu, capturing=False)
        keys = {key[1] for key in hip._RANGE_COPIES}
        assert ((0, 3), (3, 3)) in keys and ((7, 2),) in keys
        assert ((40, 1),) not in keys and ((79, 1),) in keys
        assert len(hip._RANGE_COPIES) == hip._RANGE_COPIES_KEPT
    finally:
        hip._RANGE_COPIES.clear()
