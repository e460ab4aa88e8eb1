"""Exception types and messages of the public API, which code written against the reference
matches on (reference tests/test_input_checks.py, tests/test_validation.py). Every check here
fails before a backend is reached, so it runs on the CPU."""

import pytest
import torch

import diffrast_amd as dr
from diffrast_amd import ops
from diffrast_amd._cache import TensorCache

TRI = torch.tensor([[0, 1, 2]], dtype=torch.int32)
POS = torch.tensor([[[-0.5, -0.5, 0.0, 1.0], [0.5, -0.5, 0.0, 1.0], [0.0, 0.5, 0.0, 1.0]]])
RAST = torch.zeros(1, 8, 8, 4)


@pytest.mark.parametrize("resolution", [8, None, 8.0, (8.0, 8.0), (8.5, 8), "88", (8, 8, 8),
                                        [[8, 8]], (8, None), {8, 16}, {8: 1, 16: 2},
                                        range(8, 10), (True, 8), [8, False],
                                        torch.tensor([True, True]), torch.tensor([8.0, 16.0]),
                                        torch.tensor([[8, 16]]), torch.tensor(8)])
def test_resolution_must_be_two_ints(resolution):
    with pytest.raises(ValueError, match=r"resolution must be \(height, width\) as two ints"):
        ops._check_resolution(resolution)


def test_resolution_forms_and_sign():
    np = pytest.importorskip("numpy")
    for form in ([8, 16], (8, 16), torch.Size([8, 16]), torch.tensor([8, 16]),
                 np.array([8, 16]), (np.int64(8), torch.tensor(16))):
        size = ops._check_resolution(form)
        assert size == (8, 16) and all(type(s) is int for s in size)
    with pytest.raises(ValueError, match="as two ints"):
        ops._check_resolution(np.array([8.0, 16.0]))
    with pytest.raises(ValueError, match="as two ints"):
        ops._check_resolution(iter([8, 16]))
    for bad in ((0, 8), (8, -1), [0, 0]):
        with pytest.raises(ValueError, match="resolution must be positive"):
            ops._check_resolution(bad)
    with pytest.raises(ValueError, match=r"resolution must be .* got 8\."):
        dr.rasterize(dr.RasterizeContext("cpu"), POS, TRI, 8)


def test_layouts_and_batch_hints():
    with pytest.raises(ValueError, match=r"rast must have shape \[batch, height, width, 4\].*"
                                         r"rast\[None\]"):
        dr.interpolate(POS, torch.zeros(8, 8, 4), TRI)
    with pytest.raises(ValueError, match=r"pos must have shape \[batch, vertices, 4\], got "
                                         r"\(3, 4\); add a batch"):
        ops._check(POS[0], "pos", ndim=3, last=4)
    with pytest.raises(ValueError, match=r"tex must have shape \[batch, tex_height.*tex\[None\]"):
        ops._check(torch.zeros(4, 4, 3), "tex", ndim=4)
    with pytest.raises(ValueError, match=r"tri must have shape \[triangles, 3\], got \(1, 4\)"):
        dr.interpolate(POS, RAST, torch.zeros(1, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match=r"attr must have shape \[batch, vertices, channels\] or "
                                         r"\[vertices, channels\], got \(4,\)\.$"):
        dr.interpolate(POS[0, 0], RAST, TRI)
    with pytest.raises(ValueError, match=r"rast_db must have shape \[batch, height, width, 4\]"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST[..., :2], diff_attrs="all")
    with pytest.raises(ValueError, match=r"same shape as rast, got \(1, 4, 8, 4\) and"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST[:, :4], diff_attrs="all")
    with pytest.raises(ValueError, match=r"color must match rast.*\(1, 4, 4, 3\) and"):
        dr.antialias(torch.zeros(1, 4, 4, 3), RAST, POS, TRI)
    # Placeholders where the argument's usual layout does not fit.
    with pytest.raises(ValueError, match=r"weights must have shape \[\.\.\., \.\.\., 5\], got"):
        ops._check(torch.zeros(2), "weights", ndim=3, last=5)
    with pytest.raises(ValueError, match=r"uv must have shape \[\.\.\., \.\.\., \.\.\., 3\]"):
        ops._check(torch.zeros(1, 2, 2, 2), "uv", ndim=4, last=3)
    with pytest.raises(ValueError,
                       match=r"tex must have shape \[\.\.\., \.\.\., \.\.\., \.\.\., \.\.\.\]"):
        ops._check(torch.zeros(1, 2, 2, 2), "tex", ndim=5)
    with pytest.raises(ValueError, match=r"pos must have shape \[vertices, 4\], got \(3,\)\.$"):
        ops._check(torch.zeros(3), "pos", ndim=2, last=4, layout="[vertices, 4]")
    with pytest.raises(ValueError, match=r"mip_level_bias must have shape "
                                         r"\[batch, height, width\], got \(2, 2\); add a batch"):
        ops._check(torch.zeros(2, 2), "mip_level_bias", ndim=3)


def test_types_and_conversions():
    with pytest.raises(TypeError, match=r"tri must be torch\.int32, got torch\.int64; convert "
                                        r"it with tri\.int\(\)\.$"):
        dr.interpolate(POS, RAST, TRI.long())
    with pytest.raises(TypeError, match=r"attr must be torch\.float32, got torch\.float64; .*"
                                        r"attr\.float\(\)"):
        dr.interpolate(POS.double(), RAST, TRI)
    with pytest.raises(TypeError, match=r"pos must be torch\.float32, got torch\.int64"):
        dr.antialias(RAST, RAST, POS.long(), TRI)
    with pytest.raises(TypeError, match=r"tri must be torch\.int32, got torch\.float32"):
        dr.antialias(RAST, RAST, POS, TRI.float())
    with pytest.raises(TypeError, match=r"level 1 must be torch\.float32, got torch\.int32\.$"):
        ops._check(TRI, "level 1", ndim=2, dtype=torch.float32)
    with pytest.raises(TypeError, match=r"attr must be a torch\.Tensor, got list"):
        dr.interpolate(POS.tolist(), RAST, TRI)
    with pytest.raises(TypeError, match=r"rast_db must be a torch\.Tensor, got bool"):
        dr.interpolate(POS, RAST, TRI, rast_db=True)
    with pytest.raises(TypeError, match=r"pos must be a torch\.Tensor, got NoneType"):
        dr.antialias(RAST, RAST, None, TRI)
    with pytest.raises(TypeError, match=r"rast_db must be torch\.float32"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST.double())
    for boost in ("2", None, [1.0]):
        with pytest.raises(TypeError, match="pos_gradient_boost must be a number"):
            dr.antialias(RAST, RAST, POS, TRI, pos_gradient_boost=boost)


def test_diff_attrs():
    for bad in (1, 1.5, [0.5], [None]):
        with pytest.raises(TypeError, match="diff_attrs must be a sequence of channel indices"):
            dr.interpolate(POS, RAST, TRI, rast_db=RAST, diff_attrs=bad)
    with pytest.raises(ValueError, match="'all' or None, got 'ALL'"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST, diff_attrs="ALL")
    with pytest.raises(ValueError, match=r"diff_attrs \[4\] out of range for 4 channels"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST, diff_attrs=[4])
    assert ops._diff_channels(torch.tensor([2, 0]), 4) == [2, 0]
    assert ops._diff_channels(range(2, -1, -2), 4) == [2, 0]
    assert ops._diff_channels("all", 3) == [0, 1, 2] and ops._diff_channels(None, 3) == []
    with pytest.raises(ValueError, match="rast_db is required when diff_attrs is set.$"):
        dr.interpolate(POS, RAST, TRI, diff_attrs="all")
    with pytest.raises(ValueError, match="rast_db is required when diff_attrs is set, but the "
                                         "one given is empty"):
        dr.interpolate(POS, RAST, TRI, rast_db=RAST[..., :0], diff_attrs="all")
    with pytest.raises(ValueError, match=r"rast_db must have shape \[batch, height, width, 4\]"):
        dr.interpolate(POS, RAST, TRI, rast_db=torch.zeros(3))
    with pytest.raises(ValueError, match="attr batch size 3 does not match rast batch size 1"):
        dr.interpolate(torch.zeros(3, 3, 2), RAST, TRI)


def test_vertex_indices():
    tri = torch.tensor([[0, 1, 2], [2, 1, 3]], dtype=torch.int32)
    ops._check_indices(tri, 4)
    ops._check_indices(tri[:0], 0)
    with pytest.raises(ValueError, match="uv_idx refers to vertex 3, but valid indices are 0 to "
                                         "2 for 3 vertices"):
        ops._check_indices(tri, 3, name="uv_idx")
    with pytest.raises(ValueError, match=r"tri refers to vertex 3, but there are no vertices\.$"):
        ops._check_indices(tri, 0)
    with pytest.raises(ValueError, match="tri refers to vertex -1"):
        ops._check_indices(tri - 1, 4)
    with pytest.raises(ValueError, match="tri refers to vertex 2, but valid indices are 0 to 1"):
        dr.interpolate(torch.zeros(2, 2), RAST, TRI)
    with pytest.raises(ValueError, match="tri refers to vertex 2"):
        dr.antialias(torch.zeros(1, 8, 8, 3), RAST, POS[0, :2], TRI)


def test_index_range_found_once_per_tensor(monkeypatch):
    scans = []

    def compute(tri):
        scans.append(tri.shape[0])
        return ops._index_range(tri)

    monkeypatch.setattr(ops, "_index_ranges", TensorCache(compute))
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    for _ in range(3):
        ops._check_indices(tri, 3)
        ops._check_indices(tri, 40)
        with pytest.raises(ValueError):
            ops._check_indices(tri, 2)
    assert len(scans) == 1
    tri[0, 0] = 5
    with pytest.raises(ValueError, match="refers to vertex 5"):
        ops._check_indices(tri, 3)
    ops._check_indices(tri.clone(), 6)
    assert len(scans) == 3


def test_texture_messages():
    tex, uv = torch.zeros(1, 16, 16, 3), torch.zeros(1, 8, 8, 2)
    with pytest.raises(ValueError, match=r"Unknown filter_mode 'cubic'; expected one of"):
        dr.texture(tex, uv, filter_mode="cubic")
    with pytest.raises(ValueError, match=r"Unknown boundary_mode 'mirror'; expected one of"):
        dr.texture(tex, uv, boundary_mode="mirror")
    with pytest.raises(ValueError, match="filter_mode 'linear-mipmap-linear' requires uv_da or "
                                         "mip_level_bias"):
        dr.texture(tex, uv, filter_mode="linear-mipmap-linear")
    with pytest.raises(TypeError, match="mip must be a list of tensors or the result of "
                                        "texture_construct_mip, got Tensor"):
        dr.texture(tex, uv, mip=torch.zeros(1, 8, 8, 3))
    with pytest.raises(ValueError, match="mip_level_bias must match uv in batch, height and "
                                         "width"):
        dr.texture(tex, uv, mip_level_bias=torch.zeros(1, 8, 4))
    with pytest.raises(ValueError, match="uv_da must match uv in batch, height and width"):
        dr.texture(tex, uv, uv_da=torch.zeros(1, 8, 4, 4))
    with pytest.raises(ValueError, match="tex batch size 2 does not match uv batch size 1"):
        dr.texture(torch.zeros(2, 16, 16, 3), uv)
    with pytest.raises(ValueError, match=r"boundary_mode=\"cube\" needs tex to be a cube map"):
        dr.texture(tex, torch.zeros(1, 8, 8, 3), boundary_mode="cube")
    with pytest.raises(ValueError, match="at least one texel and one channel"):
        dr.texture(torch.zeros(1, 0, 16, 3), uv)
    with pytest.raises(ValueError, match=r"cube_mode=True needs tex to be a cube map"):
        dr.texture_construct_mip(tex, cube_mode=True)
    with pytest.raises(ValueError, match="mip level 1 has 2 channels but tex has 3"):
        dr.texture(tex, uv, uv_da=torch.zeros(1, 8, 8, 4), mip=[torch.zeros(1, 8, 8, 2)])
    with pytest.raises(ValueError, match="mip level 1 has batch size 3; expected 1 or that of "
                                         "tex, 1"):
        dr.texture(tex, uv, uv_da=torch.zeros(1, 8, 8, 4), mip=[torch.zeros(3, 8, 8, 3)])
    with pytest.raises(ValueError, match="max_mip_level must be non-negative, got -1"):
        dr.texture_construct_mip(tex, max_mip_level=-1)


def test_antialias_and_rasterize_messages():
    color = torch.zeros(1, 8, 8, 3)
    with pytest.raises(ValueError, match="pos batch size 2 does not match rast batch size 1"):
        dr.antialias(color, RAST, POS.expand(2, 3, 4), TRI)
    with pytest.raises(ValueError, match=r"pos must have shape \[batch, vertices, 4\] or "
                                         r"\[vertices, 4\]"):
        dr.antialias(color, RAST, POS[..., :3], TRI)
    ctx = dr.RasterizeContext("cpu")
    with pytest.raises(ValueError, match="ranges is required when pos has shape "
                                         r"\[vertices, 4\] \(range mode\)"):
        dr.rasterize(ctx, POS[0], TRI, (8, 8))
    with pytest.raises(ValueError, match=r"ranges\[1\] = \(start 1, count 1\) does not lie "
                                         "within the 1 triangles of tri"):
        dr.rasterize(ctx, POS[0], TRI, (8, 8),
                     ranges=torch.tensor([[0, 1], [1, 1]], dtype=torch.int32))
    with pytest.raises(ValueError, match=r"All inputs must be on the same device; got pos on "
                                         r"cpu, tri on meta"):
        dr.rasterize(ctx, POS, TRI.to("meta"), (8, 8))
    with pytest.raises(ValueError, match="pos is on cpu but the context is on meta"):
        dr.rasterize(dr.RasterizeContext("meta"), POS, TRI, (8, 8))


def test_contexts():
    with pytest.raises(TypeError, match="device must be a torch.device, a string or a GPU "
                                        "index, got 1.5"):
        dr.RasterizeContext(1.5)
    with pytest.raises(TypeError, match="device must be"):
        dr.RasterizeContext(True)
    with pytest.raises(ValueError, match="device must not be a negative GPU index, got -1"):
        dr.RasterizeContext(-1)
    ctx = dr.RasterizeContext("cpu")
    assert repr(ctx) == "RasterizeContext(device='cpu')" and ctx.output_db
    assert dr.RasterizeCudaContext is dr.RasterizeContext
    gl = dr.RasterizeGLContext(output_db=False, device="cpu")
    assert repr(gl) == "RasterizeGLContext(output_db=False, device='cpu')"
    assert gl.mode == "automatic" and gl.set_context() is None and gl.release_context() is None
    with pytest.raises(TypeError, match="output_db must be a bool, got 'cpu'; pass the device "
                                        "as device=..."):
        dr.RasterizeGLContext("cpu")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="no CUDA or ROCm device is available"):
            dr.RasterizeContext("cuda")
