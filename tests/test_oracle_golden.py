"""The oracle against golden vectors written by the reference itself (tests/golden).

tests/golden/make_golden.py imported the reference's pure-PyTorch backend in the build
container and recorded its outputs on seeded scenes; here the oracle must reproduce them:
triangle ids and every rast value bit for bit across four depth layers, and the other ops to
float32 rounding (1e-6 relative) with gradients.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as R

GOLDEN = Path(__file__).parent / "golden"


def load(name):
    return {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / f"{name}.npz").items()}


def close(a, b, tol=1e-6):
    a, b = a.double(), b.double()
    assert torch.equal(a.isnan(), b.isnan())
    err = ((a - b).nan_to_num().abs() / b.nan_to_num().abs().clamp_min(1)).max().item()
    assert err <= tol, err


@pytest.mark.parametrize("scene", ["random", "crossing", "clipped", "tiny"])
def test_rasterize_layers_bit_exact(scene):
    g = load("raster")
    pos, tri = g[f"{scene}/pos"], g[f"{scene}/tri"]
    res = tuple(int(v) for v in g[f"{scene}/res"])
    state = None
    for layer in range(4):
        rast, db, state = R.rasterize_layer(pos, tri, res, True, state)
        assert torch.equal(rast, g[f"{scene}/rast{layer}"]), layer
        if layer == 0:
            assert torch.equal(db, g[f"{scene}/db0"])


def test_interpolate_with_gradients():
    g = load("interpolate")
    ins = [g[k].clone().requires_grad_(True) for k in ("attr", "rast", "rast_db")]
    out, out_da = R.interpolate(ins[0], ins[1], g["tri"], ins[2], [3, 0])
    ((out * g["weights"]).sum() + (out_da * g["weights_da"]).sum()).backward()
    assert torch.equal(out, g["out"]) and torch.equal(out_da, g["out_da"])
    for t, key in zip(ins, ("grad_attr", "grad_rast", "grad_rast_db")):
        close(t.grad, g[key])


@pytest.mark.parametrize("boundary", ["wrap", "clamp", "zero"])
@pytest.mark.parametrize("filter_mode", ["nearest", "linear", "linear-mipmap-nearest",
                                         "linear-mipmap-linear"])
def test_texture_with_gradients(filter_mode, boundary):
    g = load("texture")
    mip = "mipmap" in filter_mode
    ins = [g[k].clone().requires_grad_(True) for k in ("tex", "uv", "uv_da", "bias")]
    out = R.texture(ins[0], ins[1], ins[2] if mip else None, filter_mode, boundary, None,
                    mip_level_bias=ins[3] if mip else None)
    (out * g["weights"]).sum().backward()
    key = f"{filter_mode}/{boundary}"
    close(out.detach(), g[f"{key}/out"])
    for t, name in zip(ins, ("tex", "uv", "uv_da", "bias")):
        grad = t.grad if t.grad is not None else torch.zeros_like(t)
        close(grad, g[f"{key}/grad_{name}"])


def test_texture_out_of_range_and_non_finite_coordinates():
    g = load("texture")
    for boundary in ("wrap", "clamp", "zero"):
        for filter_mode in ("nearest", "linear"):
            out = R.texture(g["tex"][:1], g["special/uv"], None, filter_mode, boundary, None)
            close(out, g[f"special/{filter_mode}/{boundary}"])


@pytest.mark.parametrize("filter_mode", ["nearest", "linear", "linear-mipmap-linear"])
def test_cube_map_with_gradients(filter_mode):
    g = load("texture")
    mip = "mipmap" in filter_mode
    ins = [g[f"cube/{k}"].clone().requires_grad_(True) for k in ("tex", "dirs", "dirs_da")]
    out = R.texture(ins[0], ins[1], ins[2] if mip else None, filter_mode, "cube", None)
    (out * g["cube/weights"]).sum().backward()
    close(out.detach(), g[f"cube/{filter_mode}/out"])
    for t, name in zip(ins, ("tex", "dirs", "dirs_da")):
        grad = t.grad if t.grad is not None else torch.zeros_like(t)
        close(grad, g[f"cube/{filter_mode}/grad_{name}"])


@pytest.mark.parametrize("case", ["plain", "crossing", "boost"])
def test_antialias_with_gradients(case):
    g = load("antialias")
    c = g[f"{case}/color"].clone().requires_grad_(True)
    p = g[f"{case}/pos"].clone().requires_grad_(True)
    out = R.antialias(c, g[f"{case}/rast"], p, g[f"{case}/tri"], float(g[f"{case}/boost"]))
    (out * g[f"{case}/weights"]).sum().backward()
    close(out.detach(), g[f"{case}/out"])
    close(c.grad, g[f"{case}/grad_color"])
    close(p.grad, g[f"{case}/grad_pos"])


def test_edge_adjacency_and_silhouettes():
    g = load("antialias")
    assert torch.equal(R.edge_neighbours(g["sil/tri"]), g["sil/neighbours"])
    assert torch.equal(R.silhouette_edges(g["sil/pos"], g["sil/tri"].long()), g["sil/silhouette"])
