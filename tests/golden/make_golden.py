"""Write golden input/output vectors from the reference diffrast (run in the build container only).

Usage: ``python tests/golden/make_golden.py /path/to/reference/src``

It imports the reference's pure-PyTorch backend (``src/diffrast/backends/reference.py``) and
records its outputs for behaviour that no closed form pins: triangle ids and ``rast`` across
depth layers of meshes in general position, antialias outputs and gradients, texture and cube
lookups with gradients, and silhouette classification. The fixtures are plain ``.npz`` arrays
(inputs and expected outputs); the tests load them with ``allow_pickle=False`` and compare the
oracle against them. Nothing here runs on the GPU machine.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def random_mesh(num_tri, gen, batch=1, z_range=0.9, w_range=(1.0, 2.0), xy_range=1.2):
    n = 3 * num_tri
    xy = (torch.rand(batch, n, 2, generator=gen) * 2 - 1) * xy_range
    z = (torch.rand(batch, n, 1, generator=gen) * 2 - 1) * z_range
    w = torch.rand(batch, n, 1, generator=gen) * (w_range[1] - w_range[0]) + w_range[0]
    pos = torch.cat([xy * w, z * w, w], -1)
    return pos, torch.arange(n, dtype=torch.int32).view(num_tri, 3)


def tiny_mesh(num_tri, gen, size, batch=1):
    centre = torch.rand(batch, num_tri, 1, 2, generator=gen) * 2.2 - 1.1
    offset = (torch.rand(batch, num_tri, 3, 2, generator=gen) * 2 - 1) * size
    xy = (centre + offset).reshape(batch, 3 * num_tri, 2)
    z = torch.rand(batch, 3 * num_tri, 1, generator=gen) * 1.8 - 0.9
    w = torch.rand(batch, 3 * num_tri, 1, generator=gen) + 1.0
    pos = torch.cat([xy * w, z * w, w], -1)
    return pos, torch.arange(3 * num_tri, dtype=torch.int32).view(num_tri, 3)


def raster_fixtures(ref):
    scenes = {
        "random": (random_mesh(120, torch.Generator().manual_seed(11)), (40, 56)),
        "crossing": (random_mesh(80, torch.Generator().manual_seed(12), w_range=(-1.0, 2.0)),
                     (48, 48)),
        "clipped": (random_mesh(100, torch.Generator().manual_seed(13), z_range=2.0,
                                xy_range=3.0), (37, 61)),
        "tiny": (tiny_mesh(1200, torch.Generator().manual_seed(14), 0.03), (48, 48)),
    }
    out = {}
    for name, ((pos, tri), res) in scenes.items():
        state = None
        out[f"{name}/pos"] = pos.numpy()
        out[f"{name}/tri"] = tri.numpy()
        out[f"{name}/res"] = np.array(res, dtype=np.int32)
        for layer in range(4):
            rast, rast_db, state = ref.rasterize_layer(pos, tri, res, True, state)
            out[f"{name}/rast{layer}"] = rast.numpy()
            if layer == 0:
                out[f"{name}/db0"] = rast_db.numpy()
    return out


def antialias_fixtures(ref):
    out = {}
    cases = {
        "plain": ({}, 1.0),
        "crossing": ({"w_range": (-1.0, 2.0)}, 1.0),
        "boost": ({}, 2.5),
    }
    for name, (mesh, boost) in cases.items():
        gen = torch.Generator().manual_seed(21)
        batch = 2 if name == "plain" else 1
        pos, tri = random_mesh(60, gen, batch=batch, **mesh)
        rast, _ = ref.rasterize(pos, tri, (36, 44), True)
        color = torch.rand(batch, 36, 44, 3, generator=gen)
        weights = torch.randn(batch, 36, 44, 3, generator=gen)
        c = color.clone().requires_grad_(True)
        p = pos.clone().requires_grad_(True)
        result = ref.antialias(c, rast, p, tri, boost)
        (result * weights).sum().backward()
        for key, value in (("pos", pos), ("tri", tri), ("rast", rast), ("color", color),
                           ("weights", weights), ("out", result.detach()), ("grad_color", c.grad),
                           ("grad_pos", p.grad)):
            out[f"{name}/{key}"] = value.numpy()
        out[f"{name}/boost"] = np.array(boost, dtype=np.float32)
    # Silhouettes of a closed mesh under a random projection, and of a folded strip.
    gen = torch.Generator().manual_seed(22)
    verts = torch.randn(40, 3, generator=gen)
    tri = torch.randint(0, 40, (90, 3), generator=gen, dtype=torch.int32)
    tri = tri[(tri[:, 0] != tri[:, 1]) & (tri[:, 1] != tri[:, 2]) & (tri[:, 0] != tri[:, 2])]
    pos = torch.cat([verts, torch.rand(40, 1, generator=gen) + 0.5], -1)[None]
    out["sil/pos"] = pos.numpy()
    out["sil/tri"] = tri.numpy()
    out["sil/neighbours"] = ref.edge_neighbours(tri).numpy()
    out["sil/silhouette"] = ref._silhouette_edges(pos, tri.long()).numpy()
    return out


def texture_fixtures(ref):
    out = {}
    gen = torch.Generator().manual_seed(31)
    tex = torch.randn(2, 13, 10, 3, generator=gen)
    uv = torch.rand(2, 8, 9, 2, generator=gen) * 1.6 - 0.3
    uv_da = torch.rand(2, 8, 9, 4, generator=gen) * 0.4 - 0.2
    bias = torch.rand(2, 8, 9, generator=gen) * 3 - 1
    weights = torch.randn(2, 8, 9, 3, generator=gen)
    out.update({"tex": tex.numpy(), "uv": uv.numpy(), "uv_da": uv_da.numpy(),
                "bias": bias.numpy(), "weights": weights.numpy()})
    for filt in ("nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear"):
        for boundary in ("wrap", "clamp", "zero"):
            mip = "mipmap" in filt
            inputs = [t.clone().requires_grad_(True) for t in (tex, uv, uv_da, bias)]
            result = ref.texture(inputs[0], inputs[1], inputs[2] if mip else None, filt,
                                 boundary, None, mip_level_bias=inputs[3] if mip else None)
            (result * weights).sum().backward()
            key = f"{filt}/{boundary}"
            out[f"{key}/out"] = result.detach().numpy()
            for name, t in zip(("tex", "uv", "uv_da", "bias"), inputs):
                g = t.grad if t.grad is not None else torch.zeros_like(t)
                out[f"{key}/grad_{name}"] = g.numpy()
    # Out-of-range and non-finite coordinates.
    special = torch.tensor([0.0, 1.0, -1e30, 1e30, float("inf"), -float("inf"), float("nan"),
                            -0.25, 1.75, 0.5])
    su, sv = torch.meshgrid(special, special, indexing="ij")
    suv = torch.stack([su, sv], -1)[None]
    out["special/uv"] = suv.numpy()
    for boundary in ("wrap", "clamp", "zero"):
        for filt in ("nearest", "linear"):
            out[f"special/{filt}/{boundary}"] = ref.texture(tex[:1], suv, None, filt, boundary,
                                                            None).numpy()
    # Cube map lookups.
    cube = torch.rand(1, 6, 8, 8, 3, generator=gen)
    dirs = torch.randn(2, 9, 7, 3, generator=gen)
    dirs[0, 0, 0] = torch.tensor([1.0, 1.0, 1.0])
    dirs[0, 0, 1] = torch.tensor([0.0, 0.0, 0.0])
    dirs[0, 0, 2] = torch.tensor([1.0, -1.0, 0.5])
    dirs_da = torch.randn(2, 9, 7, 6, generator=gen) * 0.2
    cweights = torch.randn(2, 9, 7, 3, generator=gen)
    out.update({"cube/tex": cube.numpy(), "cube/dirs": dirs.numpy(),
                "cube/dirs_da": dirs_da.numpy(), "cube/weights": cweights.numpy()})
    for filt in ("nearest", "linear", "linear-mipmap-linear"):
        mip = "mipmap" in filt
        inputs = [t.clone().requires_grad_(True) for t in (cube, dirs, dirs_da)]
        result = ref.texture(inputs[0], inputs[1], inputs[2] if mip else None, filt, "cube",
                             None)
        (result * cweights).sum().backward()
        out[f"cube/{filt}/out"] = result.detach().numpy()
        for name, t in zip(("tex", "dirs", "dirs_da"), inputs):
            g = t.grad if t.grad is not None else torch.zeros_like(t)
            out[f"cube/{filt}/grad_{name}"] = g.numpy()
    return out


def interpolate_fixtures(ref):
    gen = torch.Generator().manual_seed(41)
    pos, tri = random_mesh(80, gen, batch=2)
    rast, rast_db = ref.rasterize(pos, tri, (24, 28), True)
    attr = torch.randn(2, pos.shape[1], 5, generator=gen)
    weights = torch.randn(2, 24, 28, 5, generator=gen)
    weights_da = torch.randn(2, 24, 28, 4, generator=gen)
    inputs = [t.clone().requires_grad_(True) for t in (attr, rast, rast_db)]
    o, o_da = ref.interpolate(inputs[0], inputs[1], tri, inputs[2], [3, 0])
    ((o * weights).sum() + (o_da * weights_da).sum()).backward()
    data = {"attr": attr, "rast": rast, "rast_db": rast_db, "tri": tri, "weights": weights,
            "weights_da": weights_da, "out": o.detach(), "out_da": o_da.detach(),
            "grad_attr": inputs[0].grad, "grad_rast": inputs[1].grad,
            "grad_rast_db": inputs[2].grad}
    return {k: v.numpy() for k, v in data.items()}


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, src)
    from diffrast.backends import reference as ref

    assert Path(ref.__file__).resolve().is_relative_to(Path(src).resolve()), ref.__file__
    torch.set_num_threads(8)
    for name, make in (("raster", raster_fixtures), ("antialias", antialias_fixtures),
                       ("texture", texture_fixtures), ("interpolate", interpolate_fixtures)):
        data = make(ref)
        np.savez_compressed(HERE / f"{name}.npz", **data)
        size = (HERE / f"{name}.npz").stat().st_size
        print(f"{name}.npz: {len(data)} arrays, {size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
