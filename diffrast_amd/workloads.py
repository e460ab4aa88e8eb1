"""Synthetic scenes of the benchmark workloads: meshes, cameras and seeded inputs.

Meshes and cameras follow the conventions of the reference's examples (examples/common.py:
uv sphere by revolution, icosphere by midpoint subdivision, (p, q) torus knot, OpenGL
perspective and look-at). Everything is generated on the CPU from a seed and then moved to the
device, so a workload is identical on every machine.

Workloads (per-image resolution, images per batch):

* ``sphere``   -- uv sphere of 32 rings x 64 segments (3,968 triangles), 1 x 256x256,
  rasterize -> interpolate(colours) -> antialias -> MSE.
* ``textured`` -- icosphere(5) (20,480 triangles), 4 x 512x512, spherical uv with derivatives,
  a 512x512x3 texture with its mip stack rebuilt every step, trilinear wrap lookup,
  antialias, MSE; gradients to the texture and positions.
* ``large``    -- icosphere(8) (1,310,720 triangles) with radially perturbed vertices,
  8 x 1024x1024, 8 feature channels plus spherical uv, a 1024x1024x4 texture with a full mip
  chain built per call, trilinear lookup, antialias on the shaded colour, MSE; gradients to
  positions, features and texture.
* ``cubemap``  -- (2, 3) torus knot, 512 x 32 tube segments (32,768 triangles), 4 x 1024x1024,
  reflection vectors (and their derivatives, by the chain rule through the view rays and the
  interpolated normals) into a 6x512x512x3 cube map, antialias, MSE; gradients to the cube
  map and positions.
* ``instances`` -- 256 icosphere(4) instances (1,310,720 triangles) in range mode, 512x512,
  four depth layers, then antialias on layer 0.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch import Tensor

# ---------------------------------------------------------------------------------------------
# Meshes
# ---------------------------------------------------------------------------------------------


def uv_sphere(rings: int = 32, segments: int = 64) -> tuple[Tensor, Tensor]:
    """Unit sphere as a surface of revolution around y; single-vertex poles."""
    theta = torch.linspace(0, math.pi, rings + 1, dtype=torch.float64)
    phi = torch.arange(segments, dtype=torch.float64) * (2 * math.pi / segments)
    r, y = torch.sin(theta[1:-1])[:, None], torch.cos(theta[1:-1])[:, None]
    ring = torch.stack([r * torch.cos(phi), y.expand(-1, segments), -r * torch.sin(phi)], -1)
    verts = torch.cat([torch.tensor([[0.0, 1.0, 0.0]], dtype=torch.float64),
                       ring.reshape(-1, 3),
                       torch.tensor([[0.0, -1.0, 0.0]], dtype=torch.float64)])
    south = verts.shape[0] - 1

    def ring_vertex(i, s):  # ring i in [1, rings - 1]
        return 1 + (i - 1) * segments + s % segments

    faces = []
    for s in range(segments):
        faces.append([0, ring_vertex(1, s), ring_vertex(1, s + 1)])
        for i in range(1, rings - 1):
            a, b = ring_vertex(i, s), ring_vertex(i + 1, s)
            c, d = ring_vertex(i + 1, s + 1), ring_vertex(i, s + 1)
            faces += [[a, b, c], [a, c, d]]
        faces.append([ring_vertex(rings - 1, s), south, ring_vertex(rings - 1, s + 1)])
    return verts.float(), torch.tensor(faces, dtype=torch.int32)


def icosphere(subdivisions: int) -> tuple[Tensor, Tensor]:
    """Unit icosphere: an icosahedron whose faces are split in four, ``subdivisions`` times."""
    g = (1 + math.sqrt(5)) / 2
    verts = torch.tensor(
        [[-1, g, 0], [1, g, 0], [-1, -g, 0], [1, -g, 0], [0, -1, g], [0, 1, g], [0, -1, -g],
         [0, 1, -g], [g, 0, -1], [g, 0, 1], [-g, 0, -1], [-g, 0, 1]], dtype=torch.float64)
    faces = torch.tensor(
        [[0, 11, 5], [0, 5, 1], [0, 1, 7], [0, 7, 10], [0, 10, 11], [1, 5, 9], [5, 11, 4],
         [11, 10, 2], [10, 7, 6], [7, 1, 8], [3, 9, 4], [3, 4, 2], [3, 2, 6], [3, 6, 8],
         [3, 8, 9], [4, 9, 5], [2, 4, 11], [6, 2, 10], [8, 6, 7], [9, 8, 1]])
    verts = F.normalize(verts, dim=-1)
    for _ in range(subdivisions):
        n = verts.shape[0]
        edges = torch.cat([faces[:, [0, 1]], faces[:, [1, 2]], faces[:, [2, 0]]])
        edges = edges.sort(-1).values
        keys = edges[:, 0] * n + edges[:, 1]
        unique, inverse = torch.unique(keys, return_inverse=True)
        mids = F.normalize((verts[unique // n] + verts[unique % n]) / 2, dim=-1)
        m = (inverse + n).view(3, -1)
        a, b, c = faces.unbind(-1)
        ab, bc, ca = m
        faces = torch.cat([torch.stack([a, ab, ca], -1), torch.stack([b, bc, ab], -1),
                           torch.stack([c, ca, bc], -1), torch.stack([ab, bc, ca], -1)])
        verts = torch.cat([verts, mids])
    return verts.float(), faces.to(torch.int32)


def torus_knot(p: int = 2, q: int = 3, segments: int = 512, sides: int = 32,
               tube: float = 0.2) -> tuple[Tensor, Tensor]:
    """Tube around a (p, q) torus knot, scaled into the unit sphere."""
    def curve(t):
        r = 2 + torch.cos(q * t)
        return torch.stack([r * torch.cos(p * t), r * torch.sin(p * t), -torch.sin(q * t)], -1)

    t = torch.arange(segments, dtype=torch.float64) * (2 * math.pi / segments)
    h = 1e-4
    centre, ahead, behind = curve(t), curve(t + h), curve(t - h)
    tangent = F.normalize(ahead - behind, dim=-1)
    bend = ahead - 2 * centre + behind
    normal = F.normalize(bend - (bend * tangent).sum(-1, keepdim=True) * tangent, dim=-1)
    binormal = torch.linalg.cross(tangent, normal, dim=-1)
    angle = torch.arange(sides, dtype=torch.float64) * (2 * math.pi / sides)
    ring = torch.cos(angle)[:, None] * normal[:, None] + torch.sin(angle)[:, None] * binormal[:, None]
    verts = ((centre[:, None] + 3 * tube * ring) / (3 + 3 * tube)).reshape(-1, 3)
    i, j = torch.meshgrid(torch.arange(segments), torch.arange(sides), indexing="ij")
    i, j = i.flatten(), j.flatten()

    def index(a, b):
        return (a % segments) * sides + b % sides

    a, b, c, d = index(i, j), index(i + 1, j), index(i + 1, j + 1), index(i, j + 1)
    faces = torch.cat([torch.stack([a, c, b], -1), torch.stack([a, d, c], -1)])
    return verts.float(), faces.to(torch.int32)


def displaced_grid(num_tri: int) -> tuple[Tensor, Tensor, int]:
    """The reference's benchmark surface (benchmarks/bench_rasterize.py:19-29): a square grid
    over [-1, 1]^2 in the x-z plane, n x n cells of two triangles with n = round(sqrt(num_tri /
    2)), raised to y = 0.1 sin(6x) cos(5z). Vertices row by row ((n + 1) per row, x fastest);
    triangles as the reference lists them, first (a, b, d) of every cell, then (a, d, c), where
    a, b are a cell's corners on its first row and c, d those on the next. Returns the vertices
    [(n + 1)^2, 3], the triangles and n."""
    n = max(1, round(math.sqrt(num_tri / 2)))
    line = torch.linspace(-1, 1, n + 1)
    z, x = (g.reshape(-1) for g in torch.meshgrid(line, line, indexing="ij"))
    verts = torch.stack([x, 0.1 * torch.sin(6 * x) * torch.cos(5 * z), z], -1)
    corner = (torch.arange(n)[:, None] * (n + 1) + torch.arange(n)[None, :]).reshape(-1)
    a, b, c, d = corner, corner + 1, corner + n + 1, corner + n + 2
    tri = torch.cat([torch.stack([a, b, d], -1), torch.stack([a, d, c], -1)])
    return verts, tri.to(torch.int32), n


def grid_views(verts: Tensor, views: int) -> Tensor:
    """Clip-space positions [views, vertices, 4] of the grid seen as in the reference's
    benchmark (benchmarks/bench_rasterize.py:31-52): view i turns the grid by 2 pi i / views
    about y, moves it by (0, -0.6, 2.2) and projects with focal length 1.5, near 0.1 and far 10,
    w being the camera-space z (the camera looks along +z)."""
    focal, near, far = 1.5, 0.1, 10.0
    out = []
    for i in range(views):
        angle = 2 * math.pi * i / max(views, 1)
        c, s = math.cos(angle), math.sin(angle)
        x, y, z = verts.unbind(-1)
        cx, cy, cz = c * x + s * z, y - 0.6, c * z - s * x + 2.2
        depth = (far + near) / (far - near) * cz - 2 * far * near / (far - near)
        out.append(torch.stack([focal * cx, focal * cy, depth, cz], -1))
    return torch.stack(out)


def grid_uv(n: int) -> Tensor:
    """Planar texture coordinates of the grid's vertices [(n + 1)^2, 2]: (column, row) / n."""
    line = torch.linspace(0, 1, n + 1)
    v, u = torch.meshgrid(line, line, indexing="ij")
    return torch.stack([u, v], -1).reshape(-1, 2)


def vertex_normals(verts: Tensor, faces: Tensor) -> Tensor:
    """Area-weighted vertex normals."""
    f = faces.long()
    v0, v1, v2 = verts[f[:, 0]], verts[f[:, 1]], verts[f[:, 2]]
    face_n = torch.linalg.cross(v1 - v0, v2 - v0, dim=-1)
    acc = torch.zeros_like(verts).index_add_(0, f.flatten(), face_n.repeat_interleave(3, 0))
    return F.normalize(acc, dim=-1)


def spherical_uv(verts: Tensor) -> Tensor:
    """u = 0.5 + atan2(z, x) / 2 pi, v = acos(y) / pi of unit-sphere directions."""
    n = F.normalize(verts, dim=-1)
    u = 0.5 + torch.atan2(n[:, 2], n[:, 0]) / (2 * math.pi)
    v = torch.acos(n[:, 1].clamp(-1, 1)) / math.pi
    return torch.stack([u, v], -1)


# ---------------------------------------------------------------------------------------------
# Cameras
# ---------------------------------------------------------------------------------------------


def perspective(fov_y: float, aspect: float, near: float = 0.1, far: float = 20.0) -> Tensor:
    """OpenGL projection matrix for a vertical field of view in degrees."""
    f = 1 / math.tan(math.radians(fov_y) / 2)
    return torch.tensor([[f / aspect, 0, 0, 0], [0, f, 0, 0],
                         [0, 0, (far + near) / (near - far), 2 * far * near / (near - far)],
                         [0, 0, -1, 0]], dtype=torch.float32)


def look_at(eye: Tensor) -> Tensor:
    """View matrices [batch, 4, 4] of cameras at ``eye`` [batch, 3] facing the origin, up +y."""
    up = eye.new_tensor([0.0, 1.0, 0.0]).expand_as(eye)
    forward = F.normalize(-eye, dim=-1)
    right = F.normalize(torch.linalg.cross(forward, up, dim=-1), dim=-1)
    true_up = torch.linalg.cross(right, forward, dim=-1)
    rot = torch.stack([right, true_up, -forward], -2)
    view = torch.eye(4).repeat(eye.shape[0], 1, 1)
    view[:, :3, :3] = rot
    view[:, :3, 3] = -(rot @ eye[..., None]).squeeze(-1)
    return view


def random_eyes(count: int, radius: float, gen: torch.Generator) -> Tensor:
    """Camera positions at ``radius`` in seed-random directions, not looking along +-y."""
    eyes = []
    while len(eyes) < count:
        d = F.normalize(torch.randn(3, generator=gen), dim=0)
        if abs(float(d[1])) <= 0.99:
            eyes.append(d * radius)
    return torch.stack(eyes)


def clip_positions(verts: Tensor, eyes: Tensor, aspect: float) -> Tensor:
    """Clip-space positions [batch, vertices, 4] of ``verts`` seen from each eye."""
    matrix = perspective(45.0, aspect) @ look_at(eyes)
    homogeneous = F.pad(verts, (0, 1), value=1.0)
    return (homogeneous @ matrix.transpose(-1, -2)).contiguous()


def view_rays(eyes: Tensor, h: int, w: int) -> tuple[Tensor, Tensor]:
    """Unit world-space view rays through the pixel centres of each camera [batch, h, w, 3] and
    their derivatives per pixel step [batch, h, w, 6], laid out like interpolate's ``out_da``
    ((d/dx, d/dy) of each component in turn). The derivatives are exact (forward-mode
    differentiation of the ray through the inverse view-projection, one pixel = 2 / size in
    NDC)."""
    inv = torch.linalg.inv(perspective(45.0, w / h) @ look_at(eyes)).double()
    xs = (torch.arange(w, dtype=torch.float64) * 2 + 1) / w - 1
    ys = (torch.arange(h, dtype=torch.float64) * 2 + 1) / h - 1
    gy, gx = (g.contiguous() for g in torch.meshgrid(ys, xs, indexing="ij"))

    def ray(x, y):
        ndc = torch.stack([x, y, torch.ones_like(x), torch.ones_like(x)], -1)
        far = torch.einsum("bij,hwj->bhwi", inv, ndc)
        return F.normalize(far[..., :3] / far[..., 3:] - eyes.double()[:, None, None], dim=-1)

    view, dx = torch.func.jvp(lambda x: ray(x, gy), (gx,), (torch.full_like(gx, 2.0 / w),))
    _, dy = torch.func.jvp(lambda y: ray(gx, y), (gy,), (torch.full_like(gy, 2.0 / h),))
    view_da = torch.stack([dx, dy], -1).reshape(*view.shape[:-1], 6)
    return view.float().contiguous(), view_da.float().contiguous()


def reflect(view: Tensor, view_da: Tensor, n: Tensor, n_da: Tensor) -> tuple[Tensor, Tensor]:
    """Reflection r = v - 2 (n . v) n of the view rays about the interpolated normals, and its
    screen-space derivatives by the chain rule from those of both the rays and the normals
    (layouts of interpolate's ``out_da``: (d/dx, d/dy) per component)."""
    d = (view * n).sum(-1, keepdim=True)
    dirs = view - 2 * d * n
    # The derivatives as [..., component, axis], both axes at once (no strided slices).
    dv, dn = view_da.unflatten(-1, (3, 2)), n_da.unflatten(-1, (3, 2))
    dd = (dv * n[..., None]).sum(-2) + (view[..., None] * dn).sum(-2)  # [..., axis]
    dirs_da = dv - 2 * (dd[..., None, :] * n[..., None] + d[..., None] * dn)
    return dirs, dirs_da.flatten(-2)


# ---------------------------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------------------------


@dataclass
class Workload:
    name: str
    batch: int
    resolution: tuple[int, int]
    tensors: dict = field(default_factory=dict)
    # Scale used to shrink a workload for quick tests; 1 is the benchmark size.
    note: str = ""


def build(name: str, device: torch.device | str = "cpu", scale: int = 1) -> Workload:
    """Inputs of workload ``name``; ``scale`` divides the resolution (for tests)."""
    builders = {"sphere": _sphere, "textured": _textured, "large": _large,
                "cubemap": _cubemap, "instances": _instances}
    if name not in builders:
        raise ValueError(f"unknown workload {name!r}; expected one of {sorted(builders)}")
    w = builders[name](scale)
    w.tensors = {k: (v.to(device) if isinstance(v, Tensor) else v) for k, v in w.tensors.items()}
    return w


def _sphere(scale):
    gen = torch.Generator().manual_seed(0)
    verts, tri = uv_sphere(32, 64)
    h = w = 256 // scale
    pos = clip_positions(verts * 1.0, random_eyes(1, 3.0, gen), w / h)
    attr = torch.rand(1, verts.shape[0], 3, generator=gen)
    target = torch.rand(1, h, w, 3, generator=gen)
    return Workload("sphere", 1, (h, w), {"pos": pos, "tri": tri, "attr": attr,
                                          "target": target})


def _textured(scale):
    gen = torch.Generator().manual_seed(2)
    verts, tri = icosphere(5)
    h = w = 512 // scale
    pos = clip_positions(verts, random_eyes(4, 3.0, gen), w / h)
    tex = torch.rand(1, 512 // scale, 512 // scale, 3, generator=gen)
    target = torch.rand(4, h, w, 3, generator=gen)
    return Workload("textured", 4, (h, w), {"pos": pos, "tri": tri, "uv": spherical_uv(verts),
                                            "tex": tex, "target": target})


def _large(scale):
    gen = torch.Generator().manual_seed(1)
    verts, tri = icosphere(8)
    verts = verts * (1 + 0.02 * torch.randn(verts.shape[0], 1, generator=gen))
    h = w = 1024 // scale
    pos = clip_positions(verts, random_eyes(8, 3.0, gen), w / h)
    feat = torch.randn(1, verts.shape[0], 8, generator=gen)
    tex = torch.rand(1, 1024 // scale, 1024 // scale, 4, generator=gen)
    target = torch.rand(8, h, w, 4, generator=gen)
    return Workload("large", 8, (h, w), {"pos": pos, "tri": tri, "feat": feat,
                                         "uv": spherical_uv(verts)[None], "tex": tex,
                                         "target": target})


def _cubemap(scale):
    gen = torch.Generator().manual_seed(4)
    verts, tri = torus_knot(2, 3, 512, 32)
    h = w = 1024 // scale
    eyes = random_eyes(4, 3.0, gen)
    pos = clip_positions(verts, eyes, w / h)
    cube = torch.rand(1, 6, 512 // scale, 512 // scale, 3, generator=gen)
    target = torch.rand(4, h, w, 3, generator=gen)
    view, view_da = view_rays(eyes, h, w)
    return Workload("cubemap", 4, (h, w), {"pos": pos, "tri": tri,
                                           "normals": vertex_normals(verts, tri)[None],
                                           "view": view, "view_da": view_da, "cube": cube,
                                           "target": target})


def _instances(scale):
    gen = torch.Generator().manual_seed(5)
    verts, faces = icosphere(4)
    count = 256
    offset = torch.rand(count, 1, 3, generator=gen) * 2 - 1
    size = torch.rand(count, 1, 1, generator=gen) * 0.3 + 0.2
    world = (verts[None] * size + offset).reshape(-1, 3)
    tri = (faces[None] + torch.arange(count)[:, None, None] * verts.shape[0]).reshape(-1, 3)
    h = w = 512 // scale
    pos = clip_positions(world, random_eyes(1, 4.0, gen), w / h)[0]
    per = faces.shape[0]
    ranges = torch.tensor([[per * i, per * min(4, count - i)] for i in range(count)],
                          dtype=torch.int32)
    color = torch.rand(count, h, w, 3, generator=gen)
    return Workload("instances", count, (h, w), {"pos": pos, "tri": tri.to(torch.int32),
                                                 "ranges": ranges, "color": color})
