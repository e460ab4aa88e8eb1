"""Benchmark: ms per forward+backward render of the four-op pipeline on one MI355X.

Default workload (the headline configuration, ``--workload large``): icosphere(8), 1,310,720
triangles, radially perturbed, 8 views at 1024x1024. One step is

    rasterize -> interpolate(features [1, V, 8]) and interpolate(uv, rast_db, 'all')
    -> texture(1024x1024x4, full mip chain built in the call, trilinear, wrap)
    -> shade = colour + 0.1 * (f[..., 0:4] + f[..., 4:8]) -> antialias -> MSE -> backward

with gradients to positions, features and texture. ``--workload`` selects one of the other
four configurations (``make_step`` shows each step) and ``--all-workloads`` runs all five, one
JSON line each. Inputs are synthetic and resident on the GPU before timing starts.

Timing: the first two of the ``--warmup`` untimed steps are timed one by one as the first-call
costs (``first_call``); ``--steps`` steps are timed back to back between synchronisations
(``value``); then ``--repeats`` individually synchronised steps give the median, p10 and p90
(``synced_steps``, the reference benchmarks' rule).

Per-kernel time: HIP events around the C-ABI entry points, on the stream they launch on (in the
timed steps only around the dominant one; every entry point in 15 further steps for the
per-kernel and per-op tables, with each op's p10 and p90 over those steps). Algorithmic bytes
are the unique-byte model of ``BytesModel``: every input read once and every output written
once, from each call's own arguments. ``roofline`` reports the longest-running entry point that
launches a single kernel (so that its event time is that kernel's duration): its unique bytes
per launch over its mean duration, against 8 TB/s; its vector issue against the issue peak
(``valu``, from the committed counter summary); each op's forward+backward time against the HBM
time of its unique bytes (``ops``); the whole step against the four ops' bytes (``step``); and
the device atomics of the backward scatters (``atomics``, from the committed counter summary,
rated over the live launch times). ``traffic`` is the HBM bytes per launch measured for that
kernel with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE, each scaled by the counter's reading
for a copy of known size), from ``profiles/kernels.<workload>.pmc.txt`` when present.
``--graph`` times a step captured in a HIP graph and replayed, the loss reduction outside the
graph (the eager time stays in the line as ``eager_ms_per_step``).

CPU baseline: the oracle (a pure-PyTorch restatement of the reference backend) on the host
cores, the whole step where its brute-force visibility is small enough (the sphere and textured
workloads), else a bounded sample of the same workload -- one image, its visibility over a
subset of the triangles and the rest of the pipeline in full -- extrapolated linearly to all
triangles, layers and images.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from collections import defaultdict
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import diffrast_amd as dr  # noqa: E402
from diffrast_amd import workloads  # noqa: E402
from diffrast_amd.backends import hip  # noqa: E402

HBM_PEAK = 8.0e12  # bytes/s, MI355X
METRIC = "ms per fwd+bwd render (4-op pipeline) at 8×1024², 1.3M tris; % HBM roofline"


# Entry points that launch exactly one kernel, and that kernel. (dr_interpolate_backward
# launches interp_bwd_kernel with an attribute gradient and interp_bwd_rast_kernel without.)
SINGLE_KERNEL = {
    "dr_raster_visibility_tiles": "raster_tile_kernel",
    "dr_resolve_forward": "resolve_fwd_kernel",
    "dr_resolve_backward": "resolve_bwd_kernel",
    "dr_interpolate_forward": "interp_fwd_kernel",
    "dr_texture_forward": "tex_fwd_kernel",
    "dr_texture_backward": "tex_bwd_kernel",
    "dr_antialias_backward": "aa_bwd_kernel",
}


class KernelTimer:
    """HIP events around the backend's C-ABI calls, on the current stream, with the algorithmic
    bytes of each call: its kernel's own (``kernel_bytes``) and its share of its op's
    (``op_bytes``). Each event pair is tagged with ``step_index`` at the time of the call."""

    def __init__(self, model):
        self.model = model
        self.active = False
        self.only = None  # entry point names to time (None: every one)
        self.step_index = 0
        self._call = hip.call
        self.reset()

    def reset(self):
        self.events = defaultdict(list)
        self.bytes = defaultdict(float)
        self.op_bytes = defaultdict(float)

    def install(self):
        def timed(name, *args):
            if (not self.active or name.endswith("_size")
                    or (self.only is not None and name not in self.only)):
                return self._call(name, *args)  # (size queries launch nothing)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            self._call(name, *args)
            end.record()
            self.events[name].append((start, end, self.step_index))
            self.bytes[name] += self.model.kernel_bytes(name, args)
            self.op_bytes[name] += self.model.op_bytes(name, args)

        hip.call = timed

    def uninstall(self):
        hip.call = self._call

    def summary(self):
        """name -> (total ms, launches)."""
        torch.cuda.synchronize()
        out = {}
        for name, pairs in self.events.items():
            times = [s.elapsed_time(e) for s, e, _ in pairs]
            out[name] = (sum(times), len(times))
        return out

    def per_step(self, names) -> dict[int, float]:
        """step index -> ms of the entry points ``names`` in that step."""
        torch.cuda.synchronize()
        out = defaultdict(float)
        for name in names:
            for s, e, index in self.events.get(name, ()):
                out[index] += s.elapsed_time(e)
        return out


def _struct(arg):
    """The ctypes structure a byref() argument points to."""
    return arg._obj


# The entry points that find visibility (the keys), before the resolve.
VISIBILITY_ENTRIES = ("dr_raster_visibility_begin", "dr_raster_visibility_start",
                      "dr_raster_visibility_bin", "dr_raster_visibility_tiles",
                      "dr_raster_visibility", "dr_raster_visibility_overflow",
                      "dr_raster_visibility_static", "dr_raster_order")

# Which of the four ops each C-ABI entry point belongs to (its event time counts there).
OP_OF = {
    "dr_raster_visibility_begin": "rasterize",
    "dr_raster_visibility_start": "rasterize",
    "dr_raster_visibility_bin": "rasterize",
    "dr_raster_visibility_tiles": "rasterize",
    "dr_raster_visibility": "rasterize",
    "dr_raster_visibility_overflow": "rasterize",
    "dr_raster_visibility_static": "rasterize",
    "dr_raster_order": "rasterize",
    "dr_resolve_forward": "rasterize",
    "dr_resolve_backward": "rasterize",
    "dr_interpolate_forward": "interpolate",
    "dr_interpolate_backward": "interpolate",
    "dr_texture_forward": "texture",
    "dr_texture_backward": "texture",
    "dr_mip_build": "texture",
    "dr_mip_build_backward": "texture",
    "dr_edge_neighbours": "antialias",
    "dr_silhouette_mask": "antialias",
    "dr_antialias_forward": "antialias",
    "dr_antialias_backward": "antialias",
}


class BytesModel:
    """Algorithmic bytes: the unique-byte model -- every input tensor read once and every output
    written once, 4 B per fp32 value, 12 B per triangle of ``tri``, 24 B per triangle of int64
    edge neighbours, gathered arrays (pos, tri, attributes, texels) counted whole -- from each
    call's own arguments and the workload's mesh sizes. With P pixels, Pb images of ``pos``, V
    vertices, T triangles, C channels, D derivative channels, L texels of the packed mip chain
    and N0 of its base level, the op formulas are

        rasterize fwd    Pb V 16 + T 12 + P 16 (1 + [rast_db])
        rasterize bwd    P 16 (1 + [rast_db]) + P 8 (keys) + 2 Pb V 16 + T 12
        interpolate fwd  P 16 (1 + [D>0]) + T 12 + V C 4 + P C 4 + P 2D 4
        interpolate bwd  P C 4 + P 2D 4 + 2 P 16 (1 + [D>0]) + T 12 + 2 V C 4
        texture fwd      L C 4 + P (coords + derivatives) 4 + P C 4 + mip build L C 4
        texture bwd      P C 4 + 2 P (coords + derivatives) 4 + 2 L C 4 + mip adjoint L C 4
        antialias fwd    2 P C 4 + P 16 + Pb V 16 + T 12 + T 24
        antialias bwd    3 P C 4 + P 16 + 2 Pb V 16 + T 12 + T 24

    (coordinates: 2 and 4 derivative values per pixel for a 2D texture, 3 and 6 for a cube
    map; a per-pixel mip level bias adds P 4). ``op_bytes`` gives each entry point's share of
    its op (the visibility passes carry none: rasterize's bytes sit on the resolve calls).
    ``kernel_bytes`` gives the unique bytes of the work a single-kernel entry point does, for
    the per-kernel roofline: the tile pass of the visibility is credited with the whole
    visibility's unique bytes (pos and tri read, the keys written, the previous layer's keys
    read when peeling), since its setup and binning passes move only intermediate data."""

    def __init__(self, w):
        pos = w.tensors["pos"]
        self.vertices = pos.shape[-2]
        self.tri = w.tensors["tri"].shape[0]

    def pos_bytes(self, g_or_a) -> int:
        images = g_or_a.batch if g_or_a.pos_batch_stride else 1
        return images * self.vertices * 16

    @staticmethod
    def _pixels(a):
        return a.batch * a.height * a.width

    def op_bytes(self, name, args):
        model = getattr(self, "op_" + name[3:], None)
        return 0 if model is None else model(args)

    def kernel_bytes(self, name, args):
        if name == "dr_raster_visibility_tiles":
            g = _struct(args[0])
            P = self._pixels(g)
            return self.pos_bytes(g) + self.tri * 12 + P * 8 * (2 if args[1] else 1)
        return self.op_bytes(name, args)

    def op_resolve_forward(self, args):
        g = _struct(args[0])
        P = self._pixels(g)
        return self.pos_bytes(g) + self.tri * 12 + P * 16 * (2 if args[3] else 1)

    def op_resolve_backward(self, args):
        g = _struct(args[0])
        P = self._pixels(g)
        return P * 16 * (2 if args[3] else 1) + P * 8 + 2 * self.pos_bytes(g) + self.tri * 12

    @staticmethod
    def _interp(a):
        P, C, D = a.batch * a.height * a.width, a.channels, a.num_diff
        attr = (a.batch if a.attr_batch_stride else 1) * a.num_vertices * C * 4
        return P, C, D, attr, P * 16 * (2 if D else 1)

    def op_interpolate_forward(self, args):
        P, C, D, attr, rast = self._interp(_struct(args[0]))
        return rast + self.tri * 12 + attr + P * C * 4 + P * 2 * D * 4

    def op_interpolate_backward(self, args):
        P, C, D, attr, rast = self._interp(_struct(args[0]))
        return P * C * 4 + P * 2 * D * 4 + 2 * rast + self.tri * 12 + 2 * attr

    @staticmethod
    def _texture(a):
        P, C = a.batch * a.height * a.width, a.channels
        cube = a.boundary == hip.BOUNDARIES["cube"]
        coords = P * (12 if cube else 8) + (P * (24 if cube else 16) if a.uv_da else 0)
        coords += P * 4 if a.bias else 0
        return P, C, coords, a.tex_batch * a.num_texels * C * 4

    def op_texture_forward(self, args):
        P, C, coords, texels = self._texture(_struct(args[0]))
        return texels + coords + P * C * 4

    def op_texture_backward(self, args):
        P, C, coords, texels = self._texture(_struct(args[0]))
        return P * C * 4 + 2 * coords + 2 * texels

    def op_mip_build(self, args):
        tex_batch, channels, total = args[2], args[3], args[4]
        return tex_batch * total * channels * 4  # base read, levels written

    def op_mip_build_backward(self, args):
        tex_batch, channels, total = args[1], args[2], args[3]
        return tex_batch * total * channels * 4  # the adjoint

    def _aa(self, args):
        a = _struct(args[0])
        P, C = self._pixels(a), a.channels
        return P, C, self.pos_bytes(a), a.num_tri

    def op_antialias_forward(self, args):
        P, C, pos, T = self._aa(args)
        return 2 * P * C * 4 + P * 16 + pos + T * 12 + T * 24

    def op_antialias_backward(self, args):
        P, C, pos, T = self._aa(args)
        return 3 * P * C * 4 + P * 16 + 2 * pos + T * 12 + T * 24


# ---- the five workloads' steps ----------------------------------------------------------------

class _MSE(torch.autograd.Function):
    """mean((x - target)^2) with a gradient for x only: the difference once (kept for the
    backward pass) and its squared norm (one reduction pass; the BLAS dot product takes twice
    as long at 2 x 10^8 values); the backward pass scales the difference. Three full-size
    passes (the library form takes six launches and five passes)."""

    @staticmethod
    def forward(ctx, x, target):
        d = torch.sub(x, target)
        ctx.save_for_backward(d)
        flat = d.view(-1)
        return torch.linalg.vector_norm(flat).square().div_(flat.numel())

    @staticmethod
    def backward(ctx, g):
        (d,) = ctx.saved_tensors
        return torch.mul(d, g * (2.0 / d.numel())), None


def _mse(x, target):
    return _MSE.apply(x, target)


class _Shade(torch.autograd.Function):
    """col + 0.1 * (f[..., :4] + f[..., 4:]) for 8-channel features, in two launches: the two
    halves summed, then scaled and added to col in one kernel; the backward pass writes 0.1 * g
    into both halves of the feature gradient in one kernel (autograd through the expression
    takes five launches forward and a strided copy backward)."""

    @staticmethod
    def forward(ctx, col, f):
        return torch.add(col, f[..., :4] + f[..., 4:], alpha=0.1)

    @staticmethod
    def backward(ctx, g):
        halves = g.unsqueeze(-2).expand(*g.shape[:-1], 2, g.shape[-1])
        return g, torch.mul(halves, 0.1).flatten(-2)


class Step:
    """One forward+backward step of a workload on the GPU: ``render()`` runs the four ops and
    returns the final image and its target; ``__call__`` computes the MSE loss
    mean((image - target)^2) and runs the backward pass from it: the render's backward seeded
    with the loss's gradient 2 (image - target) / n, as ``loss.backward()`` would (the same
    values; seeding through autograd would scale by a one-element device tensor, which
    PyTorch does in a non-vectorized kernel over the whole image). ``leaves`` are the tensors
    that receive gradients."""

    def __init__(self, render, leaves):
        self.render, self.leaves = render, leaves

    def __call__(self):
        for x in self.leaves:
            x.grad = None
        image, target = self.render()
        diff = torch.sub(image, target)
        loss = _loss_of(diff)
        image.backward(torch.mul(diff, 2.0 / diff.numel()))
        return loss


def make_step(w, device) -> Step:
    """One forward+backward step of workload ``w`` on the GPU (inputs copied to ``device``)."""
    # Range tables stay on the host, as nvdiffrast takes them (reading them needs no device
    # synchronisation, so the step can be captured in a HIP graph).
    t = {k: (v.to(device) if isinstance(v, torch.Tensor) and k != "ranges" else v)
         for k, v in w.tensors.items()}
    ctx = dr.RasterizeContext(device)
    res = w.resolution
    leaves = []

    def leaf(name):
        x = t[name].requires_grad_(True)
        leaves.append(x)
        return x

    if w.name == "sphere":
        pos, attr = leaf("pos"), leaf("attr")
        tri, target = t["tri"], t["target"]

        def render():
            rast, _ = dr.rasterize(ctx, pos, tri, res, grad_db=False)
            col, _ = dr.interpolate(attr, rast, tri)
            return dr.antialias(col, rast, pos, tri), target
    elif w.name == "textured":
        pos, tex = leaf("pos"), leaf("tex")
        tri, uv_attr, target = t["tri"], t["uv"], t["target"]

        def render():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            uv, uv_da = dr.interpolate(uv_attr, rast, tri, rast_db, diff_attrs="all")
            mip = dr.texture_construct_mip(tex)
            col = dr.texture(tex, uv, uv_da, mip=mip, filter_mode="linear-mipmap-linear",
                             boundary_mode="wrap")
            return dr.antialias(col, rast, pos, tri), target
    elif w.name == "large":
        pos, feat, tex = leaf("pos"), leaf("feat"), leaf("tex")
        tri, uv_attr, target = t["tri"], t["uv"], t["target"]

        def render():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            f, _ = dr.interpolate(feat, rast, tri)
            st, st_da = dr.interpolate(uv_attr, rast, tri, rast_db, diff_attrs="all")
            col = dr.texture(tex, st, st_da, filter_mode="linear-mipmap-linear",
                             boundary_mode="wrap")
            shaded = _Shade.apply(col, f)  # col + 0.1 * (f[..., :4] + f[..., 4:])
            return dr.antialias(shaded, rast, pos, tri), target
    elif w.name == "cubemap":
        pos, cube = leaf("pos"), leaf("cube")
        tri, normals, target = t["tri"], t["normals"], t["target"]
        view, view_da = t["view"], t["view_da"]

        def render():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            n, n_da = dr.interpolate(normals, rast, tri, rast_db, diff_attrs="all")
            dirs, dirs_da = workloads.reflect(view, view_da, n, n_da)
            col = dr.texture(cube, dirs, dirs_da, filter_mode="linear-mipmap-linear",
                             boundary_mode="cube")
            return dr.antialias(col, rast, pos, tri), target
    elif w.name == "instances":
        pos, color = leaf("pos"), leaf("color")
        tri, ranges = t["tri"], t["ranges"]
        target = torch.zeros_like(color)

        def render():
            with dr.DepthPeeler(ctx, pos, tri, res, ranges=ranges) as peeler:
                layers = [peeler.rasterize_next_layer()[0] for _ in range(4)]
            return dr.antialias(color, layers[0], pos, tri), target
    else:
        raise ValueError(w.name)
    return Step(render, leaves)


def image_ids(w, device, images: int = 1):
    """Triangle ids [images, H, W] (-1: none) of the first images (range mode: item 0's first
    layer), from the GPU, for the CPU baseline's rest-of-pipeline leg."""
    t = w.tensors
    ctx = dr.RasterizeContext(device)
    with torch.no_grad():
        if w.name == "instances":
            rast, _ = dr.rasterize(ctx, t["pos"].to(device), t["tri"].to(device),
                                   w.resolution, ranges=t["ranges"][:images])
        else:
            rast, _ = dr.rasterize(ctx, t["pos"][:images].to(device), t["tri"].to(device),
                                   w.resolution)
    return (rast[..., 3].long() - 1).cpu()


def host_threads() -> tuple[int, int]:
    """(threads to use, cores this process may run on): the affinity count, limited by
    OMP_NUM_THREADS where the environment sets it (a machine's share of cores for this job)."""
    affinity = len(os.sched_getaffinity(0))
    limit = os.environ.get("OMP_NUM_THREADS")
    threads = min(affinity, int(limit)) if limit and limit.isdigit() and int(limit) > 0 \
        else affinity
    return threads, affinity


def cpu_baseline(w, sample_tris: int, device, full_work: float) -> dict:
    """The oracle on the host. Where the visibility's brute force (images x triangles x pixels
    evaluations) is at most ``full_work``, the whole step on every image, median of up to three
    individually timed runs; beyond it, one image's brute-force visibility over a sample of its
    triangles and the rest of the pipeline forward and backward on that image in full (with the
    true visibility), extrapolated linearly to all triangles, layers and images (the
    reference's own skip rule, benchmarks/bench_pipeline.py:56, :73-75)."""
    from oracle import reference as R

    threads, affinity = host_threads()
    torch.set_num_threads(threads)
    t = w.tensors
    (H, W), B = w.resolution, w.batch
    tri = t["tri"]
    layers = 1
    if w.name == "instances":
        start, count = (int(v) for v in t["ranges"][0])
        own = tri[start:start + count]
        layers = 4
    else:
        own = tri
    T = own.shape[0]
    full = w.name != "instances" and B * T * H * W <= full_work
    images = B if full else 1
    ids = image_ids(w, device, images)
    pos_n = t["pos"][None] if w.name == "instances" else t["pos"][:images].clone()
    sample = T if full else min(sample_tris, T)
    keep = torch.randperm(T, generator=torch.Generator().manual_seed(0))[:sample]
    sub = own if full else own[keep]
    px, py = R.pixel_centres(H, W, pos_n)

    def rest(p):
        if w.name == "sphere":
            attr = t["attr"].clone().requires_grad_(True)
            rast, _ = R.rasterize_from_ids(p, tri, ids, False)
            col, _ = R.interpolate(attr, rast, tri, None, [])
            _mse(R.antialias(col, rast, p, tri), t["target"][:images]).backward()
        elif w.name == "textured":
            tex = t["tex"].clone().requires_grad_(True)
            rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
            uv, uv_da = R.interpolate(t["uv"], rast, tri, rast_db, [0, 1])
            col = R.texture(tex, uv, uv_da, "linear-mipmap-linear", "wrap", None)
            _mse(R.antialias(col, rast, p, tri), t["target"][:images]).backward()
        elif w.name == "large":
            feat = t["feat"].clone().requires_grad_(True)
            tex = t["tex"].clone().requires_grad_(True)
            rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
            f, _ = R.interpolate(feat, rast, tri, None, [])
            st, st_da = R.interpolate(t["uv"], rast, tri, rast_db, [0, 1])
            col = R.texture(tex, st, st_da, "linear-mipmap-linear", "wrap", None)
            shaded = col + 0.1 * (f[..., 0:4] + f[..., 4:8])
            _mse(R.antialias(shaded, rast, p, tri), t["target"][:images]).backward()
        elif w.name == "cubemap":
            cube = t["cube"].clone().requires_grad_(True)
            rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
            n, n_da = R.interpolate(t["normals"], rast, tri, rast_db, [0, 1, 2])
            dirs, dirs_da = workloads.reflect(t["view"][:images], t["view_da"][:images], n, n_da)
            col = R.texture(cube, dirs, dirs_da, "linear-mipmap-linear", "cube", None)
            _mse(R.antialias(col, rast, p, tri), t["target"][:images]).backward()
        elif w.name == "instances":
            color = t["color"][:1].clone().requires_grad_(True)
            rast, _ = R.rasterize_from_ids(p, tri, ids, False)
            _mse(R.antialias(color, rast, p, tri), torch.zeros_like(color)).backward()

    runs = []
    while True:
        start_s = time.perf_counter()
        with torch.no_grad():
            R.visible_triangles(pos_n, sub, px, py)
        vis_s = time.perf_counter() - start_s
        start_s = time.perf_counter()
        rest(pos_n.clone().requires_grad_(True))
        rest_s = time.perf_counter() - start_s
        runs.append((vis_s + rest_s, vis_s, rest_s))
        if not full or len(runs) == 3 or sum(r[0] for r in runs) > 20.0:
            break
    total_s, vis_s, rest_s = sorted(runs)[len(runs) // 2]
    what = "item" if w.name == "instances" else "view"
    if full:
        total_ms = total_s * 1e3
        sample_text = (f"the whole step on all {B} {what}s at {H}x{W}: reference brute-force "
                       f"visibility over all {T} triangles ({vis_s:.1f} s) and the rest of the "
                       f"pipeline fwd+bwd ({rest_s:.1f} s); median of {len(runs)} run(s)")
    else:
        total_ms = B * (layers * vis_s * T / sample + rest_s) * 1e3
        sample_text = (f"one {what} of {B} at {H}x{W}: reference brute-force visibility over "
                       f"{sample} of its {T} triangles ({vis_s:.1f} s), x{layers} layer(s), and "
                       f"the rest of the pipeline fwd+bwd in full ({rest_s:.1f} s), extrapolated "
                       f"linearly to all triangles, layers and {what}s")
    return {
        "value": round(total_ms, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "affinity_cores": affinity,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": sample_text,
        "extrapolated": not full,
    }


def profiled_traffic(kernel: str, workload: str) -> dict | None:
    """HBM bytes per launch of ``kernel`` from the workload's committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by its reading for a copy of known size):
    lines ``<kernel>.fetch_bytes: N`` and ``<kernel>.write_bytes: N``."""
    path = ROOT / "profiles" / f"kernels.{workload}.pmc.txt"
    if not path.exists():
        return None
    f = _profile_fields(path)
    fetch, write = f.get(f"{kernel}.fetch_bytes"), f.get(f"{kernel}.write_bytes")
    if fetch is None or write is None:
        return None
    return {"bytes": fetch + write, "source": str(path.relative_to(ROOT))}


# Vector issue of the MI355X: 256 CUs x 4 SIMDs, each issuing one wave64 VALU instruction
# (64 lanes over a 16-lane SIMD) every 4 clocks without packed fp32, which the kernels do not
# use; at 2.4 GHz that is 614 G wave instructions/s (39.3 T lane operations/s; with fused
# multiply-adds counted twice and packed fp32, the published 157.3 TFLOP/s).
SIMDS = 256 * 4
CLOCK_HZ = 2.4e9
VALU_ISSUE_PEAK = SIMDS * CLOCK_HZ / 4  # wave64 VALU instructions per second


def _profile_fields(path: Path) -> dict:
    fields = {}
    for line in path.read_text().splitlines():
        key, sep, value = line.partition(":")
        if sep:
            try:
                fields[key.strip()] = float(value)
            except ValueError:
                pass
    return fields


def profiled_valu(kernel: str, workload: str, mean_ms: float) -> dict | None:
    """Vector issue of ``kernel`` from the workload's committed rocprofv3 counter summary
    (lines ``<kernel>.valu_instructions: N`` and ``<kernel>.valu_busy: F``): wave64 VALU
    instructions per launch (SQ_INSTS_VALU) over the live mean duration, against the issue
    peak, and the VALU-busy fraction that the summary derives from SQ_ACTIVE_INST_VALU (its
    header states how)."""
    path = ROOT / "profiles" / f"valu.{workload}.txt"
    if not path.exists():
        return None
    f = _profile_fields(path)
    if f"{kernel}.valu_instructions" not in f:
        return None
    instructions = f[f"{kernel}.valu_instructions"]
    rate = instructions / (mean_ms * 1e-3)
    out = {"instructions": int(instructions),
           "issue_rate": round(rate / 1e9, 1), "issue_peak": round(VALU_ISSUE_PEAK / 1e9, 1),
           "unit": "G wave64 instructions/s", "issue_frac": round(rate / VALU_ISSUE_PEAK, 4)}
    if f"{kernel}.valu_busy" in f:
        out["busy_frac"] = round(f[f"{kernel}.valu_busy"], 4)
    out["source"] = str(path.relative_to(ROOT))
    return out


def copy_probe(mib: int, device) -> None:
    """One device-to-device copy of ``mib`` MiB from memory no cache holds, the calibration of
    the HBM byte counters: the source is written, then a 2 GiB fill evicts it from the L2s and
    the Infinity Cache, then it is copied."""
    src = torch.ones(mib << 18, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    evict = torch.empty(1 << 29, dtype=torch.float32, device=device)
    evict.fill_(0.0)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del evict


WORKLOADS = {
    "sphere": "uv sphere 32x64 (3,968 triangles), 1 view at 256x256, colours [1,V,3], "
              "rasterize + interpolate + antialias, MSE, grads to pos/colours",
    "textured": "icosphere(5) (20,480 triangles), 4 views at 512x512, spherical uv with "
                "derivatives, 512x512x3 texture with mips from texture_construct_mip, trilinear "
                "wrap, antialias, MSE, grads to pos/texture",
    "large": "icosphere(8) radially perturbed, 1,310,720 triangles, 8 views x 1024x1024, "
             "features [1,V,8] + uv with derivatives, 1024x1024x4 texture with a full mip chain "
             "per call, trilinear wrap, antialias, MSE, grads to pos/feat/tex",
    "cubemap": "(2,3) torus knot 512x32 (32,768 triangles), 4 views at 1024x1024, reflected "
               "view rays from interpolated normals, derivatives by the chain rule through rays "
               "and normals, 6x512x512x3 cube map, trilinear, antialias, MSE, grads to "
               "pos/cube map",
    "instances": "256 icosphere(4) instances (1,310,720 triangles) in range mode at 512x512, "
                 "depth peeling to 4 layers, antialias of layer 0, MSE, grads to pos/colours",
}


def dominant_entry(per_kernel: dict) -> str:
    """The longest-running entry point that launches a single kernel (so that its event time is
    that kernel's time)."""
    return max((n for n in per_kernel if n in SINGLE_KERNEL), key=lambda n: per_kernel[n][0])


def cpu_model() -> str:
    """The host processor as /proc/cpuinfo names it, with its family, model, clock and the
    logical CPUs the kernel lists."""
    fields, logical = {}, 0
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, value = line.partition(":")
            key = key.strip()
            if key == "processor":
                logical += 1
            elif key in ("model name", "cpu family", "model", "cpu MHz") and key not in fields:
                fields[key] = value.strip()
    except OSError:
        return "unknown"
    return (f"{fields.get('model name', 'unknown')} (family {fields.get('cpu family', '?')}, "
            f"model {fields.get('model', '?')}, {fields.get('cpu MHz', '?')} MHz, "
            f"{logical} logical CPUs listed)")


def _loss_of(diff):
    """The MSE from the difference image, as _MSE computes it."""
    flat = diff.view(-1)
    return torch.linalg.vector_norm(flat).square().div_(flat.numel())


# hipGraphNodeType values (hip_runtime_api.h) named in the node counts.
_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
               6: "wait_event", 7: "event_record", 10: "mem_alloc", 11: "mem_free"}


def _graph_nodes(graph) -> dict | None:
    """Nodes of a captured graph by type, read through the HIP runtime (hipGraphGetNodes,
    hipGraphNodeGetType); None where the graph or the runtime does not give them."""
    import ctypes

    try:
        handle = graph.raw_cuda_graph()
        hip_rt = ctypes.CDLL("libamdhip64.so")
    except (RuntimeError, OSError) as error:
        print(f"graph nodes unavailable: {error}", file=sys.stderr)
        return None
    count = ctypes.c_size_t(0)
    if hip_rt.hipGraphGetNodes(ctypes.c_void_p(handle), None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * count.value)()
    if hip_rt.hipGraphGetNodes(ctypes.c_void_p(handle), nodes, ctypes.byref(count)) != 0:
        return None
    out = defaultdict(int)
    kind = ctypes.c_int(0)
    for node in nodes[:count.value]:
        if hip_rt.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(kind)) != 0:
            return None
        out[_NODE_TYPES.get(kind.value, f"type{kind.value}")] += 1
    out.setdefault("memset", 0)
    return dict(out)


def graph_step(step: Step, steps: int, repeats: int) -> dict | None:
    """A step captured once in a HIP graph (torch.cuda.graph) and replayed: the render and its
    backward pass, seeded with the MSE's gradient 2 (image - target) / n, are captured; the
    loss itself -- a multi-workgroup reduction, whose semaphores PyTorch clears with a memory
    fill that must not be replayed from a graph -- runs eagerly after each replay, so a step is
    one replay plus one reduction. Before timing, one replay's gradients and loss are compared
    with an eager step's. Returns the timing (``steps`` back to back, and the median, p10 and
    p90 of ``repeats`` individually synchronised ones), the check and the graph's node counts;
    None when the step cannot be captured (the reason goes to stderr)."""

    def captured():
        for x in step.leaves:
            x.grad = None
        image, target = step.render()
        diff = torch.sub(image, target)
        image.backward(torch.mul(diff, 2.0 / diff.numel()))
        return diff

    # The leaves' gradient accumulators were made on the default stream by the eager steps;
    # the warm-up on the side stream reuses them, which PyTorch reports (harmlessly) each time.
    quiet = getattr(torch.autograd.graph, "set_warn_on_accumulate_grad_stream_mismatch", None)
    if quiet is not None:
        quiet(False)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    try:
        with torch.cuda.stream(side):  # capture wants its allocations warmed on a side stream
            for _ in range(2):
                captured()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph):
            diff = captured()
        grads = [x.grad for x in step.leaves]
    except RuntimeError as error:
        print(f"graph capture failed, eager timing only: {error}", file=sys.stderr)
        torch.cuda.synchronize()
        return None
    graph.instantiate()
    nodes = _graph_nodes(graph)

    # One replay against one eager step of the same inputs.
    graph.replay()
    replay_loss = _loss_of(diff).item()
    replayed = [g.clone() for g in grads]
    eager_loss = step().item()
    torch.cuda.synchronize()
    worst = 0.0
    for ours, leaf in zip(replayed, step.leaves):
        scale = leaf.grad.abs().max().item()
        worst = max(worst, (ours - leaf.grad).abs().max().item() / max(scale, 1e-30))
    loss_diff = abs(replay_loss - eager_loss) / max(abs(eager_loss), 1e-30)
    check = {"gradients_max_rel_diff": worst, "loss_rel_diff": loss_diff,
             "passed": worst < 1e-5 and loss_diff < 1e-5}

    def one():
        graph.replay()
        return _loss_of(diff)

    one()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - start) * 1e3 / steps
    synced = synced_steps(one, repeats)
    del graph
    torch.cuda.synchronize()
    return {"ms_per_step": ms, "synced": synced, "check": check, "nodes": nodes}


def _percentile(values: list[float], q: float) -> float:
    """The q-quantile of values, linear between order statistics."""
    v = sorted(values)
    k = (len(v) - 1) * q
    lo = int(k)
    hi = min(lo + 1, len(v) - 1)
    return v[lo] + (v[hi] - v[lo]) * (k - lo)


def synced_steps(fn, repeats: int) -> dict:
    """Median, p10 and p90 of ``repeats`` individually synchronised calls of ``fn`` (ms), the
    rule of the reference's benchmarks (benchmarks/bench_rasterize.py:56-72)."""
    times = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        start = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - start) * 1e3)
    return {"n": repeats, "median_ms": round(_percentile(times, 0.5), 4),
            "p10_ms": round(_percentile(times, 0.1), 4),
            "p90_ms": round(_percentile(times, 0.9), 4)}


# Entry points whose results are cached per mesh (tri): they run in the first step only.
ONCE_PER_MESH = ("dr_raster_order", "dr_edge_neighbours")

# Single-kernel entry points of the backward scatters, by kernel (their live times rate the
# atomic counts of the committed counter summary).
SCATTER_ENTRY = {k: n for n, k in SINGLE_KERNEL.items() if n.endswith("_backward")}


def profiled_atomics(workload: str, live_ms: dict) -> dict | None:
    """Device atomic requests per launch of the kernels of a step that issue them (the backward
    scatters, the visibility's setup and bin passes), from the workload's committed counter
    summary (lines ``<kernel>.launches``, ``<kernel>.atomic_requests``,
    ``<kernel>.atomic_beyond_l2`` and ``<kernel>.mean_us``, the kernel-trace mean), rated per
    second over the live mean launch of the kernel's entry point where it launches that kernel
    alone, else over the summary's mean. Kernels launched once per mesh are left out."""
    path = ROOT / "profiles" / f"atomics.{workload}.pmc.txt"
    if not path.exists():
        return None
    f = _profile_fields(path)
    out = {}
    for key in f:
        if not key.endswith(".atomic_requests"):
            continue
        kernel = key[:-len(".atomic_requests")]
        if f.get(f"{kernel}.launches", 2) < 2:
            continue  # once per mesh (edge hash, processing order), not per step
        entry = SCATTER_ENTRY.get(kernel)
        ms = live_ms.get(entry) if entry else None
        source = "live"
        if ms is None:
            ms = f.get(f"{kernel}.mean_us", 0.0) * 1e-3
            source = "profile"
        if not ms:
            continue
        requests = f[key]
        out[kernel] = {"requests_per_launch": int(requests),
                       "beyond_l2_per_launch": int(f.get(f"{kernel}.atomic_beyond_l2", -1)),
                       "G_requests_per_s": round(requests / (ms * 1e-3) / 1e9, 2),
                       "mean_launch_ms": round(ms, 4), "duration_from": source}
    return {"kernels": out, "source": str(path.relative_to(ROOT))} if out else None


def run(name: str, steps: int, warmup: int, device, cpu: bool, sample_tris: int,
        graph: bool = False, repeats: int = 20, cpu_full_work: float = 2.2e10) -> dict:
    """The first two warm-up steps timed one by one (the first call of the process and of the
    mesh: library code loaded, processing order and edge adjacency computed, the visibility's
    list sizes learnt with one host wait), the other warm-up steps timed per entry point to
    find the dominant kernel, then exactly `steps` timed steps back to back in which only the
    dominant entry point carries HIP events (the roofline's live launch time; events around
    every call would add ~0.13 ms per step), then `repeats` individually synchronised steps
    (median, p10, p90), then 15 steps with every entry point timed for the per-kernel and
    per-op tables. With `graph`, `value` is instead the time per step of a captured step
    replayed `steps` times (the eager time stays in the line)."""
    w = workloads.build(name)
    step = make_step(w, device)
    model = BytesModel(w)
    timer = KernelTimer(model)
    timer.install()
    first_call = None
    for i in range(warmup):
        timer.active = i > 0 or warmup == 1
        if i < 2 and warmup >= 2:
            timer.active = i == 0
            torch.cuda.synchronize()
            start = time.perf_counter()
            step()
            torch.cuda.synchronize()
            wall = (time.perf_counter() - start) * 1e3
            if i == 0:
                once = timer.summary()
                timer.reset()
                first_call = {"first_step_ms": round(wall, 3), "once_per_mesh_ms": {
                    n: round(once[n][0], 4) for n in ONCE_PER_MESH if n in once}}
            else:
                first_call["second_step_ms"] = round(wall, 3)
            continue
        timer.step_index += 1
        step()
    timer.active = False
    torch.cuda.synchronize()
    dominant = dominant_entry(timer.summary()) if timer.events else None
    timer.reset()
    timer.only = None if dominant is None else {dominant}

    timer.active = True
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(device)
    start = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    after = torch.cuda.memory_stats(device)
    timer.active = False
    # Device memory the caching allocator took from or gave back to the runtime during the
    # timed steps (0 in a steady state: every buffer reused).
    allocator = {k: int(after.get(k, 0) - before.get(k, 0))
                 for k in ("segment.all.allocated", "segment.all.freed", "num_alloc_retries")}
    ms_per_step = elapsed * 1e3 / steps
    live = timer.summary()
    if dominant is None:  # no warm-up: every entry point was timed in the timed steps
        dominant = dominant_entry(live)
    dom_total, dom_count = live[dominant]
    dom_ms = dom_total / dom_count
    dom_bytes = timer.bytes[dominant] / dom_count

    synced = synced_steps(step, repeats)

    # The per-kernel and per-op tables, from their own steps after the timed ones.
    table_steps = 15
    timer.reset()
    timer.only = None
    timer.active = True
    for i in range(table_steps):
        timer.step_index = i
        step()
    torch.cuda.synchronize()
    timer.active = False
    timer.uninstall()
    per_kernel = timer.summary()
    kernels = {}
    op_ms, op_bytes = defaultdict(float), defaultdict(float)
    op_entries = defaultdict(list)
    for kname, (total_ms, count) in per_kernel.items():
        mean_ms = total_ms / count
        entry = {"ms_per_step": round(total_ms / table_steps, 4), "launches_per_step":
                 round(count / table_steps, 2), "mean_launch_ms": round(mean_ms, 4)}
        if timer.bytes[kname]:
            gbs = timer.bytes[kname] / count / (mean_ms * 1e-3) / 1e9
            entry["GB/s"] = round(gbs, 1)
            entry["frac"] = round(gbs * 1e9 / HBM_PEAK, 4)
        kernels[kname] = entry
        op = OP_OF.get(kname)
        if op is not None:
            op_ms[op] += total_ms / table_steps
            op_bytes[op] += timer.op_bytes[kname] / table_steps
            op_entries[op].append(kname)
    # The tile pass carries the whole visibility's unique bytes: its rate is quoted over the
    # four visibility entry points together (in range mode the setup pass does most of the work
    # and the tile pass alone would read above the HBM peak).
    tiles = kernels.get("dr_raster_visibility_tiles")
    if tiles is not None and "GB/s" in tiles:
        del tiles["GB/s"], tiles["frac"]
        vis_ms = sum(kernels[k]["ms_per_step"] for k in kernels if k in VISIBILITY_ENTRIES)
        gbs = timer.bytes["dr_raster_visibility_tiles"] / table_steps / (vis_ms * 1e-3) / 1e9
        tiles["visibility_ms_per_step"] = round(vis_ms, 4)
        tiles["visibility_GB/s"] = round(gbs, 1)
        tiles["visibility_frac"] = round(gbs * 1e9 / HBM_PEAK, 4)
    ops = {}
    for op in ("rasterize", "interpolate", "texture", "antialias"):
        if op not in op_ms:
            continue
        floor_ms = op_bytes[op] / HBM_PEAK * 1e3
        per_step = list(timer.per_step(op_entries[op]).values())
        ops[op] = {"ms": round(op_ms[op], 4), "p10_ms": round(_percentile(per_step, 0.1), 4),
                   "p90_ms": round(_percentile(per_step, 0.9), 4), "bytes": int(op_bytes[op]),
                   "roofline_ms": round(floor_ms, 4), "frac": round(floor_ms / op_ms[op], 4)}
    step_bytes = sum(op_bytes.values())
    step_floor_ms = step_bytes / HBM_PEAK * 1e3
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = profiled_traffic(SINGLE_KERNEL[dominant], name)
    atomics = profiled_atomics(name, {k: v["mean_launch_ms"] for k, v in kernels.items()})

    eager_ms = ms_per_step
    replay = graph_step(step, steps, repeats) if graph else None
    if replay is not None:
        ms_per_step = replay["ms_per_step"]

    baseline = None
    if cpu:
        baseline = cpu_baseline(w, sample_tris, device, cpu_full_work)

    tris = w.tensors["tri"].shape[0]
    result = {
        "metric": METRIC if name == "large" else "ms per fwd+bwd render (4-op pipeline)",
        "value": round(ms_per_step, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 3),
        "timing": "HIP graph replay" if replay is not None else "eager",
        "eager_ms_per_step": round(eager_ms, 3),
        # The reference's rule: median (and p10, p90) of individually synchronised steps.
        "synced_steps": synced,
        "first_call": first_call,
        "allocator_during_timed_steps": allocator,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[name],
            "name": name,
            "images": w.batch,
            "resolution": list(w.resolution),
            "triangles": tris,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": SINGLE_KERNEL[dominant],
            "entry_point": dominant,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(achieved * 1e9 / HBM_PEAK, 4),
            "traffic": None if traffic is None else int(traffic["bytes"]),
            "traffic_source": None if traffic is None else traffic["source"],
            "algorithmic_bytes": int(dom_bytes),
            "mean_launch_ms": round(dom_ms, 4),
            # The rasterizer's own bound: vector issue (no HBM stream limits it).
            "valu": profiled_valu(SINGLE_KERNEL[dominant], name, dom_ms),
            # Each op's forward+backward against the HBM time of its unique bytes, and the
            # whole step (the ops' bytes; the glue between them is timed but not credited).
            "ops": ops,
            "step": {"bytes": int(step_bytes), "roofline_ms": round(step_floor_ms, 4),
                     "frac": round(step_floor_ms / ms_per_step, 4),
                     "ops_ms": round(sum(op_ms.values()), 4)},
            # The backward scatters' device atomics (counter summary, live launch times).
            "atomics": atomics,
        },
        "cpu_baseline": baseline,
        "kernels": kernels,
    }
    if replay is not None:
        result["graph"] = {"synced_steps": replay["synced"], "check": replay["check"],
                           "nodes": replay["nodes"]}
    return result


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", default="large", choices=sorted(WORKLOADS))
    parser.add_argument("--all-workloads", action="store_true",
                        help="one JSON line per workload (the headline first)")
    parser.add_argument("--cpu-sample-tris", type=int, default=4096)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-full-work", type=float, default=2.2e10,
                        help="CPU baseline measured in full up to this many coverage "
                             "evaluations (images x triangles x pixels), sampled beyond")
    parser.add_argument("--graph", action="store_true",
                        help="time a captured step replayed as a HIP graph (eager time kept)")
    parser.add_argument("--repeats", type=int, default=20,
                        help="individually synchronised steps for the median, p10 and p90")
    parser.add_argument("--copy-probe-mib", type=int, default=0,
                        help="run one copy of this size first (counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported (the views would "
              "shard across GPUs with one all-reduce of the shared gradients, which this "
              "build does not launch).", file=sys.stderr)
        sys.exit(2)

    device = torch.device("cuda", 0)
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib, device)
    names = ["large"] + [n for n in WORKLOADS if n != "large"] if args.all_workloads \
        else [args.workload]
    for name in names:
        result = run(name, args.steps, args.warmup, device, not args.no_cpu_baseline,
                     args.cpu_sample_tris, args.graph, args.repeats, args.cpu_full_work)
        print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
