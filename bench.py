"""Benchmark: ms per forward+backward render of the four-op pipeline on one MI355X.

Default workload (the headline configuration, ``--workload large``): icosphere(8), 1,310,720
triangles, radially perturbed, 8 views at 1024x1024. One step is

    rasterize -> interpolate(features [1, V, 8]) and interpolate(uv, rast_db, 'all')
    -> texture(1024x1024x4, full mip chain built in the call, trilinear, wrap)
    -> shade = colour + 0.1 * (f[..., 0:4] + f[..., 4:8]) -> antialias -> MSE -> backward

with gradients to positions, features and texture (the feature sum is written as a sum over a
[..., 2, 4] view of f: one reduction instead of two strided slices). ``--workload`` selects one
of the other four configurations (``make_step`` shows each step) and ``--all-workloads`` runs
all five, one JSON line each. Inputs are synthetic and resident on the GPU before timing
starts. ``--steps`` steps are timed between synchronisations, after ``--warmup`` untimed ones.

Per-kernel time: HIP events around the C-ABI entry points, on the stream they launch on (in the
timed steps only around the dominant one; every entry point in five further steps for the
per-kernel table). Algorithmic bytes are the unique-byte model of ``BytesModel``: every input
read once and every output written once, from each call's own arguments. ``roofline`` reports
the longest-running entry point that launches a single kernel (so that its event time is that
kernel's duration): its unique bytes per launch over its mean duration, against 8 TB/s; its
vector issue against the issue peak (``valu``, from the committed counter summary); each op's
forward+backward time against the HBM time of its unique bytes (``ops``); and the whole step
against the four ops' bytes (``step``). ``traffic`` is the HBM bytes per launch measured for
that kernel with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE, each scaled by the counter's
reading for a copy of known size), from ``profiles/kernels.<workload>.pmc.txt`` when present.
``--graph`` times a step captured in a HIP graph and replayed (the eager time stays in the
line as ``eager_ms_per_step``).

CPU baseline: the oracle (a pure-PyTorch restatement of the reference backend) on the host
cores, on a bounded sample of the same workload -- one image, its visibility over a subset of
the triangles and the rest of the pipeline in full -- extrapolated linearly to all triangles,
layers and images.
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


# Entry points that launch exactly one kernel, and that kernel.
SINGLE_KERNEL = {
    "dr_raster_visibility_tiles": "raster_tile_kernel",
    "dr_resolve_forward": "resolve_fwd_kernel",
    "dr_resolve_backward": "resolve_bwd_kernel",
    "dr_interpolate_forward": "interp_fwd_kernel",
    "dr_interpolate_backward": "interp_bwd_kernel",
    "dr_texture_forward": "tex_fwd_kernel",
    "dr_texture_backward": "tex_bwd_kernel",
    "dr_antialias_backward": "aa_bwd_kernel",
}


class KernelTimer:
    """HIP events around the backend's C-ABI calls, on the current stream, with the algorithmic
    bytes of each call: its kernel's own (``kernel_bytes``) and its share of its op's
    (``op_bytes``)."""

    def __init__(self, model):
        self.model = model
        self.active = False
        self.only = None  # entry point names to time (None: every one)
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
            self.events[name].append((start, end))
            self.bytes[name] += self.model.kernel_bytes(name, args)
            self.op_bytes[name] += self.model.op_bytes(name, args)

        hip.call = timed

    def uninstall(self):
        hip.call = self._call

    def summary(self):
        torch.cuda.synchronize()
        out = {}
        for name, pairs in self.events.items():
            times = [s.elapsed_time(e) for s, e in pairs]
            out[name] = (sum(times), len(times))
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


def make_step(w, device):
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

        def body():
            rast, _ = dr.rasterize(ctx, pos, tri, res, grad_db=False)
            col, _ = dr.interpolate(attr, rast, tri)
            return _mse(dr.antialias(col, rast, pos, tri), target)
    elif w.name == "textured":
        pos, tex = leaf("pos"), leaf("tex")
        tri, uv_attr, target = t["tri"], t["uv"], t["target"]

        def body():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            uv, uv_da = dr.interpolate(uv_attr, rast, tri, rast_db, diff_attrs="all")
            mip = dr.texture_construct_mip(tex)
            col = dr.texture(tex, uv, uv_da, mip=mip, filter_mode="linear-mipmap-linear",
                             boundary_mode="wrap")
            return _mse(dr.antialias(col, rast, pos, tri), target)
    elif w.name == "large":
        pos, feat, tex = leaf("pos"), leaf("feat"), leaf("tex")
        tri, uv_attr, target = t["tri"], t["uv"], t["target"]

        def body():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            f, _ = dr.interpolate(feat, rast, tri)
            st, st_da = dr.interpolate(uv_attr, rast, tri, rast_db, diff_attrs="all")
            col = dr.texture(tex, st, st_da, filter_mode="linear-mipmap-linear",
                             boundary_mode="wrap")
            shaded = _Shade.apply(col, f)  # col + 0.1 * (f[..., :4] + f[..., 4:])
            return _mse(dr.antialias(shaded, rast, pos, tri), target)
    elif w.name == "cubemap":
        pos, cube = leaf("pos"), leaf("cube")
        tri, normals, target = t["tri"], t["normals"], t["target"]
        view, view_da = t["view"], t["view_da"]

        def body():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            n, n_da = dr.interpolate(normals, rast, tri, rast_db, diff_attrs="all")
            dirs, dirs_da = workloads.reflect(view, view_da, n, n_da)
            col = dr.texture(cube, dirs, dirs_da, filter_mode="linear-mipmap-linear",
                             boundary_mode="cube")
            return _mse(dr.antialias(col, rast, pos, tri), target)
    elif w.name == "instances":
        pos, color = leaf("pos"), leaf("color")
        tri, ranges = t["tri"], t["ranges"]
        target = torch.zeros_like(color)

        def body():
            with dr.DepthPeeler(ctx, pos, tri, res, ranges=ranges) as peeler:
                layers = [peeler.rasterize_next_layer()[0] for _ in range(4)]
            return _mse(dr.antialias(color, layers[0], pos, tri), target)
    else:
        raise ValueError(w.name)

    def step():
        for x in leaves:
            x.grad = None
        loss = body()
        loss.backward()
        return loss

    return step


def first_image_ids(w, device):
    """Triangle ids [1, H, W] (-1: none) of the first image (range mode: item 0's first layer),
    from the GPU, for the CPU baseline's rest-of-pipeline leg."""
    t = w.tensors
    ctx = dr.RasterizeContext(device)
    with torch.no_grad():
        if w.name == "instances":
            rast, _ = dr.rasterize(ctx, t["pos"].to(device), t["tri"].to(device),
                                   w.resolution, ranges=t["ranges"][:1])
        else:
            rast, _ = dr.rasterize(ctx, t["pos"][:1].to(device), t["tri"].to(device),
                                   w.resolution)
    return (rast[..., 3].long() - 1).cpu()


def cpu_baseline(w, sample_tris: int, ids) -> dict:
    """The oracle on the host: one image's brute-force visibility over a sample of its
    triangles, and the rest of the pipeline forward and backward on that image in full (with
    the true visibility), extrapolated linearly to all triangles, layers and images."""
    from oracle import reference as R

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    t = w.tensors
    (H, W), B = w.resolution, w.batch
    tri = t["tri"]
    layers = 1
    if w.name == "instances":
        start, count = (int(v) for v in t["ranges"][0])
        own = tri[start:start + count]
        pos1 = t["pos"][None]
        layers = 4
    else:
        own = tri
        pos1 = t["pos"][:1].clone()
    T = own.shape[0]
    sample = min(sample_tris, T)
    sub = own[torch.randperm(T, generator=torch.Generator().manual_seed(0))[:sample]]
    px, py = R.pixel_centres(H, W, pos1)
    start_s = time.perf_counter()
    with torch.no_grad():
        R.visible_triangles(pos1, sub, px, py)
    vis_s = time.perf_counter() - start_s

    p = pos1.clone().requires_grad_(True)
    start_s = time.perf_counter()
    if w.name == "sphere":
        attr = t["attr"].clone().requires_grad_(True)
        rast, _ = R.rasterize_from_ids(p, tri, ids, False)
        col, _ = R.interpolate(attr, rast, tri, None, [])
        _mse(R.antialias(col, rast, p, tri), t["target"][:1]).backward()
    elif w.name == "textured":
        tex = t["tex"].clone().requires_grad_(True)
        rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
        uv, uv_da = R.interpolate(t["uv"], rast, tri, rast_db, [0, 1])
        col = R.texture(tex, uv, uv_da, "linear-mipmap-linear", "wrap", None)
        _mse(R.antialias(col, rast, p, tri), t["target"][:1]).backward()
    elif w.name == "large":
        feat = t["feat"].clone().requires_grad_(True)
        tex = t["tex"].clone().requires_grad_(True)
        rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
        f, _ = R.interpolate(feat, rast, tri, None, [])
        st, st_da = R.interpolate(t["uv"], rast, tri, rast_db, [0, 1])
        col = R.texture(tex, st, st_da, "linear-mipmap-linear", "wrap", None)
        shaded = col + 0.1 * (f[..., 0:4] + f[..., 4:8])
        _mse(R.antialias(shaded, rast, p, tri), t["target"][:1]).backward()
    elif w.name == "cubemap":
        cube = t["cube"].clone().requires_grad_(True)
        rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
        n, n_da = R.interpolate(t["normals"], rast, tri, rast_db, [0, 1, 2])
        dirs, dirs_da = workloads.reflect(t["view"][:1], t["view_da"][:1], n, n_da)
        col = R.texture(cube, dirs, dirs_da, "linear-mipmap-linear", "cube", None)
        _mse(R.antialias(col, rast, p, tri), t["target"][:1]).backward()
    elif w.name == "instances":
        color = t["color"][:1].clone().requires_grad_(True)
        rast, _ = R.rasterize_from_ids(p, tri, ids, False)
        _mse(R.antialias(color, rast, p, tri), torch.zeros_like(color)).backward()
    rest_s = time.perf_counter() - start_s
    total_ms = B * (layers * vis_s * T / sample + rest_s) * 1e3
    what = "item" if w.name == "instances" else "view"
    return {
        "value": round(total_ms, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"one {what} of {B} at {H}x{W}: reference brute-force visibility over "
                   f"{sample} of its {T} triangles ({vis_s:.1f} s), x{layers} layer(s), and the "
                   f"rest of the pipeline fwd+bwd in full ({rest_s:.1f} s), extrapolated "
                   f"linearly to all triangles, layers and {what}s"),
        "extrapolated": sample < T or B > 1,
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
# (64 lanes over a 16-lane SIMD) every 4 clocks without packed fp32, which this build does not
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
    """Vector issue of ``kernel`` from its committed rocprofv3 counter summary: wave64 VALU
    instructions per launch (SQ_INSTS_VALU) over the live mean duration, against the issue
    peak, and the VALU-busy fraction that the summary derives from SQ_ACTIVE_INST_VALU (its
    header states how)."""
    path = ROOT / "profiles" / f"{kernel}.{workload}.valu.txt"
    if not path.exists():
        return None
    f = _profile_fields(path)
    if "valu_instructions" not in f:
        return None
    rate = f["valu_instructions"] / (mean_ms * 1e-3)
    out = {"instructions": int(f["valu_instructions"]),
           "issue_rate": round(rate / 1e9, 1), "issue_peak": round(VALU_ISSUE_PEAK / 1e9, 1),
           "unit": "G wave64 instructions/s", "issue_frac": round(rate / VALU_ISSUE_PEAK, 4)}
    if "valu_busy" in f:
        out["busy_frac"] = round(f["valu_busy"], 4)
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
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def graph_step_ms(step, steps: int) -> float | None:
    """ms per step when one step, captured in a HIP graph (torch.cuda.graph), is replayed
    `steps` times back to back: the same kernels with no host work between them. None when the
    step cannot be captured (the reason goes to stderr)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    try:
        with torch.cuda.stream(side):  # capture wants its allocations warmed on a side stream
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
    except RuntimeError as error:
        print(f"graph capture failed, eager timing only: {error}", file=sys.stderr)
        torch.cuda.synchronize()
        return None
    graph.replay()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - start) * 1e3 / steps
    del graph
    torch.cuda.synchronize()
    return ms


def run(name: str, steps: int, warmup: int, device, cpu: bool, sample_tris: int,
        graph: bool = False) -> dict:
    """Warm-up steps (timed per entry point after the first, to find the dominant kernel), then
    exactly `steps` timed steps in which only the dominant entry point carries HIP events (the
    roofline's live launch time; events around every call would add ~0.13 ms per step), then a
    few more steps with every entry point timed, for the per-kernel and per-op tables. With
    `graph`, `value` is instead the time per step of a captured step replayed `steps` times
    (the eager time stays in the line, and the kernel times come from the eager steps)."""
    w = workloads.build(name)
    step = make_step(w, device)
    model = BytesModel(w)
    timer = KernelTimer(model)
    timer.install()
    for i in range(warmup):
        timer.active = i > 0 or warmup == 1
        step()
    timer.active = False
    torch.cuda.synchronize()
    dominant = dominant_entry(timer.summary()) if timer.events else None
    timer.reset()
    timer.only = None if dominant is None else {dominant}

    timer.active = True
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    timer.active = False
    ms_per_step = elapsed * 1e3 / steps
    live = timer.summary()
    if dominant is None:  # no warm-up: every entry point was timed in the timed steps
        dominant = dominant_entry(live)
    dom_total, dom_count = live[dominant]
    dom_ms = dom_total / dom_count
    dom_bytes = timer.bytes[dominant] / dom_count

    # The per-kernel and per-op tables, from their own steps after the timed ones.
    table_steps = min(steps, 5)
    timer.reset()
    timer.only = None
    timer.active = True
    for _ in range(table_steps):
        step()
    torch.cuda.synchronize()
    timer.active = False
    timer.uninstall()
    per_kernel = timer.summary()
    kernels = {}
    op_ms, op_bytes = defaultdict(float), defaultdict(float)
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
        ops[op] = {"ms": round(op_ms[op], 4), "bytes": int(op_bytes[op]),
                   "roofline_ms": round(floor_ms, 4), "frac": round(floor_ms / op_ms[op], 4)}
    step_bytes = sum(op_bytes.values())
    step_floor_ms = step_bytes / HBM_PEAK * 1e3
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = profiled_traffic(SINGLE_KERNEL[dominant], name)

    eager_ms = ms_per_step
    replay_ms = graph_step_ms(step, steps) if graph else None
    if replay_ms is not None:
        ms_per_step = replay_ms

    baseline = None
    if cpu:
        baseline = cpu_baseline(w, sample_tris, first_image_ids(w, device))

    tris = w.tensors["tri"].shape[0]
    return {
        "metric": METRIC if name == "large" else "ms per fwd+bwd render (4-op pipeline)",
        "value": round(ms_per_step, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 3),
        "timing": "HIP graph replay" if replay_ms is not None else "eager",
        "eager_ms_per_step": round(eager_ms, 3),
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
        },
        "cpu_baseline": baseline,
        "kernels": kernels,
    }


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
    parser.add_argument("--graph", action="store_true",
                        help="time a captured step replayed as a HIP graph (eager time kept)")
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
                     args.cpu_sample_tris, args.graph)
        print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
