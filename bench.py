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

Per-kernel time: every C-ABI entry point called in the timed steps is bracketed by HIP events
on the stream it launches on. ``roofline`` reports the longest-running entry point that
launches a single kernel (so that its event time is that kernel's duration): its algorithmic
bytes per launch -- the unique bytes its algorithm must move, from the call's arguments
(``BytesModel``) -- over its mean duration, against 8 TB/s. ``traffic`` is the HBM bytes per
launch measured for that kernel with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE, each scaled
by the counter's reading for a copy of known size), read from the summary under profiles/ when
one exists for it and the workload.

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
    """HIP events around the backend's C-ABI calls, on the current stream, and the algorithmic
    bytes of each call."""

    def __init__(self, bytes_of):
        self.events = defaultdict(list)
        self.bytes = defaultdict(float)
        self.pending = defaultdict(list)
        self.bytes_of = bytes_of
        self.active = False
        self.only = None  # entry point names to time (None: every one)
        self._call = hip.call

    def reset(self):
        self.events = defaultdict(list)
        self.bytes = defaultdict(float)
        self.pending = defaultdict(list)

    def resolve(self):
        """Bytes of the timed calls; a model may return a function of counts that are known
        only after the call (the tile pass queued before its list sizes arrive)."""
        for name, amounts in self.pending.items():
            self.bytes[name] += sum(a() if callable(a) else a for a in amounts)
        self.pending = defaultdict(list)

    def install(self):
        def timed(name, *args):
            if not self.active or (self.only is not None and name not in self.only):
                return self._call(name, *args)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            self._call(name, *args)
            end.record()
            self.events[name].append((start, end))
            amount = self.bytes_of(name, args)
            if amount is not None:
                self.pending[name].append(amount)

        hip.call = timed

    def uninstall(self):
        hip.call = self._call

    def summary(self):
        torch.cuda.synchronize()
        self.resolve()
        out = {}
        for name, pairs in self.events.items():
            times = [s.elapsed_time(e) for s, e in pairs]
            out[name] = (sum(times), len(times))
        return out


# Tile rasterization, per tile list entry: the entry (4 B) and the 64-byte record it names
# (three clip-space vertices, triangle row, tile rectangle); per tile with entries: its 256
# keys read and written once (16 B each).
TILE_ENTRY_BYTES = 4 + 64
TILE_KEY_BYTES = 256 * 16


def _struct(arg):
    """The ctypes structure a byref() argument points to."""
    return arg._obj


class BytesModel:
    """Algorithmic bytes of each C-ABI call: the unique bytes its algorithm must move (inputs
    read once, outputs written once, fp32 = 4 B), from the call's own arguments and the
    workload's mesh sizes. Gathered arrays (pos, tri, attributes, texels) count whole."""

    def __init__(self, w):
        pos = w.tensors["pos"]
        self.vertices = pos.shape[-2]
        self.pos_images = pos.shape[0] if pos.ndim == 3 else 1
        self.tri = w.tensors["tri"].shape[0]

    def pos_bytes(self, images):
        return images * self.vertices * 16

    def __call__(self, name, args):
        model = getattr(self, name[3:], None)
        return None if model is None else model(args)

    @staticmethod
    def _pixels(g):
        return g.batch * g.height * g.width

    def raster_visibility_start(self, args):
        g = _struct(args[0])
        return self.pos_bytes(self.pos_images) + self.tri * 12 + self._pixels(g) * 8

    def raster_visibility_tiles(self, args):
        # The counts array holds the list sizes once the caller has them (after the call when
        # the pass was queued before they arrived).
        counts = args[6]
        return lambda: counts[1] * TILE_ENTRY_BYTES + counts[3] * TILE_KEY_BYTES

    def resolve_forward(self, args):
        P = self._pixels(_struct(args[0]))
        return (P * 8 + self.pos_bytes(self.pos_images) + self.tri * 12
                + P * 16 * (2 if args[3] else 1))

    def resolve_backward(self, args):
        P = self._pixels(_struct(args[0]))
        return (P * 8 + P * 16 * (2 if args[3] else 1) + 2 * self.pos_bytes(self.pos_images)
                + self.tri * 12)

    def interpolate_forward(self, args):
        a = _struct(args[0])
        P, ch, nd = a.batch * a.height * a.width, a.channels, a.num_diff
        images = a.batch if a.attr_batch_stride else 1
        return (P * 16 * (2 if nd else 1) + self.tri * 12 + images * a.num_vertices * ch * 4
                + P * ch * 4 + P * 2 * nd * 4)

    def interpolate_backward(self, args):
        a = _struct(args[0])
        P, ch, nd = a.batch * a.height * a.width, a.channels, a.num_diff
        images = a.batch if a.attr_batch_stride else 1
        return (P * ch * 4 + P * 2 * nd * 4 + P * 16 * (2 if nd else 1) + self.tri * 12
                + 2 * images * a.num_vertices * ch * 4 + P * 16 * (2 if nd else 1))

    @staticmethod
    def _texture_io(a):
        P, C = a.batch * a.height * a.width, a.channels
        cube = a.boundary == hip.BOUNDARIES["cube"]
        coords = P * (12 if cube else 8) + (P * (24 if cube else 16) if a.uv_da else 0)
        return P, C, coords + (P * 4 if a.bias else 0), a.tex_batch * a.num_texels * C * 4

    def texture_forward(self, args):
        P, C, coords, texels = self._texture_io(_struct(args[0]))
        return texels + coords + P * C * 4

    def texture_backward(self, args):
        P, C, coords, texels = self._texture_io(_struct(args[0]))
        return P * C * 4 + 2 * coords + 2 * texels

    @staticmethod
    def _mip(args):
        tex_batch, channels, total, faces = args[1], args[2], args[3], args[4]
        base = faces * args[6][0] * args[7][0]
        return tex_batch * channels * 4 * (2 * total - base)

    def mip_build(self, args):
        return self._mip(args)

    def mip_build_backward(self, args):
        return self._mip(args)

    def silhouette_mask(self, args):
        pos_batch, num_tri, batch, height, width = args[2], args[4], args[7], args[8], args[9]
        P = batch * height * width if args[6] else 0
        return P * 16 + 2 * pos_batch * num_tri + self.pos_bytes(pos_batch) + num_tri * 24

    def antialias_forward(self, args):
        a = _struct(args[0])
        P, C = a.batch * a.height * a.width, a.channels
        images = a.batch if a.pos_batch_stride else 1
        return (2 * P * C * 4 + P * 16 + self.pos_bytes(images) + a.num_tri * 12
                + images * a.num_tri + P * 10)

    def antialias_backward(self, args):
        a = _struct(args[0])
        P, C = a.batch * a.height * a.width, a.channels
        images = a.batch if a.pos_batch_stride else 1
        return (3 * P * C * 4 + P * 16 + P * 10 + 2 * self.pos_bytes(images)
                + a.num_tri * 12 + images * a.num_tri)


# ---- the five workloads' steps ----------------------------------------------------------------

def reflect(view, n, n_da):
    """Reflection of the view rays about the interpolated normals, and its screen-space
    derivatives from those of the normals (the rays' own derivatives are left out)."""
    d = (view * n).sum(-1, keepdim=True)
    dirs = view - 2 * d * n
    parts = []
    for axis in (0, 1):
        dn = n_da[..., axis::2]
        dd = (view * dn).sum(-1, keepdim=True)
        parts.append(-2 * (dd * n + d * dn))
    return dirs, torch.stack(parts, -1).reshape(*dirs.shape[:-1], 6)


def _mse(x, target):
    return torch.nn.functional.mse_loss(x, target)


class _Shade(torch.autograd.Function):
    """col + 0.1 * (f[..., :4] + f[..., 4:]) for 8-channel features. The same values and
    gradients as autograd through the expression (bit for bit); its backward repeats the
    gradient into both halves in one copy, where autograd's view/sum backward makes a strided
    copy of the expanded gradient (~0.11 ms at 8 x 1024^2)."""

    @staticmethod
    def forward(ctx, col, f):
        return col + 0.1 * (f[..., :4] + f[..., 4:])

    @staticmethod
    def backward(ctx, g):
        return g, (0.1 * g).repeat(*([1] * (g.dim() - 1)), 2)


def make_step(w, device):
    """One forward+backward step of workload ``w`` on the GPU (inputs copied to ``device``)."""
    t = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in w.tensors.items()}
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
            return _mse(col, target)
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
        tri, normals, view, target = t["tri"], t["normals"], t["view"], t["target"]

        def body():
            rast, rast_db = dr.rasterize(ctx, pos, tri, res)
            n, n_da = dr.interpolate(normals, rast, tri, rast_db, diff_attrs="all")
            dirs, dirs_da = reflect(view, n, n_da)
            col = dr.texture(cube, dirs, dirs_da, filter_mode="linear-mipmap-linear",
                             boundary_mode="cube")
            return _mse(col, target)
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
        _mse(col, t["target"][:1]).backward()
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
        dirs, dirs_da = reflect(t["view"][:1], n, n_da)
        col = R.texture(cube, dirs, dirs_da, "linear-mipmap-linear", "cube", None)
        _mse(col, t["target"][:1]).backward()
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
        "kind": "port",
        "sample": (f"one {what} of {B} at {H}x{W}: reference brute-force visibility over "
                   f"{sample} of its {T} triangles ({vis_s:.1f} s), x{layers} layer(s), and the "
                   f"rest of the pipeline fwd+bwd in full ({rest_s:.1f} s), extrapolated "
                   f"linearly to all triangles, layers and {what}s"),
        "extrapolated": sample < T or B > 1,
    }


def profiled_traffic(kernel: str, workload: str) -> dict | None:
    """HBM bytes per launch of ``kernel`` from its committed rocprofv3 counter summary."""
    path = ROOT / "profiles" / f"{kernel}.{workload}.pmc.txt"
    if not path.exists():
        return None
    fields = {}
    for line in path.read_text().splitlines():
        key, sep, value = line.partition(":")
        if sep and key.strip() in ("fetch_bytes", "write_bytes", "copy_factor_fetch",
                                   "copy_factor_write"):
            fields[key.strip()] = float(value)
    if len(fields) != 4:
        return None
    return {"bytes": fields["fetch_bytes"] + fields["write_bytes"], "source": str(
        path.relative_to(ROOT))}


# fp32 vector issue peak of the MI355X in lane operations per second: 256 CUs x 4 SIMDs x 32
# lanes x 2.4 GHz (the published 157.3 TFLOP/s counts a fused multiply-add as two operations).
VALU_PEAK = 256 * 4 * 32 * 2.4e9


def profiled_valu(kernel: str, workload: str, mean_ms: float) -> dict | None:
    """VALU utilisation of ``kernel``: its vector instructions per launch (SQ_INSTS_VALU, wave64
    instructions, from its committed rocprofv3 counter summary) times 64 lanes, over its mean
    duration, against VALU_PEAK."""
    path = ROOT / "profiles" / f"{kernel}.{workload}.valu.txt"
    if not path.exists():
        return None
    n = None
    for line in path.read_text().splitlines():
        key, sep, value = line.partition(":")
        if sep and key.strip() == "valu_instructions":
            n = float(value)
    if n is None:
        return None
    ops = n * 64 / (mean_ms * 1e-3)
    return {"instructions": int(n), "achieved": round(ops / 1e12, 2), "peak": VALU_PEAK / 1e12,
            "unit": "T lane-ops/s", "frac": round(ops / VALU_PEAK, 4),
            "source": str(path.relative_to(ROOT))}


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
                "wrap, MSE, grads to pos/texture",
    "large": "icosphere(8) radially perturbed, 1,310,720 triangles, 8 views x 1024x1024, "
             "features [1,V,8] + uv with derivatives, 1024x1024x4 texture with a full mip chain "
             "per call, trilinear wrap, antialias, MSE, grads to pos/feat/tex",
    "cubemap": "(2,3) torus knot 512x32 (32,768 triangles), 4 views at 1024x1024, reflected "
               "view rays from interpolated normals with derivatives, 6x512x512x3 cube map, "
               "trilinear, MSE, grads to pos/cube map",
    "instances": "256 icosphere(4) instances (1,310,720 triangles) in range mode at 512x512, "
                 "depth peeling to 4 layers, antialias of layer 0, MSE, grads to pos/colours",
}


def dominant_entry(per_kernel: dict, timed_bytes: dict) -> str:
    """The longest-running entry point that launches a single kernel (so that its event time is
    that kernel's time) and has a byte model."""
    return max((n for n in per_kernel if n in SINGLE_KERNEL and n in timed_bytes),
               key=lambda n: per_kernel[n][0])


def run(name: str, steps: int, warmup: int, device, cpu: bool, sample_tris: int) -> dict:
    """Warm-up steps (timed per entry point after the first, to find the dominant kernel), then
    exactly `steps` timed steps in which only the dominant entry point carries HIP events (the
    roofline's live launch time; events around every call would add ~0.13 ms per step), then a
    few more steps with every entry point timed, for the per-kernel table."""
    w = workloads.build(name)
    step = make_step(w, device)
    timer = KernelTimer(BytesModel(w))
    timer.install()
    for i in range(warmup):
        timer.active = i > 0 or warmup == 1
        step()
    timer.active = False
    torch.cuda.synchronize()
    dominant = None
    if timer.events:
        dominant = dominant_entry(timer.summary(), timer.bytes)
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
        dominant = dominant_entry(live, timer.bytes)
    dom_total, dom_count = live[dominant]
    dom_ms = dom_total / dom_count
    dom_bytes = timer.bytes[dominant] / dom_count

    # The per-kernel table, from its own steps after the timed ones.
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
    for kname, (total_ms, count) in per_kernel.items():
        mean_ms = total_ms / count
        entry = {"ms_per_step": round(total_ms / table_steps, 4), "launches_per_step":
                 count // table_steps, "mean_launch_ms": round(mean_ms, 4)}
        if kname in timer.bytes:
            gbs = timer.bytes[kname] / count / (mean_ms * 1e-3) / 1e9
            entry["GB/s"] = round(gbs, 1)
            entry["frac"] = round(gbs * 1e9 / HBM_PEAK, 4)
        kernels[kname] = entry
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = profiled_traffic(SINGLE_KERNEL[dominant], name)

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
                     args.cpu_sample_tris)
        print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
