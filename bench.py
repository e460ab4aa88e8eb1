"""Benchmark: ms per forward+backward render of the four-op pipeline on one MI355X.

Default workload (the headline configuration): icosphere(8), 1,310,720 triangles, radially
perturbed, 8 views at 1024x1024. One step is

    rasterize -> interpolate(features [1, V, 8]) and interpolate(uv, rast_db, 'all')
    -> texture(1024x1024x4, full mip chain built in the call, trilinear, wrap)
    -> shade = colour + 0.1 * (f[..., 0:4] + f[..., 4:8]) -> antialias -> MSE -> backward

(the feature sum is written as a sum over a [..., 2, 4] view of f, one reduction instead of
two strided slices).

with gradients to positions, features and texture. Inputs are synthetic and resident on the
GPU before timing starts. ``--steps`` steps are timed between synchronisations, after
``--warmup`` untimed ones; the line printed is JSON.

Per-kernel time: every C-ABI entry point called in the timed steps is bracketed by HIP events
on the stream it launches on. ``roofline`` reports the longest-running entry point that
launches a single kernel (so that its event time is that kernel's duration): its algorithmic
bytes per launch -- the unique bytes its algorithm must move, stated per entry point in
``algorithmic_bytes`` -- over its mean duration, against 8 TB/s. ``traffic`` is the HBM bytes
per launch measured for that kernel with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE, each
scaled by the counter's reading for a copy of known size), read from the summary under
profiles/ when one exists for it.

CPU baseline: the oracle (a pure-PyTorch restatement of the reference backend) on the host
cores, on a bounded sample of the same workload -- one view, the visibility pass over a subset
of the triangles and the rest of the pipeline in full -- extrapolated linearly to all triangles
and views.
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
        self.bytes_of = bytes_of
        self.active = False
        self._call = hip.call

    def install(self):
        def timed(name, *args):
            if not self.active:
                return self._call(name, *args)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            self._call(name, *args)
            end.record()
            self.events[name].append((start, end))
            amount = self.bytes_of(name, args)
            if amount is not None:
                self.bytes[name] += amount

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


# Tile rasterization, per tile list entry: the entry (4 B) and the 64-byte record it names
# (three clip-space vertices, triangle row, tile rectangle); per work chunk: the 256 keys of its
# tile read and merged (16 B each).
TILE_ENTRY_BYTES = 4 + 64
TILE_CHUNK_BYTES = 256 * 16


def algorithmic_bytes(w):
    """Unique bytes each entry point must move per launch for this workload (fp32 = 4 B); a
    callable where they depend on the call (the tile pass, on its list sizes)."""
    t = w.tensors
    B, (H, W) = w.batch, w.resolution
    P = B * H * W
    T = t["tri"].shape[0]
    V = t["pos"].shape[1]
    tex_h, tex_w, C = t["tex"].shape[1:]
    L = 0
    h, ww = tex_h, tex_w
    while True:
        L += h * ww
        if max(h, ww) == 1:
            break
        h, ww = (h + 1) // 2, (ww + 1) // 2
    N0 = tex_h * tex_w
    pos = B * V * 16
    tri = T * 12

    def interpolate_forward(args):
        a = args[0]._obj  # rast (and rast_db) in, attributes once, outputs out
        ch, nd = a.channels, a.num_diff
        return (P * 16 + (P * 16 if nd else 0) + tri + a.num_vertices * ch * 4
                + P * ch * 4 + P * 2 * nd * 4)

    def interpolate_backward(args):
        a = args[0]._obj  # output grads and rast in, attribute and rast grads out
        ch, nd = a.channels, a.num_diff
        return (P * ch * 4 + P * 2 * nd * 4 + P * 16 + (P * 16 if nd else 0) + tri
                + 2 * a.num_vertices * ch * 4 + P * 16 + (P * 16 if nd else 0))

    return {
        # visibility set-up: pos and tri in, one key per pixel out
        "dr_raster_visibility_begin": pos + tri + P * 8,
        "dr_raster_visibility_tiles": lambda args: (
            args[6][1] * TILE_ENTRY_BYTES + args[6][2] * TILE_CHUNK_BYTES),
        "dr_resolve_forward": P * 8 + pos + tri + 2 * P * 16,
        "dr_resolve_backward": P * 8 + 2 * P * 16 + pos + tri + pos,
        "dr_interpolate_forward": interpolate_forward,
        "dr_interpolate_backward": interpolate_backward,
        "dr_mip_build": N0 * C * 4 + (L - N0) * C * 4,
        "dr_texture_forward": L * C * 4 + P * 8 + P * 16 + P * C * 4,
        "dr_texture_backward": P * C * 4 + P * 8 + P * 16 + 2 * L * C * 4 + P * 16,
        "dr_mip_build_backward": N0 * C * 4 + (L - N0) * C * 4,
        # rast ids in, the mask cleared and written; the shown triangles' rows and vertices
        "dr_silhouette_mask": P * 16 + 2 * B * T + pos + tri + T * 4 * 3,
        "dr_antialias_forward": 2 * P * C * 4 + P * 16 + pos + tri + B * T,
        "dr_antialias_backward": 3 * P * C * 4 + P * 16 + 2 * pos + tri + B * T,
    }


def make_step(w, device):
    t = {k: v.to(device) for k, v in w.tensors.items()}
    ctx = dr.RasterizeContext(device)
    pos = t["pos"].requires_grad_(True)
    feat = t["feat"].requires_grad_(True)
    tex = t["tex"].requires_grad_(True)
    tri, uv, target = t["tri"], t["uv"], t["target"]

    def step():
        pos.grad = feat.grad = tex.grad = None
        rast, rast_db = dr.rasterize(ctx, pos, tri, w.resolution)
        f, _ = dr.interpolate(feat, rast, tri)
        st, st_da = dr.interpolate(uv, rast, tri, rast_db, diff_attrs="all")
        col = dr.texture(tex, st, st_da, filter_mode="linear-mipmap-linear", boundary_mode="wrap")
        shaded = col + 0.1 * f.view(*f.shape[:-1], 2, 4).sum(-2)  # f[..., :4] + f[..., 4:]
        aa = dr.antialias(shaded, rast, pos, tri)
        loss = torch.nn.functional.mse_loss(aa, target)
        loss.backward()
        return loss

    return step


def cpu_baseline(w, sample_tris: int) -> dict:
    """The oracle on one view: visibility over ``sample_tris`` triangles, the rest in full."""
    from oracle import reference as R

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    t = w.tensors
    B, (H, W) = w.batch, w.resolution
    T = t["tri"].shape[0]
    pos1 = t["pos"][:1].clone()
    tri = t["tri"]
    # (a) visibility on a triangle subset (the reference's brute force over all pixels).
    sub = tri[torch.randperm(T, generator=torch.Generator().manual_seed(0))[:sample_tris]]
    px, py = R.pixel_centres(H, W, pos1)
    start = time.perf_counter()
    with torch.no_grad():
        R.visible_triangles(pos1, sub, px, py)
    vis_s = time.perf_counter() - start
    # (b) everything else on the same view, with the true visibility supplied.
    ids = torch.full((1, H, W), -1, dtype=torch.long)
    if "ids" in t:
        ids = t["ids"][:1]
    p = pos1.clone().requires_grad_(True)
    feat = t["feat"].clone().requires_grad_(True)
    tex = t["tex"].clone().requires_grad_(True)
    start = time.perf_counter()
    rast, rast_db = R.rasterize_from_ids(p, tri, ids, True)
    f, _ = R.interpolate(feat, rast, tri, None, [])
    st, st_da = R.interpolate(t["uv"], rast, tri, rast_db, [0, 1])
    col = R.texture(tex, st, st_da, "linear-mipmap-linear", "wrap", None)
    shaded = col + 0.1 * (f[..., 0:4] + f[..., 4:8])
    aa = R.antialias(shaded, rast, p, tri)
    (aa - t["target"][:1]).square().mean().backward()
    rest_s = time.perf_counter() - start
    total_ms = B * (vis_s * T / sample_tris + rest_s) * 1e3
    return {
        "value": round(total_ms, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one of {B} views at {H}x{W}: reference brute-force visibility over "
                   f"{sample_tris} of {T} triangles ({vis_s:.1f} s) and the rest of the "
                   f"pipeline fwd+bwd in full ({rest_s:.1f} s), extrapolated linearly to "
                   f"{T} triangles and {B} views"),
        "extrapolated": True,
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


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", default="large")
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
    if args.workload != "large":
        raise SystemExit("only the headline workload 'large' is benchmarked here")

    device = torch.device("cuda", 0)
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib, device)
    w = workloads.build(args.workload)
    step = make_step(w, device)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    bytes_model = algorithmic_bytes(w)

    def bytes_of(name, call_args):
        model = bytes_model.get(name)
        return model(call_args) if callable(model) else model

    timer = KernelTimer(bytes_of)
    timer.install()
    timer.active = True
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    timer.active = False
    timer.uninstall()
    ms_per_step = elapsed * 1e3 / args.steps

    per_kernel = timer.summary()
    kernels = {}
    for name, (total_ms, count) in per_kernel.items():
        mean_ms = total_ms / count
        entry = {"ms_per_step": round(total_ms / args.steps, 4), "launches_per_step":
                 count // args.steps, "mean_launch_ms": round(mean_ms, 4)}
        if name in timer.bytes:
            gbs = timer.bytes[name] / count / (mean_ms * 1e-3) / 1e9
            entry["GB/s"] = round(gbs, 1)
            entry["frac"] = round(gbs * 1e9 / HBM_PEAK, 4)
        kernels[name] = entry
    dominant = max((n for n in per_kernel if n in SINGLE_KERNEL and n in timer.bytes),
                   key=lambda n: per_kernel[n][0])
    dom_total, dom_count = per_kernel[dominant]
    dom_ms = dom_total / dom_count
    dom_bytes = timer.bytes[dominant] / dom_count
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = profiled_traffic(SINGLE_KERNEL[dominant], args.workload)

    cpu = None
    if not args.no_cpu_baseline:
        # The true visibility of view 0 for the CPU rest-of-pipeline leg, from the GPU.
        with torch.no_grad():
            rast, _ = dr.rasterize(dr.RasterizeContext(device), w.tensors["pos"][:1].to(device),
                                   w.tensors["tri"].to(device), w.resolution)
        w.tensors["ids"] = (rast[..., 3].long() - 1).cpu()
        cpu = cpu_baseline(w, args.cpu_sample_tris)

    tris = w.tensors["tri"].shape[0]
    result = {
        "metric": METRIC,
        "value": round(ms_per_step, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"icosphere(8) radially perturbed, {tris} triangles, "
                         f"{w.batch} views x {w.resolution[0]}x{w.resolution[1]}, features "
                         "[1,V,8] + uv with derivatives, 1024x1024x4 texture with a full mip "
                         "chain per call, trilinear wrap, antialias, MSE, grads to pos/feat/tex"),
            "views": w.batch,
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
        },
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
