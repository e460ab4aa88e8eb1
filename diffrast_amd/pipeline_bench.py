"""Time the full differentiable render on the reference's published benchmark scene, and draw
the table as an SVG chart.

The scene and the timing rule are those of the reference's benchmarks/bench_pipeline.py:21-44
and bench_rasterize.py:19-73: a displaced grid of about 10k, 100k or 1M triangles seen from 8
views at 256^2 to 2048^2, planar uv, a 1024x1024x3 texture, and per call

    rasterize -> interpolate(uv, rast_db, 'all') -> texture(linear-mipmap-linear, mip chain
    built in the call) -> antialias

timed without autograd ("forward") and with ``.sum().backward()`` into positions and texture
("forward + backward"). Each figure is the median of individually synchronised calls after a
warm-up. The reference's own figures for an RX 9070 XT (README.md:208-212) are printed beside
ours, with the ratio.

Usage:
    python -m diffrast_amd.pipeline_bench [--triangles ...] [--resolutions ...] [--views ...]
        [--repeats 15] [--warmup 1.0] [--json results.json] [--svg chart.svg]
    python -m diffrast_amd.pipeline_bench --plot results.json chart.svg
"""

from __future__ import annotations

import argparse
import json
import math
import platform
import statistics
import time
from html import escape

import torch

# The reference's figures, RX 9070 XT, 8 views (README.md:208-212, docs/images/pipeline.svg):
# requested triangles -> resolution -> (forward ms, forward + backward ms).
PUBLISHED_DEVICE = "AMD Radeon RX 9070 XT (reference, Triton backend)"
PUBLISHED = {
    10_000: {256: (3.96, 6.92), 512: (5.33, 12.64), 1024: (7.39, 39.56), 2048: (20.75, 139.08)},
    100_000: {256: (4.87, 8.30), 512: (7.39, 13.19), 1024: (9.39, 39.15),
              2048: (25.62, 137.71)},
    1_000_000: {256: (25.89, 28.77), 512: (25.86, 34.67), 1024: (27.32, 57.88),
                2048: (43.05, 144.38)},
}
PUBLISHED_VIEWS = 8


class Scene:
    """The grid of about ``num_tri`` triangles from ``views`` cameras, on ``device``."""

    def __init__(self, num_tri: int, views: int, device: torch.device) -> None:
        from diffrast_amd import workloads

        verts, tri, n = workloads.displaced_grid(num_tri)
        self.requested = num_tri
        self.views = views
        self.pos = workloads.grid_views(verts, views).to(device)
        self.tri = tri.to(device)
        self.uv = workloads.grid_uv(n).to(device)
        gen = torch.Generator().manual_seed(0)
        self.tex = torch.rand(1, 1024, 1024, 3, generator=gen).to(device)

    @property
    def triangles(self) -> int:
        return self.tri.shape[0]


def render(dr, ctx, scene: Scene, pos, tex, res: int):
    rast, rast_db = dr.rasterize(ctx, pos, scene.tri, (res, res))
    uv, uv_da = dr.interpolate(scene.uv, rast, scene.tri, rast_db=rast_db, diff_attrs="all")
    color = dr.texture(tex, uv, uv_da, filter_mode="linear-mipmap-linear")
    return dr.antialias(color, rast, pos, scene.tri)


def median_ms(fn, repeats: int, warmup_s: float) -> float:
    """Median wall time of ``repeats`` calls of ``fn``, each followed by a device
    synchronisation, after calling it for ``warmup_s`` seconds (at least twice)."""
    start, calls = time.perf_counter(), 0
    while calls < 2 or time.perf_counter() - start < warmup_s:
        fn()
        torch.cuda.synchronize()
        calls += 1
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e3


def measure(dr, ctx, scene: Scene, res: int, repeats: int, warmup_s: float):
    pos = scene.pos.clone().requires_grad_(True)
    tex = scene.tex.clone().requires_grad_(True)

    def forward():
        with torch.no_grad():
            render(dr, ctx, scene, pos, tex, res)

    def forward_backward():
        render(dr, ctx, scene, pos, tex, res).sum().backward()

    return median_ms(forward, repeats, warmup_s), median_ms(forward_backward, repeats, warmup_s)


def published(requested: int, res: int, views: int):
    if views != PUBLISHED_VIEWS:
        return None
    return PUBLISHED.get(requested, {}).get(res)


def sweep(args) -> dict:
    import diffrast_amd as dr

    device = torch.device("cuda", 0)
    ctx = dr.RasterizeContext(device)
    name = torch.cuda.get_device_name(device)
    print(f"device: {name}, torch {torch.__version__}", flush=True)
    head = "{:>10} {:>5} {:>5} {:>9} {:>11} {:>14} {:>14}"
    print(head.format("triangles", "res", "views", "fwd ms", "fwd+bwd ms", "ref fwd (x)",
                      "ref f+b (x)"), flush=True)
    results = []
    for num_tri in args.triangles:
        for views in args.views:
            scene = Scene(num_tri, views, device)
            for res in args.resolutions:
                fwd, both = measure(dr, ctx, scene, res, args.repeats, args.warmup)
                ref = published(num_tri, res, views)
                row = {"triangles": scene.triangles, "requested_triangles": num_tri,
                       "resolution": res, "views": views, "forward_ms": round(fwd, 3),
                       "forward_backward_ms": round(both, 3)}
                cells = ["", ""]
                if ref is not None:
                    row["published_forward_ms"], row["published_forward_backward_ms"] = ref
                    cells = [f"{ref[0]:.2f} ({ref[0] / fwd:.1f})",
                             f"{ref[1]:.2f} ({ref[1] / both:.1f})"]
                results.append(row)
                print(head.format(scene.triangles, res, views, f"{fwd:.2f}", f"{both:.2f}",
                                  *cells), flush=True)
            del scene
            torch.cuda.empty_cache()
    return {"device": name, "torch": torch.__version__, "platform": platform.platform(),
            "published_device": PUBLISHED_DEVICE, "repeats": args.repeats,
            "warmup_s": args.warmup, "results": results}


# ---- chart -------------------------------------------------------------------------------------

_BACK, _RULE, _INK, _SOFT = "#ffffff", "#e3e3e3", "#202020", "#707070"
_SHADES = ("#0b4f6c", "#20a4a4", "#97d8c4")  # ours: one hue per triangle count
_THEIRS = ("#8c2f39", "#c8553d", "#f2a541")  # published: another hue per triangle count
_W, _H = 880, 470
_TOP, _BOTTOM = 120, 380


def _short(count: int) -> str:
    if count >= 950_000:
        return f"{count / 1e6:.0f}M"
    return f"{count / 1e3:.0f}k"


def _label(x, y, body, size=12, color=_SOFT, anchor="start", bold=False) -> str:
    weight = ' font-weight="600"' if bold else ""
    return (f'<text x="{x:.1f}" y="{y:.1f}" font-size="{size}" fill="{color}" '
            f'text-anchor="{anchor}"{weight}>{escape(body)}</text>')


def chart(report: dict, views: int = PUBLISHED_VIEWS) -> str:
    """Two log-scale panels (forward; forward + backward) of ms against resolution, one solid
    line per triangle count for these kernels and a dashed one for the published figures."""
    rows = [r for r in report["results"] if r["views"] == views]
    if not rows:
        raise ValueError(f"no results for {views} views")
    res_axis = sorted({r["resolution"] for r in rows})
    counts = sorted({r["requested_triangles"] for r in rows})
    keys = (("forward_ms", "published_forward_ms", "forward"),
            ("forward_backward_ms", "published_forward_backward_ms", "forward + backward"))
    values = [r[k] for r in rows for pair in keys for k in pair[:2] if k in r]
    lo = 10 ** math.floor(math.log10(min(values)))
    hi = 10 ** math.ceil(math.log10(max(values)))

    def y_at(ms):
        f = (math.log10(ms) - math.log10(lo)) / (math.log10(hi) - math.log10(lo))
        return _BOTTOM - f * (_BOTTOM - _TOP)

    svg = [f'<svg xmlns="http://www.w3.org/2000/svg" width="{_W}" height="{_H}" '
           f'viewBox="0 0 {_W} {_H}" font-family="Helvetica, Arial, sans-serif">',
           f'<rect width="{_W}" height="{_H}" fill="{_BACK}"/>',
           _label(20, 30, f"Differentiable render of a displaced grid, {views} views per call",
                  16, _INK, bold=True),
           _label(20, 50, "rasterize, interpolate with derivatives, mipmapped 1024² texture, "
                  "antialias; ms per call (median), log scale")]
    x = 20
    for i, n in enumerate(counts):
        for dashed, colors, who in ((False, _SHADES, "MI355X"), (True, _THEIRS, "RX 9070 XT")):
            if dashed and not any("published_forward_ms" in r for r in rows
                                  if r["requested_triangles"] == n):
                continue
            dash = ' stroke-dasharray="5 4"' if dashed else ""
            color = colors[i % len(colors)]
            svg.append(f'<line x1="{x}" y1="74" x2="{x + 24}" y2="74" stroke="{color}" '
                       f'stroke-width="2.5"{dash}/>')
            name = f"{_short(n)} tris, {who}"
            svg.append(_label(x + 30, 78, name, 11, _INK))
            x += 46 + 6.2 * len(name)
    for p, (ours, theirs, title) in enumerate(keys):
        left = 70 + p * 420
        right = left + 360
        svg.append(_label(left, _TOP - 14, title, 13, _INK, bold=True))
        span = (right - left - 20) / max(len(res_axis) - 1, 1)

        def x_at(res, left=left, span=span):
            return left + 10 + res_axis.index(res) * span

        decade = lo
        while decade <= hi * 1.0001:
            y = y_at(decade)
            svg.append(f'<line x1="{left}" y1="{y:.1f}" x2="{right}" y2="{y:.1f}" '
                       f'stroke="{_RULE}"/>')
            text = f"{decade:g} ms" if decade < 1000 else f"{decade / 1000:g} s"
            svg.append(_label(left - 6, y + 4, text, 10, _SOFT, "end"))
            decade *= 10
        for res in res_axis:
            svg.append(_label(x_at(res), _BOTTOM + 18, f"{res}²", 10, _SOFT, "middle"))
        svg.append(_label((left + right) / 2, _BOTTOM + 38, "pixels per view", 10, _SOFT,
                          "middle"))
        for i, n in enumerate(counts):
            mine = [r for r in rows if r["requested_triangles"] == n]
            for key, colors, dashed in ((ours, _SHADES, False), (theirs, _THEIRS, True)):
                points = sorted((r["resolution"], r[key]) for r in mine if key in r)
                if not points:
                    continue
                color = colors[i % len(colors)]
                dash = ' stroke-dasharray="5 4"' if dashed else ""
                line = " ".join(f"{x_at(res):.1f},{y_at(ms):.1f}" for res, ms in points)
                svg.append(f'<polyline points="{line}" fill="none" stroke="{color}" '
                           f'stroke-width="2.5"{dash}/>')
                for res, ms in points:
                    svg.append(f'<circle cx="{x_at(res):.1f}" cy="{y_at(ms):.1f}" r="3.5" '
                               f'fill="{color}"><title>{_short(n)} triangles, {res}²: '
                               f'{ms:.2f} ms</title></circle>')
    foot = f"{report['device']}, torch {report['torch']}"
    if any("published_forward_ms" in r for r in rows):
        foot += f"; dashed: {report.get('published_device', PUBLISHED_DEVICE)}"
    svg.append(_label(20, _H - 14, foot, 10, _SOFT))
    svg.append("</svg>")
    return "\n".join(svg)


def main(argv=None) -> None:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--triangles", nargs="+", type=int, default=[10_000, 100_000, 1_000_000])
    parser.add_argument("--resolutions", nargs="+", type=int, default=[256, 512, 1024, 2048])
    parser.add_argument("--views", nargs="+", type=int, default=[PUBLISHED_VIEWS])
    parser.add_argument("--repeats", type=int, default=15)
    parser.add_argument("--warmup", type=float, default=1.0, help="warm-up seconds per timing")
    parser.add_argument("--json", help="write the results to this file")
    parser.add_argument("--svg", help="draw the results to this file")
    parser.add_argument("--plot", nargs=2, metavar=("RESULTS", "SVG"),
                        help="only draw an earlier --json file")
    args = parser.parse_args(argv)
    if args.plot:
        with open(args.plot[0]) as f:
            report = json.load(f)
        with open(args.plot[1], "w", encoding="utf-8") as f:
            f.write(chart(report))
        return
    report = sweep(args)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(report, f, indent=1)
    if args.svg:
        with open(args.svg, "w", encoding="utf-8") as f:
            f.write(chart(report))


if __name__ == "__main__":
    main()
