"""Benchmark scenes on the CPU: the reference's published one (displaced grid) against closed
forms of its construction (benchmarks/bench_rasterize.py:19-52, bench_pipeline.py:24-28), the
chart of its sweep as well-formed SVG whose points follow the values, and the cube-map
workload's reflected rays against forward-mode derivatives."""

import json
import math
import xml.etree.ElementTree as ET

import pytest
import torch

from diffrast_amd import pipeline_bench, workloads


@pytest.mark.parametrize("requested,count", [(10_000, 10_082), (100_000, 100_352),
                                             (1_000_000, 999_698)])
def test_grid_triangle_counts_are_the_published_ones(requested, count):
    # The published table's triangle counts (README.md:210-212).
    _, tri, n = workloads.displaced_grid(requested)
    assert tri.shape == (count, 3) and 2 * n * n == count


def test_grid_vertices_triangles_and_uv():
    verts, tri, n = workloads.displaced_grid(200)
    assert n == 10 and verts.shape == ((n + 1) ** 2, 3)
    i, j = torch.meshgrid(torch.arange(n + 1), torch.arange(n + 1), indexing="ij")
    x, z = (-1 + 2 * j / n).reshape(-1), (-1 + 2 * i / n).reshape(-1)
    torch.testing.assert_close(verts[:, 0].double(), x.double(), atol=1e-6, rtol=0)
    torch.testing.assert_close(verts[:, 2].double(), z.double(), atol=1e-6, rtol=0)
    height = 0.1 * torch.sin(6 * x.double()) * torch.cos(5 * z.double())
    torch.testing.assert_close(verts[:, 1].double(), height, atol=1e-6, rtol=0)
    # The triangles tile the square [-1, 1]^2 once, all with one winding: their signed areas
    # in the x-z plane share a sign and add up to 4.
    p = verts[:, [0, 2]].double()[tri.long()]
    e1, e2 = p[:, 1] - p[:, 0], p[:, 2] - p[:, 0]
    area = (e1[:, 0] * e2[:, 1] - e1[:, 1] * e2[:, 0]) / 2
    assert (area > 0).all() or (area < 0).all()
    assert abs(area.abs().sum().item() - 4) < 1e-9
    # A closed-up surface without cracks: every interior edge in exactly two triangles, every
    # border edge in one, and 4 n border edges.
    edges = torch.cat([tri[:, [0, 1]], tri[:, [1, 2]], tri[:, [2, 0]]]).sort(-1).values
    _, uses = torch.unique(edges, dim=0, return_counts=True)
    assert set(uses.tolist()) == {1, 2} and (uses == 1).sum().item() == 4 * n
    # The first half of the list holds each cell's triangle on the (a, b, d) diagonal.
    a = tri[: n * n, 0].long()
    assert torch.equal(tri[: n * n, 1].long(), a + 1)
    assert torch.equal(tri[: n * n, 2].long(), a + n + 2)
    # Planar uv: (x + 1) / 2 and (z + 1) / 2 of each vertex.
    uv = workloads.grid_uv(n)
    torch.testing.assert_close(uv.double(), (verts[:, [0, 2]].double() + 1) / 2, atol=1e-6,
                               rtol=0)


def test_grid_views_turn_about_y_and_project():
    verts, _, _ = workloads.displaced_grid(2_000)
    clip = workloads.grid_views(verts, 8).double()
    v = verts.double()
    cam_x, cam_z = clip[..., 0] / 1.5, clip[..., 3]
    # A turn about the vertical through (0, 2.2): distances to that axis are kept, and height
    # is only shifted.
    radius = cam_x ** 2 + (cam_z - 2.2) ** 2
    torch.testing.assert_close(radius, (v[:, 0] ** 2 + v[:, 2] ** 2).expand_as(radius),
                               atol=1e-5, rtol=0)
    torch.testing.assert_close(clip[..., 1] / 1.5, (v[:, 1] - 0.6).expand_as(cam_x), atol=1e-6,
                               rtol=0)
    # View 2 of 8 is a quarter turn: camera x is world z and camera z is 2.2 - world x.
    torch.testing.assert_close(cam_x[2], v[:, 2], atol=1e-6, rtol=0)
    torch.testing.assert_close(cam_z[2], 2.2 - v[:, 0], atol=1e-6, rtol=0)
    # OpenGL depth: z / w is -1 at the near plane (0.1) and +1 at the far plane (10).
    for w, ndc in ((0.1, -1.0), (10.0, 1.0)):
        a, b = 10.1 / 9.9, 2 * 10 * 0.1 / 9.9
        assert math.isclose((a * w - b) / w, ndc, abs_tol=1e-12)
    z_over_w = clip[..., 2] / clip[..., 3]
    assert (clip[..., 3] > 0.1).all() and (z_over_w > -1).all() and (z_over_w < 1).all()


def _report():
    rows = []
    for requested, count in ((10_000, 10_082), (1_000_000, 999_698)):
        for res in (256, 512, 1024):
            fwd, both = pipeline_bench.PUBLISHED[requested][res]
            rows.append({"triangles": count, "requested_triangles": requested,
                         "resolution": res, "views": 8, "forward_ms": fwd / 5,
                         "forward_backward_ms": both / 5, "published_forward_ms": fwd,
                         "published_forward_backward_ms": both})
    return {"device": "test device", "torch": torch.__version__, "results": rows}


def test_chart_is_svg_with_a_line_per_series_and_points_in_value_order(tmp_path):
    report = _report()
    svg = ET.fromstring(pipeline_bench.chart(report))
    ns = "{http://www.w3.org/2000/svg}"
    lines = svg.findall(f"{ns}polyline")
    # 2 panels x 2 triangle counts x (ours, published).
    assert len(lines) == 8
    circles = svg.findall(f"{ns}circle")
    assert len(circles) == 8 * 3
    # The panels share one log scale: a larger time is drawn higher up (smaller y).
    points = []
    for c in circles:
        ms = float(c.find(f"{ns}title").text.split(": ")[1].split()[0])
        points.append((ms, float(c.get("cy"))))
    by_ms = sorted(points)
    assert all(y1 >= y2 for (_, y1), (_, y2) in zip(by_ms, by_ms[1:]))
    # The --plot mode draws a saved report.
    src, out = tmp_path / "r.json", tmp_path / "c.svg"
    src.write_text(json.dumps(report))
    pipeline_bench.main(["--plot", str(src), str(out)])
    assert ET.parse(out).getroot().tag == f"{ns}svg"


def test_published_figures_are_looked_up_by_requested_count_and_views():
    assert pipeline_bench.published(1_000_000, 1024, 8) == (27.32, 57.88)
    assert pipeline_bench.published(1_000_000, 1024, 1) is None
    assert pipeline_bench.published(50_000, 1024, 8) is None


def test_reflection_and_its_screen_space_derivatives():
    # The cube-map workload's directions: r = v - 2 (n . v) n, and per screen axis the
    # derivative of r along (v + t dv, n + t dn) at t = 0 (forward mode in float64), in
    # interpolate's out_da layout (d/dx, d/dy of each component in turn).
    gen = torch.Generator().manual_seed(3)
    view = torch.randn(2, 5, 7, 3, dtype=torch.float64, generator=gen)
    n = torch.randn(2, 5, 7, 3, dtype=torch.float64, generator=gen)
    view_da = torch.randn(2, 5, 7, 6, dtype=torch.float64, generator=gen)
    n_da = torch.randn(2, 5, 7, 6, dtype=torch.float64, generator=gen)
    dirs, dirs_da = workloads.reflect(view, view_da, n, n_da)

    def r(v, m):
        return v - 2 * (v * m).sum(-1, keepdim=True) * m

    torch.testing.assert_close(dirs, r(view, n), atol=1e-14, rtol=0)
    for axis in (0, 1):
        _, jvp = torch.func.jvp(r, (view, n), (view_da[..., axis::2], n_da[..., axis::2]))
        torch.testing.assert_close(dirs_da[..., axis::2], jvp, atol=1e-12, rtol=0)
