"""Whole forward+backward steps captured in a HIP graph and replayed, and the GPU path driven
from several host threads at once.

Nothing in a step waits for the host once a geometry shape has been seen: visibility sizes its
tile lists from the last counts of that shape and falls back to its overflow pass on the device
when they outgrow the buffer, so a step can be captured (torch.cuda.graph) and replayed. Every
replay is checked against the eager step, with eager work and synchronisations between replays.
"""

import threading

import pytest
import torch

import diffrast_amd as dr
from diffrast_amd import workloads
from diffrast_amd.backends import hip

pytestmark = pytest.mark.gpu


def _mse_backward(out, target):
    """The backward pass of mean((out - target)^2), started from its elementwise gradient: a
    PyTorch reduction over many workgroups records memory fills into a captured graph, which
    give wrong results on replays after the first on this platform, so the loss itself stays
    out of the graph. Returns out."""
    out.backward((out.detach() - target) * (2.0 / out.numel()))
    return out


def _sphere_step(t, ctx, res):
    pos, attr, tri, target = t["pos"], t["attr"], t["tri"], t["target"]

    def body():
        rast, _ = dr.rasterize(ctx, pos, tri, res, grad_db=False)
        col, _ = dr.interpolate(attr, rast, tri)
        out = _mse_backward(dr.antialias(col, rast, pos, tri), target)
        return out.detach(), rast

    return body, (pos, attr)


def _textured_step(t, ctx, res):
    pos, tex, tri, uv_attr, target = t["pos"], t["tex"], t["tri"], t["uv"], t["target"]

    def body():
        rast, rast_db = dr.rasterize(ctx, pos, tri, res)
        uv, uv_da = dr.interpolate(uv_attr, rast, tri, rast_db, diff_attrs="all")
        col = dr.texture(tex, uv, uv_da, mip=dr.texture_construct_mip(tex),
                         filter_mode="linear-mipmap-linear", boundary_mode="wrap")
        out = _mse_backward(dr.antialias(col, rast, pos, tri), target)
        return out.detach(), rast_db

    return body, (pos, tex)


def _instances_step(t, ctx, res):
    # Range mode with depth peeling (a new peeler every step, as an application would make it),
    # then antialias on the first layer.
    pos, color, tri, target = t["pos"], t["color"], t["tri"], torch.zeros_like(t["color"])
    ranges = t["ranges"].cpu()

    def body():
        with dr.DepthPeeler(ctx, pos, tri, res, ranges=ranges) as peeler:
            layers = [peeler.rasterize_next_layer()[0] for _ in range(4)]
        out = _mse_backward(dr.antialias(color, layers[0], pos, tri), target)
        return out.detach(), torch.cat(layers)

    return body, (pos, color)


def _assert_gradients_equal(got, expected, what):
    # Gradients gather per workgroup in fixed point (exact) and then add to global memory with
    # float atomics, whose order varies from run to run: equal up to that last rounding.
    for g, e in zip(got, expected):
        scale = e.abs().max().item()
        torch.testing.assert_close(g, e, atol=1e-6 * scale, rtol=1e-6, msg=str(what))


@pytest.mark.parametrize("name, make, scale", [("sphere", _sphere_step, 1),
                                               ("textured", _textured_step, 2),
                                               ("instances", _instances_step, 4)])
def test_step_captured_in_a_graph_matches_eager(name, make, scale):
    w = workloads.build(name, "cuda", scale=scale)
    ctx = dr.RasterizeContext("cuda")

    def fresh():
        t = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in w.tensors.items()}
        body, leaves = make(t, ctx, w.resolution)
        for x in leaves:
            x.requires_grad_(True)
        return body, leaves

    # Eager reference (the first call of the shape also learns its tile-list sizes).
    body, leaves = fresh()
    out, extra = body()
    expected = [out.clone(), extra.detach().clone()] + [x.grad.clone() for x in leaves]

    # Capture: warm up on a side stream, then record one step.
    body, leaves = fresh()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for x in leaves:
                x.grad = None
            body()
    torch.cuda.current_stream().wait_stream(side)
    for x in leaves:
        x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out, static_extra = body()
    static_grads = [x.grad for x in leaves]

    other_body, other_leaves = fresh()
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, expected[0]), (name, replay, "output")
        assert torch.equal(static_extra, expected[1]), (name, replay, "rasterize outputs")
        _assert_gradients_equal(static_grads, expected[2:], (name, replay))
        # Eager work between replays, on other tensors.
        for x in other_leaves:
            x.grad = None
        other_body()
        torch.cuda.synchronize()


def test_four_threads_rasterize_and_antialias():
    """Four host threads run rasterize + antialias, each on its own stream and its own scenes
    of two sizes (so the remembered list sizes of a shape are shared and updated concurrently),
    and must reproduce the single-threaded results."""
    w = workloads.build("textured", "cuda", scale=2)
    base_pos, tri = w.tensors["pos"], w.tensors["tri"]
    scenes = []
    for i in range(8):
        pos = base_pos.clone()
        pos[..., :2] *= 0.5 + 0.1 * i
        scenes.append(pos)
    color = torch.rand(*base_pos.shape[:1], *w.resolution, 3, device="cuda",
                       generator=torch.Generator("cuda").manual_seed(0))
    ctx = dr.RasterizeContext("cuda")

    def run(pos):
        p = pos.clone().requires_grad_(True)
        rast, _ = dr.rasterize(ctx, p, tri, w.resolution)
        out = dr.antialias(color, rast, p, tri)
        out.sum().backward()
        return rast.detach(), out.detach(), p.grad

    expected = [run(p) for p in scenes]
    torch.cuda.synchronize()
    hip._SIZES.clear()
    results, errors = {}, []

    def worker(k):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for rep in range(3):
                    for i in range(k, len(scenes), 4):
                        results[(k, rep, i)] = run(scenes[i])
            stream.synchronize()
        except Exception as exc:  # reported below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    torch.cuda.synchronize()
    assert len(results) == 3 * len(scenes)
    for (k, rep, i), got in results.items():
        assert torch.equal(got[0], expected[i][0]) and torch.equal(got[1], expected[i][1])
        _assert_gradients_equal(got[2:], expected[i][2:], (k, rep, i))
