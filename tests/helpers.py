"""Scene generators and comparisons shared by the tests."""

from __future__ import annotations

import torch


def random_mesh(num_tri, gen, batch=1, z_range=0.9, w_range=(1.0, 2.0), xy_range=1.2):
    """Independent random triangles in clip space."""
    n = 3 * num_tri
    xy = (torch.rand(batch, n, 2, generator=gen) * 2 - 1) * xy_range
    z = (torch.rand(batch, n, 1, generator=gen) * 2 - 1) * z_range
    w = torch.rand(batch, n, 1, generator=gen) * (w_range[1] - w_range[0]) + w_range[0]
    return torch.cat([xy * w, z * w, w], -1), torch.arange(n, dtype=torch.int32).view(-1, 3)


def tiny_mesh(num_tri, gen, size, batch=1):
    """Triangles about ``size`` NDC units across, over and just past the screen."""
    centre = torch.rand(batch, num_tri, 1, 2, generator=gen) * 2.2 - 1.1
    offset = (torch.rand(batch, num_tri, 3, 2, generator=gen) * 2 - 1) * size
    xy = (centre + offset).reshape(batch, 3 * num_tri, 2)
    z = torch.rand(batch, 3 * num_tri, 1, generator=gen) * 1.8 - 0.9
    w = torch.rand(batch, 3 * num_tri, 1, generator=gen) + 1.0
    pos = torch.cat([xy * w, z * w, w], -1)
    return pos, torch.arange(3 * num_tri, dtype=torch.int32).view(-1, 3)


def mixed_mesh(gen, batch=2):
    small, small_tri = tiny_mesh(1500, gen, 0.04, batch=batch)
    large, large_tri = random_mesh(40, gen, batch=batch)
    return torch.cat([small, large], 1), torch.cat([small_tri, large_tri + small.shape[1]])


def rel_error(ours, truth, floor=1.0):
    """max |ours - truth| / max(|truth|, floor)."""
    ours, truth = ours.double(), truth.double()
    return ((ours - truth).abs() / truth.abs().clamp_min(floor)).max().item()
