"""The CPU oracle wrapped in the backend protocol, for host-logic tests on the CPU.

Tests install it with the ``oracle_backend`` fixture (tests/test_host.py) to drive the public
API -- validation, range mode, DepthPeeler, MipStack, topology caching -- without a GPU. The
product never loads it.
"""

import torch

from oracle import reference as R

IMPLEMENTED = frozenset({"rasterize", "interpolate", "texture", "antialias"})
rasterize = R.rasterize
rasterize_layer = R.rasterize_layer
interpolate = R.interpolate
texture = R.texture
antialias = R.antialias
texture_construct_mip = R.texture_construct_mip
edge_neighbours = R.edge_neighbours
pack = R.pack


def rasterize_ranges(pos, tri, resolution, grad_db, ranges, previous=None):
    states = previous or [None] * ranges.shape[0]
    rasts, dbs, new = [pos.new_zeros(0, *resolution, 4)], [pos.new_zeros(0, *resolution, 4)], []
    for (start, count), state in zip(ranges.tolist(), states):
        rast, db, s = R.rasterize_layer(pos[None], tri[start:start + count], resolution,
                                        grad_db, state)
        ids = rast[..., 3:]
        rasts.append(torch.cat([rast[..., :3], torch.where(ids > 0, ids + start, ids)], -1))
        dbs.append(db)
        new.append(s)
    return torch.cat(rasts), torch.cat(dbs), new
