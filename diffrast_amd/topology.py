"""Edge adjacency of an index buffer, the part of antialiasing that depends on ``tri`` alone
(the reference's src/diffrast/topology.py API: ``TopologyHash`` and ``neighbours_for``).

The adjacency is built on the GPU (a hash table of each edge's vertex pair, csrc/antialias.hip)
once per index buffer: explicitly, by ``antialias_construct_topology_hash``, or on first use,
remembered per ``tri`` tensor object.
"""

from __future__ import annotations

import weakref

from torch import Tensor

from diffrast_amd._cache import TensorCache, fingerprint
from diffrast_amd.backends import get_backend


def _build(tri: Tensor) -> Tensor:
    return get_backend(tri.device, "antialias").edge_neighbours(tri)


class TopologyHash:
    """Edge adjacency built by ``antialias_construct_topology_hash``; its contents are private.

    Valid for the ``tri`` it was built from and for any tensor of the same shape and contents on
    the same device. An in-place edit of the original ``tri``, when PyTorch records it, makes it
    refuse that tensor.
    """

    def __init__(self, tri: Tensor) -> None:
        self._adjacency = _build(tri)
        self._shape = tuple(tri.shape)
        self._device = tri.device
        # What the source tensor looked like, to notice in-place edits of that same object.
        self._origin: tuple[weakref.ref, tuple | None] | None = (weakref.ref(tri), fingerprint(tri))

    def __repr__(self) -> str:
        return f"TopologyHash(triangles={self._shape[0]}, device={str(self._device)!r})"

    def __getstate__(self) -> dict:
        # A copy or pickle keeps the adjacency; the weak link to the source cannot travel.
        state = dict(self.__dict__)
        state["_origin"] = None
        return state

    def _edited(self, tri: Tensor) -> bool:
        if self._origin is None:
            return False
        source, recorded = self._origin
        return source() is tri and fingerprint(tri) != recorded

    def neighbours(self, tri: Tensor) -> Tensor:
        """The adjacency, int32 ``[triangles, 3]``, after checking that it fits ``tri``."""
        if (tuple(tri.shape), tri.device) != (self._shape, self._device):
            raise ValueError(
                f"topology_hash was built for a tri of shape {self._shape} on {self._device}, "
                f"got shape {tuple(tri.shape)} on {tri.device}."
            )
        if self._edited(tri):
            raise ValueError(
                "tri was modified in place after topology_hash was built from it; build a new "
                "one with antialias_construct_topology_hash."
            )
        return self._adjacency


# Each entry is the size of its index buffer: a few suffice.
_neighbour_cache: TensorCache[Tensor] = TensorCache(_build, max_entries=16)


def neighbours_for(tri: Tensor, topology_hash: TopologyHash | None) -> Tensor:
    """Adjacency of ``tri``, from ``topology_hash`` when given, else remembered per tensor."""
    if topology_hash is None:
        return _neighbour_cache.get(tri)
    if isinstance(topology_hash, TopologyHash):
        return topology_hash.neighbours(tri)
    raise TypeError(
        "topology_hash must come from antialias_construct_topology_hash, got "
        f"{type(topology_hash).__name__}."
    )
