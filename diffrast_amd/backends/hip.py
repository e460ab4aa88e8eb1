"""The HIP backend: the reference's backend protocol on MI355X kernels.

Implements the functions that ``diffrast_amd.ops`` and ``DepthPeeler`` call on a backend module,
with the signatures of the reference backends (src/diffrast/backends/triton.py:14-92,
reference.py:38-265): ``rasterize``, ``rasterize_layer``, ``interpolate``, ``texture``,
``antialias``, plus what the reference's ops layer takes from its reference backend directly
(ops.py:259-300, topology.py:16): ``texture_construct_mip``, ``pack``, ``edge_neighbours``, and
the batched range mode ``rasterize_ranges`` that replaces the per-item loop of ops.py:69-74 and
peeling.py:80-92.

Each op is a ``torch.autograd.Function`` whose forward and backward call the C ABI of
libdiffrast_hip.so on the current stream of the tensors' device. Inputs arrive validated by
``ops.py`` (float32 / int32, shapes checked) and are made contiguous here. The backward passes
are kernels and cannot be differentiated again (``first_order``).
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from collections.abc import Sequence

import torch
from torch import Tensor

from diffrast_amd.backends import _lib
from diffrast_amd.backends._autograd import first_order
from diffrast_amd.backends._lib import call, ptr, ref

IMPLEMENTED: frozenset[str] = frozenset({"rasterize", "interpolate", "texture", "antialias"})

# A key with every bit set marks a pixel that no triangle covers (uint64 max, stored in int64).
EMPTY_KEY = -1

FILTERS = {"nearest": 0, "linear": 1, "linear-mipmap-nearest": 2, "linear-mipmap-linear": 3}
BOUNDARIES = {"wrap": 0, "clamp": 1, "zero": 2, "cube": 3}


def _require(name: str, t: Tensor | None, dtype: torch.dtype) -> None:
    """The kernels read raw pointers: a tensor of another type would be reinterpreted, so it
    is refused here (the reference backend module accepts only what its kernels compute in)."""
    if t is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}.")


def _real(*named: tuple[str, Tensor | None]) -> torch.dtype:
    """The one floating type of the given tensors: float32 (the product kernels) or float64
    (their gradient-check twins, as the reference's GPU backend accepts at this level)."""
    first = next((t for _, t in named if t is not None), None)
    dtype = torch.float32 if first is None else first.dtype
    if dtype not in (torch.float32, torch.float64):
        dtype = torch.float32  # names the first tensor below
    for name, t in named:
        _require(name, t, dtype)
    return dtype


def _entry(name: str, t: Tensor) -> str:
    """The C-ABI entry point for computing in t's type: name, or its float64 twin."""
    return name + "_f64" if t.dtype == torch.float64 else name


def _dense(t: Tensor | None) -> Tensor | None:
    return None if t is None else t.contiguous()


def _saveable(t: Tensor | None) -> Tensor | None:
    # Inference tensors cannot be saved for backward (reference _triton_interpolate.py:214-215).
    return t.clone() if t is not None and t.is_inference() else t


def _stream(t: Tensor) -> int:
    return _lib.stream(t.device)


# ---------------------------------------------------------------------------------------------
# Rasterize
# ---------------------------------------------------------------------------------------------


class _Geometry:
    """DrRasterGeometry of one call, kept alive with the tensors it points to."""

    def __init__(self, pos: Tensor, tri: Tensor, resolution, ranges=None, range_prefix=None,
                 batch=None, num_instances=None):
        height, width = resolution
        self.pos, self.tri = pos, tri
        self.ranges, self.range_prefix = ranges, range_prefix
        shared = pos.ndim == 2
        self.batch = int(batch if batch is not None else pos.shape[0])
        num_tri = int(tri.shape[0])
        self.struct = _lib.RasterGeometry(
            pos=ptr(pos),
            pos_batch_stride=0 if (shared or (pos.shape[0] == 1 and self.batch > 1))
            else pos.shape[1] * 4,
            tri=ptr(tri),
            num_tri=num_tri,
            batch=self.batch,
            height=int(height),
            width=int(width),
            ranges=ptr(ranges),
            range_prefix=ptr(range_prefix),
            num_instances=int(num_instances if num_instances is not None else self.batch * num_tri),
            num_vertices=int(pos.shape[-2]),
        )
        self.shape = (self.batch, int(height), int(width))
        self.order = None  # the processing order the struct points to, kept alive with it


class _Sizes:
    """What the last finished visibility call of one geometry shape found -- its tile entries
    and tile-pass workgroups -- and the pinned buffer and event through which a later call's
    counts come back without anyone waiting for them."""

    __slots__ = ("entries", "groups", "counts", "event", "pending", "lock")

    def __init__(self, entries: int, groups: int):
        self.entries, self.groups = entries, groups
        self.counts = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        self.event = torch.cuda.Event()
        self.pending = False
        self.lock = threading.Lock()

    def refresh(self) -> None:
        """Takes in the counts of the last call that sent them back, if they have arrived."""
        if self.pending and self.event.query():
            found = [v & 0xFFFFFFFF for v in self.counts.tolist()]
            self.entries, self.groups = found[1], found[2]
            self.pending = False


_SIZES: dict[tuple, _Sizes] = {}
_SIZES_KEPT = 64
_sizes_lock = threading.Lock()
_host = threading.local()


def _entry_capacity(count: int) -> int:
    return min(count + count // 8 + 4096, 0xffffffff)


# The tile pass runs one workgroup per 16x16 tile when that grid is at most this many
# workgroups and none smaller is asked for (dr_raster_visibility_tiles).
_PLAIN_TILE_GRID = 1 << 16


def _tile_grid(geo: _Geometry, groups: int) -> int:
    """The tile pass's grid to ask for: none (one workgroup per tile) while that grid is small
    enough for the kernel without the tile loop, which keeps fewer registers; else ``groups``
    (a smaller grid runs the looping kernel, which covers every tile for any grid)."""
    batch, height, width = geo.shape
    tiles = batch * (-(-height // 16)) * (-(-width // 16))
    return 0 if tiles <= _PLAIN_TILE_GRID else groups


def _host_counts(device: torch.device) -> tuple[Tensor, torch.cuda.Event]:
    """Pinned memory for the counts of a first call and the event that marks their arrival
    (one pair per host thread and device: such a call waits for its counts)."""
    per_device = getattr(_host, "counts", None)
    if per_device is None:
        per_device = _host.counts = {}
    pair = per_device.get(device.index)
    if pair is None:
        pair = (torch.zeros(4, dtype=torch.int32, pin_memory=True), torch.cuda.Event())
        per_device[device.index] = pair
    return pair


def _remember(key: tuple, sizes: _Sizes) -> None:
    with _sizes_lock:
        if len(_SIZES) >= _SIZES_KEPT and key not in _SIZES:
            _SIZES.pop(next(iter(_SIZES)), None)
        _SIZES[key] = sizes


class _Order:
    """A mesh's processing order on the device, the tri it was computed from (a weak
    reference: the order is valid for that tensor only) and whether a captured graph refers
    to it."""

    __slots__ = ("tensor", "ref", "pinned")

    def __init__(self, tensor: Tensor, ref: weakref.ref):
        self.tensor, self.ref, self.pinned = tensor, ref, False


_ORDERS: dict[tuple, _Order] = {}
_ORDERS_KEPT = 8
# Re-entrant: a tri freed by the garbage collector while this thread holds the lock calls
# _forget_order.
_orders_lock = threading.RLock()


def _forget_order(key: tuple, dead: weakref.ref) -> None:
    # A freed tri frees its order, pinned or not: a graph that drew it reads tri's memory too,
    # so it cannot be replayed once tri is gone. The key may already name a newer tensor's
    # entry (same address and version): only the dead tensor's own entry goes.
    with _orders_lock:
        entry = _ORDERS.get(key)
        if entry is not None and entry.ref is dead:
            del _ORDERS[key]


def _order(geo: _Geometry, workspace: Tensor, workspace_bytes: int, capturing: bool) -> None:
    """Sets geo.struct.order to the processing order of geo's mesh, computed once per tri
    tensor and reused while that tensor lives and is unchanged (its version counter): the
    order is a spatial sort that only the speed of the visibility depends on, so an order
    computed from earlier positions of the same triangles stays valid. An entry is found by
    the tensor's address, version and sizes and accepted only for the very tensor it was
    computed from (a new tri at a freed tri's address, with the same sizes and a fresh version
    counter, gets its own). Under graph capture a remembered order is used and then kept while
    its tri lives (the graph refers to it); none is computed there (the captured visibility
    computes its own into the workspace)."""
    size = ctypes.c_size_t()
    call("dr_raster_order_size", ref(geo.struct), ctypes.byref(size))
    if size.value == 0:
        return
    tri, device = geo.tri, geo.pos.device
    if tri.is_inference():  # no version counter to tell a changed tri: the call orders itself
        return
    key = (device.index, tri.data_ptr(), tri._version, geo.struct.num_tri,
           geo.struct.num_vertices)
    with _orders_lock:
        entry = _ORDERS.get(key)
        if entry is not None and entry.ref() is not tri:
            entry = None  # another tensor's order at a reused address
        if entry is not None and capturing:
            entry.pinned = True
    if entry is None:
        if capturing:
            return
        tensor = torch.empty(size.value, dtype=torch.uint8, device=device)
        call("dr_raster_order", ref(geo.struct), ptr(tensor), size.value, ptr(workspace),
             workspace_bytes, _lib.stream(device))
        entry = _Order(tensor, weakref.ref(tri, lambda dead, key=key: _forget_order(key, dead)))
        with _orders_lock:
            _ORDERS.pop(key, None)
            if len(_ORDERS) >= _ORDERS_KEPT:
                for old in list(_ORDERS):
                    if not _ORDERS[old].pinned:
                        _ORDERS.pop(old)
                        break
            _ORDERS[key] = entry
    elif not capturing:
        # Freed later (once evicted) while this call's kernels may still read it.
        entry.tensor.record_stream(torch.cuda.current_stream(device))
    geo.order = entry.tensor
    geo.struct.order = entry.tensor.data_ptr()


def share_order(source: Tensor, copy: Tensor) -> bool:
    """Lets ``copy``, a tensor holding what ``source`` holds now (a depth peeler's copy of its
    tri), use the processing orders remembered for ``source``: an order depends only on the
    contents of tri (and the vertex count, part of its key), so the two can share it instead of
    the copy computing its own (some 27 ms at 1.3M triangles) in its first call. Nothing happens
    where ``source`` has no order yet or either tensor keeps no version counter. Returns
    whether an order was shared."""
    if source.is_inference() or copy.is_inference() or source.shape != copy.shape:
        return False
    shared = False
    with _orders_lock:
        found = [(key, entry) for key, entry in _ORDERS.items()
                 if entry.ref() is source and key[1] == source.data_ptr()
                 and key[2] == source._version]
        for (device, _, _, num_tri, num_vertices), entry in found:
            key = (device, copy.data_ptr(), copy._version, num_tri, num_vertices)
            held = _ORDERS.get(key)
            if held is not None and held.ref() is copy:
                shared = True
                continue
            _ORDERS.pop(key, None)
            if len(_ORDERS) >= _ORDERS_KEPT:
                for old in list(_ORDERS):
                    if not _ORDERS[old].pinned:
                        _ORDERS.pop(old)
                        break
            _ORDERS[key] = _Order(entry.tensor, weakref.ref(
                copy, lambda dead, key=key: _forget_order(key, dead)))
            shared = True
    return shared


def _visibility(geo: _Geometry, previous: Tensor | None) -> Tensor:
    """Visibility keys [batch, height, width] (int64 holding the uint64 key bits).

    The first call of a geometry shape learns the tile-list sizes from the device (one wait
    for four counts) and bins into a buffer of exactly that size. Later calls -- and every call
    under HIP graph capture -- queue the whole visibility at once with a buffer sized from the
    last counts seen for the shape, which come back through pinned memory without a wait; if
    the lists outgrow the buffer, the device rasterizes the binned triangles through its
    overflow pass instead (same keys)."""
    device = geo.pos.device
    keys = torch.empty(geo.shape, dtype=torch.int64, device=device)
    size = ctypes.c_size_t()
    call("dr_raster_workspace_size", ref(geo.struct), ctypes.byref(size))
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
    prev = None if previous is None else previous.contiguous()
    stream = _lib.stream(device)
    key = (device.index, geo.shape, geo.struct.num_tri, geo.struct.num_instances, prev is None)
    capturing = torch.cuda.is_current_stream_capturing()
    _order(geo, workspace, size.value, capturing)
    with _sizes_lock:
        sizes = _SIZES.get(key)
    if sizes is None and not capturing:
        host, arrived = _host_counts(device)
        call("dr_raster_visibility_start", ref(geo.struct), ptr(prev), ptr(keys), ptr(workspace),
             size.value, host.data_ptr(), stream)
        arrived.record(torch.cuda.current_stream(device))
        arrived.synchronize()
        found = [v & 0xFFFFFFFF for v in host.tolist()]
        counts = (ctypes.c_uint32 * 4)(found[0], found[1], _tile_grid(geo, found[2]), found[3])
        entries = torch.empty(max(found[1], 1), dtype=torch.int64, device=device)
        call("dr_raster_visibility_bin", ref(geo.struct), ptr(workspace), size.value,
             ptr(entries), counts, stream)
        call("dr_raster_visibility_tiles", ref(geo.struct), ptr(prev), ptr(keys),
             ptr(workspace), size.value, ptr(entries), counts, stream)
        _remember(key, _Sizes(found[1], found[2]))
        return keys
    if sizes is None:  # captured before any eager call of this shape: a generous guess
        capacity, groups = min(4 * geo.struct.num_instances + 4096, 0x7fffffff), 0
    else:
        with sizes.lock:
            if not capturing:  # no event may be queried while a stream is captured
                sizes.refresh()
            capacity = _entry_capacity(sizes.entries)
            groups = min(sizes.groups + sizes.groups // 8 + 8, 0xffffffff) if sizes.groups else 0
    entries = torch.empty(capacity, dtype=torch.int64, device=device)
    # The four passes of dr_raster_visibility, queued one call each (so that each can be timed
    # on its own): start, bin and tiles into the buffer, overflow when it was too small.
    spec = (ctypes.c_uint32 * 4)(0, capacity, _tile_grid(geo, groups), 0)

    def passes(readback):
        call("dr_raster_visibility_start", ref(geo.struct), ptr(prev), ptr(keys), ptr(workspace),
             size.value, ptr(readback), stream)
        call("dr_raster_visibility_bin", ref(geo.struct), ptr(workspace), size.value,
             ptr(entries), spec, stream)
        call("dr_raster_visibility_tiles", ref(geo.struct), ptr(prev), ptr(keys), ptr(workspace),
             size.value, ptr(entries), spec, stream)
        call("dr_raster_visibility_overflow", ref(geo.struct), ptr(prev), ptr(keys),
             ptr(workspace), size.value, capacity, stream)

    if sizes is None or capturing:
        passes(None)
        return keys
    with sizes.lock:
        readback = None if sizes.pending else sizes.counts
        passes(readback)
        if readback is not None:
            sizes.event.record(torch.cuda.current_stream(device))
            sizes.pending = True
    return keys


class _Resolve(torch.autograd.Function):
    """rast / rast_db from keys; gradients to pos (reference.py:69-114)."""

    @staticmethod
    def forward(ctx, pos, keys, geo, grad_db):
        batch, height, width = geo.shape
        rast = pos.new_empty(batch, height, width, 4)
        rast_db = pos.new_empty(batch, height, width, 4)
        call(_entry("dr_resolve_forward", pos), ref(geo.struct), ptr(keys), ptr(rast), ptr(rast_db),
             _stream(pos))
        ctx.geo = geo
        ctx.grad_db = grad_db
        ctx.save_for_backward(_saveable(pos), keys)
        if not grad_db:
            ctx.mark_non_differentiable(rast_db)
        # Outputs that no gradient reaches arrive as None, not as zeros to walk through.
        ctx.set_materialize_grads(False)
        return rast, rast_db

    @staticmethod
    @first_order("rasterize")
    def backward(ctx, grad_rast, grad_rast_db):
        pos, keys = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None
        geo = ctx.geo
        grad_pos = torch.zeros_like(pos, memory_format=torch.contiguous_format)
        use_db = ctx.grad_db and grad_rast_db is not None
        if grad_rast is None and not use_db:
            # Neither output carries a gradient (rast only fed antialias, say, which has none
            # for it): the positions' gradient through here is zero, as the reference's
            # resolve backward computes from zero gradients.
            return grad_pos, None, None, None
        if grad_rast is None:
            grad_rast = pos.new_zeros(*geo.shape, 4)
        grad_db = _dense(grad_rast_db) if use_db else None
        # The geometry points at the forward's tensors, which are still alive (saved).
        struct = _lib.RasterGeometry.from_buffer_copy(geo.struct)
        struct.pos = ptr(pos)
        call(_entry("dr_resolve_backward", pos), ref(struct), ptr(keys), ptr(grad_rast.contiguous()),
             ptr(grad_db), ptr(grad_pos), _stream(pos))
        return grad_pos, None, None, None


def _empty_layer(pos: Tensor, batch: int, resolution) -> tuple[Tensor, Tensor, Tensor]:
    empty = pos.new_zeros(batch, *resolution, 4)
    keys = torch.full((batch, *resolution), EMPTY_KEY, dtype=torch.int64, device=pos.device)
    return empty, empty.clone(), keys


def _single(geo: _Geometry, pos: Tensor, make) -> _Geometry:
    """The geometry visibility runs on: float32 positions (a float32 copy of float64 ones: as in
    the reference's GPU backend, visibility is float32 and only the resolve follows pos)."""
    return geo if pos.dtype == torch.float32 else make(pos.float())


def rasterize(pos: Tensor, tri: Tensor, resolution: tuple[int, int], grad_db: bool):
    """(reference: triton.py:14-18)"""
    rast, rast_db, _ = rasterize_layer(pos, tri, resolution, grad_db, None)
    return rast, rast_db


def rasterize_layer(pos: Tensor, tri: Tensor, resolution: tuple[int, int], grad_db: bool,
                    previous: Tensor | None):
    """One depth layer behind ``previous`` (the keys returned for the layer before) and its
    keys (reference: triton.py:21-40, reference.py:45-66)."""
    _real(("pos", pos))
    _require("tri", tri, torch.int32)
    _require("previous", previous, torch.int64)
    if tri.shape[0] == 0 or pos.shape[0] == 0:
        return _empty_layer(pos, pos.shape[0], resolution)
    pos, tri = pos.contiguous(), tri.contiguous()
    geo = _Geometry(pos, tri, resolution)
    keys = _visibility(_single(geo, pos, lambda p: _Geometry(p, tri, resolution)), previous)
    rast, rast_db = _Resolve.apply(pos, keys, geo, grad_db)
    return rast, rast_db, keys


# Device copies of range tables, by content: a range table drawn again (every DepthPeeler
# takes its own copy of ``ranges``) is copied to the device once, so that later calls, and a
# step captured in a HIP graph, make no host-to-device copy. A captured graph keeps the
# copies' addresses in its kernel arguments and no reference to them, so a copy used under
# capture is pinned: never evicted, for the life of the process.
_RANGE_COPIES: dict[tuple, list] = {}  # key -> [ranges, prefix, pinned]; order = recency
_RANGE_COPIES_KEPT = 16
_range_lock = threading.Lock()


def _range_tables(table: list[tuple[int, int]], prefix: list[int], device: torch.device,
                  capturing: bool | None = None) -> tuple[Tensor, Tensor]:
    if capturing is None:
        capturing = device.type == "cuda" and torch.cuda.is_current_stream_capturing()
    key = (device, tuple(table))
    with _range_lock:
        found = _RANGE_COPIES.pop(key, None)
        if found is not None:
            found[2] = found[2] or capturing
            _RANGE_COPIES[key] = found  # most recent now
            return found[0], found[1]
    copies = [torch.tensor(table, dtype=torch.int32).to(device, non_blocking=True),
              torch.tensor(prefix, dtype=torch.int64).to(device, non_blocking=True), capturing]
    with _range_lock:
        _RANGE_COPIES[key] = copies
        unpinned = [k for k, v in _RANGE_COPIES.items() if not v[2]]
        for old in unpinned[:max(0, len(_RANGE_COPIES) - _RANGE_COPIES_KEPT)]:
            del _RANGE_COPIES[old]  # least recent unpinned first
    return copies[0], copies[1]


def rasterize_ranges(pos: Tensor, tri: Tensor, resolution: tuple[int, int], grad_db: bool,
                     ranges: Tensor, previous: Tensor | None = None):
    """Range mode in one launch: image i draws ``tri[start_i : start_i + count_i]`` of the
    shared ``pos`` ([vertices, 4]); ids count from the start of ``tri``, as after the
    reference's join_ranges (ops.py:490-508). Returns ``(rast, rast_db, keys)``."""
    _real(("pos", pos))
    _require("tri", tri, torch.int32)
    _require("previous", previous, torch.int64)
    table = [(int(s), int(c)) for s, c in ranges.tolist()]
    batch = len(table)
    if batch == 0 or tri.shape[0] == 0:
        return _empty_layer(pos, batch, resolution)
    counts = [c for _, c in table]
    prefix = [0]
    for c in counts:
        prefix.append(prefix[-1] + c)
    if prefix[-1] == 0:
        return _empty_layer(pos, batch, resolution)
    pos, tri = pos.contiguous(), tri.contiguous()
    ranges_dev, prefix_dev = _range_tables(table, prefix, pos.device)

    def geometry(p):
        return _Geometry(p, tri, resolution, ranges=ranges_dev, range_prefix=prefix_dev,
                         batch=batch, num_instances=prefix[-1])

    geo = geometry(pos)
    keys = _visibility(_single(geo, pos, geometry), previous)
    rast, rast_db = _Resolve.apply(pos, keys, geo, grad_db)
    return rast, rast_db, keys


# ---------------------------------------------------------------------------------------------
# Interpolate
# ---------------------------------------------------------------------------------------------


def _interp_args(attr, rast, rast_db, tri, diff_dev, num_diff):
    batch, height, width, _ = rast.shape
    shared = attr.ndim == 2 or attr.shape[0] == 1
    return _lib.InterpolateArgs(
        attr=ptr(attr), attr_batch_stride=0 if shared else attr.shape[-2] * attr.shape[-1],
        num_vertices=attr.shape[-2], channels=attr.shape[-1], rast=ptr(rast),
        rast_db=ptr(rast_db), tri=ptr(tri), num_tri=tri.shape[0], batch=batch, height=height,
        width=width, num_diff=num_diff, diff=ptr(diff_dev))


_channel_lists: dict[tuple, Tensor] = {}


def _channel_list(channels: tuple[int, ...], device: torch.device) -> Tensor:
    """The channel list as a device int32 tensor, made once per list and device (a fresh
    host-to-device copy would wait for the stream before every call)."""
    key = (channels, device)
    found = _channel_lists.get(key)
    if found is None:
        found = torch.tensor(channels, dtype=torch.int32).to(device)
        _channel_lists[key] = found
    return found


class _Interpolate(torch.autograd.Function):
    """(reference: _triton_interpolate.py:185-254, reference.py:117-146)"""

    @staticmethod
    def forward(ctx, attr, rast, rast_db, tri, diff):
        attr, rast, tri = attr.contiguous(), rast.contiguous(), tri.contiguous()
        rast_db = _dense(rast_db) if diff else None
        batch, height, width, _ = rast.shape
        diff_dev = _channel_list(diff, rast.device) if diff else None
        out = attr.new_empty(batch, height, width, attr.shape[-1])
        out_da = attr.new_empty(batch, height, width, 2 * len(diff))
        args = _interp_args(attr, rast, rast_db, tri, diff_dev, len(diff))
        call(_entry("dr_interpolate_forward", attr), ref(args), ptr(out), ptr(out_da) if diff else None,
             _stream(rast))
        ctx.diff = diff
        ctx.save_for_backward(_saveable(attr), _saveable(rast), _saveable(rast_db), tri,
                              diff_dev)
        if not diff:
            ctx.mark_non_differentiable(out_da)
        ctx.set_materialize_grads(False)  # unreached outputs arrive as None
        return out, out_da

    @staticmethod
    @first_order("interpolate")
    def backward(ctx, grad_out, grad_out_da):
        attr, rast, rast_db, tri, diff_dev = ctx.saved_tensors
        need_attr, need_rast, need_db = ctx.needs_input_grad[:3]
        if not (need_attr or need_rast or need_db):
            return None, None, None, None, None
        diff = ctx.diff
        if grad_out is None and (grad_out_da is None or not diff):
            # No gradient reaches either output: zero for the attributes, and none to pass on
            # to rast (whose own backward then has nothing to add).
            return torch.zeros_like(attr) if need_attr else None, None, None, None, None
        if grad_out is None:
            grad_out = attr.new_zeros(*rast.shape[:3], attr.shape[-1])
        grad_out = grad_out.contiguous()
        grad_da = _dense(grad_out_da) if diff else None
        grad_attr = torch.zeros_like(attr) if need_attr else None
        grad_rast = torch.empty_like(rast) if need_rast else None
        grad_db = torch.empty_like(rast_db) if (need_db and diff) else None
        args = _interp_args(attr, rast, rast_db, tri, diff_dev, len(diff))
        call(_entry("dr_interpolate_backward", attr), ref(args), ptr(grad_out), ptr(grad_da), ptr(grad_attr),
             ptr(grad_rast), ptr(grad_db), _stream(rast))
        return grad_attr, grad_rast, grad_db, None, None


def interpolate(attr: Tensor, rast: Tensor, tri: Tensor, rast_db: Tensor | None,
                diff_attrs: Sequence[int]):
    """(reference: triton.py:50-56)"""
    _real(("attr", attr), ("rast", rast), ("rast_db", rast_db))
    _require("tri", tri, torch.int32)
    return _Interpolate.apply(attr, rast, rast_db, tri, tuple(int(c) for c in diff_attrs))


# ---------------------------------------------------------------------------------------------
# Texture
# ---------------------------------------------------------------------------------------------


def _chain_sizes(height: int, width: int, max_mip_level: int | None) -> list[tuple[int, int]]:
    """Sizes of the box-filtered chain: halve rounding up until 1x1 (reference.py:433-446)."""
    sizes = [(height, width)]
    while max(sizes[-1]) > 1 and (max_mip_level is None or len(sizes) <= max_mip_level):
        h, w = sizes[-1]
        sizes.append(((h + 1) // 2, (w + 1) // 2))
    return sizes


def _tables(sizes, faces):
    heights = tuple(h for h, _ in sizes)
    widths = tuple(w for _, w in sizes)
    offsets, total = [], 0
    for h, w in sizes:
        offsets.append(total)
        total += faces * h * w
    return heights, widths, tuple(offsets), total


def _level_arrays(heights, widths, offsets):
    n = len(heights)
    return ((ctypes.c_int32 * n)(*heights), (ctypes.c_int32 * n)(*widths),
            (ctypes.c_int64 * n)(*offsets))


def _build_chain(tex: Tensor, tables) -> tuple[Tensor, tuple]:
    """The packed buffer [tex_batch, texels, channels] of tex and its box-filtered levels
    (reference.py:433-519); level 0 is copied in by the pass that reads it."""
    tex = tex.contiguous()
    faces = 6 if tex.ndim == 5 else 1
    heights, widths, offsets = tables
    tex_batch, channels = tex.shape[0], tex.shape[-1]
    total = offsets[-1] + faces * heights[-1] * widths[-1]
    packed = tex.new_empty(tex_batch, total, channels)
    call(_entry("dr_mip_build", tex), ptr(packed), ptr(tex), tex_batch, channels, total, faces,
         len(heights),
         *_level_arrays(heights, widths, offsets), _stream(tex))
    return packed, (tex.shape, faces, tables, total, faces * heights[0] * widths[0])


def _fold_chain(grad: Tensor, meta) -> Tensor:
    """Adjoint of _build_chain, in place on the packed gradient: returns the gradient of tex (a
    view of level 0)."""
    shape, faces, (heights, widths, offsets), total, base = meta
    call(_entry("dr_mip_build_backward", grad), ptr(grad), shape[0], shape[-1], total, faces,
         len(heights),
         *_level_arrays(heights, widths, offsets), _stream(grad))
    return grad[:, :base].reshape(shape)


class _MipChain(torch.autograd.Function):
    """The packed chain of tex as a differentiable result (texture_construct_mip)."""

    @staticmethod
    def forward(ctx, tex, tables):
        packed, ctx.meta = _build_chain(tex, tables)
        return packed

    @staticmethod
    @first_order("texture")
    def backward(ctx, grad_packed):
        # The incoming gradient may be shared with other consumers: fold a copy.
        return _fold_chain(grad_packed.contiguous().clone(), ctx.meta), None


def _mip_chain(tex: Tensor, max_mip_level: int | None):
    faces = 6 if tex.ndim == 5 else 1
    heights, widths, offsets, _ = _tables(_chain_sizes(tex.shape[-3], tex.shape[-2],
                                                       max_mip_level), faces)
    tables = (heights, widths, offsets)
    return _MipChain.apply(tex, tables), tables


def _sample(ctx, texels, uv, uv_da, bias, tables, filter_mode, boundary_mode):
    texels, uv = texels.contiguous(), uv.contiguous()
    uv_da, bias = _dense(uv_da), _dense(bias)
    batch, height, width = uv.shape[:3]
    out = texels.new_empty(batch, height, width, texels.shape[-1])
    args = _texture_args(texels, uv, uv_da, bias, tables, filter_mode, boundary_mode)
    call(_entry("dr_texture_forward", texels), ref(args), ptr(out), _stream(uv))
    ctx.meta = (tables, filter_mode, boundary_mode)
    ctx.save_for_backward(_saveable(texels), _saveable(uv), _saveable(uv_da), _saveable(bias))
    return out


def _sample_backward(ctx, grad_out, need_texels):
    """(grad_texels, grad_uv, grad_uv_da, grad_bias) of a lookup; grad_texels in the packed
    layout, accumulated from zero."""
    texels, uv, uv_da, bias = ctx.saved_tensors
    tables, filter_mode, boundary_mode = ctx.meta
    need_uv, need_da, need_bias = ctx.needs_input_grad[1:4]
    grad_texels = torch.zeros_like(texels) if need_texels else None
    coord_grad = filter_mode != "nearest"
    grad_uv = torch.empty_like(uv) if (need_uv and coord_grad) else None
    grad_da = torch.empty_like(uv_da) if (need_da and uv_da is not None) else None
    grad_bias = torch.empty_like(bias) if (need_bias and bias is not None) else None
    if grad_texels is None and grad_uv is None and grad_da is None and grad_bias is None:
        return None, None, None, None
    args = _texture_args(texels, uv, uv_da, bias, tables, filter_mode, boundary_mode)
    call(_entry("dr_texture_backward", texels), ref(args), ptr(grad_out.contiguous()),
         ptr(grad_texels),
         ptr(grad_uv), ptr(grad_da), ptr(grad_bias), _stream(uv))
    return grad_texels, grad_uv, grad_da, grad_bias


class _Texture(torch.autograd.Function):
    """A lookup in packed texels (reference: _triton_texture.py:429-508, reference.py:149-194,
    _cube.py)."""

    @staticmethod
    def forward(ctx, texels, uv, uv_da, bias, tables, filter_mode, boundary_mode):
        return _sample(ctx, texels, uv, uv_da, bias, tables, filter_mode, boundary_mode)

    @staticmethod
    @first_order("texture")
    def backward(ctx, grad_out):
        return (*_sample_backward(ctx, grad_out, ctx.needs_input_grad[0]), None, None, None)


class _ChainTexture(torch.autograd.Function):
    """A lookup with the mip chain of tex built in the call (mip=None): one node, so that the
    backward pass folds the packed gradient it made itself, in place."""

    @staticmethod
    def forward(ctx, tex, uv, uv_da, bias, tables, filter_mode, boundary_mode):
        packed, chain = _build_chain(tex, tables)
        out = _sample(ctx, packed, uv, uv_da, bias, tables, filter_mode, boundary_mode)
        ctx.chain = chain
        return out

    @staticmethod
    @first_order("texture")
    def backward(ctx, grad_out):
        grads = _sample_backward(ctx, grad_out, ctx.needs_input_grad[0])
        grad_tex = None if grads[0] is None else _fold_chain(grads[0], ctx.chain)
        return grad_tex, *grads[1:], None, None, None


def _texture_args(texels, uv, uv_da, bias, tables, filter_mode, boundary_mode):
    heights, widths, offsets = tables
    n = len(heights)
    if n > _lib.MAX_LEVELS:
        raise ValueError(f"at most {_lib.MAX_LEVELS} mip levels are supported, got {n}.")
    args = _lib.TextureArgs()
    args.texels = ptr(texels)
    args.tex_batch = texels.shape[0]
    args.channels = texels.shape[-1]
    args.num_texels = texels.shape[1]
    args.num_levels = n
    args.faces = 6 if boundary_mode == "cube" else 1
    for k in range(n):
        args.level_height[k] = heights[k]
        args.level_width[k] = widths[k]
        args.level_offset[k] = offsets[k]
    args.uv = ptr(uv)
    args.uv_da = ptr(uv_da)
    args.bias = ptr(bias)
    args.batch, args.height, args.width = uv.shape[:3]
    args.filter = FILTERS[filter_mode]
    args.boundary = BOUNDARIES[boundary_mode]
    return args


def pack(levels: Sequence[Tensor]):
    """Join ``tex`` and mip levels into one buffer [tex_batch, texels, channels] and its size
    tables (reference.py:504-519). A level shared across the batch is repeated when the base
    level is not. The tables are tuples of Python ints."""
    batch, channels = levels[0].shape[0], levels[0].shape[-1]
    faces = 6 if levels[0].ndim == 5 else 1
    sizes = [(level.shape[-3], level.shape[-2]) for level in levels]
    heights, widths, offsets, _ = _tables(sizes, faces)
    parts = [level.expand(batch, *level.shape[1:]).reshape(batch, -1, channels)
             for level in levels]
    texels = parts[0] if len(parts) == 1 else torch.cat(parts, 1)
    return texels, heights, widths, offsets


def texture_construct_mip(tex: Tensor, max_mip_level: int | None) -> list[Tensor]:
    """Mip levels 1 and up of ``tex`` as views of one packed buffer, differentiable with
    respect to ``tex`` (reference.py:197-199)."""
    _real(("tex", tex))
    packed, (heights, widths, offsets) = _mip_chain(tex, max_mip_level)
    faces = 6 if tex.ndim == 5 else 1
    levels = []
    for k in range(1, len(heights)):
        count = faces * heights[k] * widths[k]
        shape = (tex.shape[0], *((6,) if faces == 6 else ()), heights[k], widths[k], tex.shape[-1])
        levels.append(packed[:, offsets[k]:offsets[k] + count].reshape(shape))
    return levels


def texture(tex: Tensor, uv: Tensor, uv_da: Tensor | None, filter_mode: str, boundary_mode: str,
            max_mip_level: int | None, mip_level_bias: Tensor | None = None,
            mip: Sequence[Tensor] | None = None, packed=None):
    """(reference: triton.py:59-79, reference.py:149-194)"""
    _real(("tex", tex), ("uv", uv), ("uv_da", uv_da), ("mip_level_bias", mip_level_bias),
          *((f"mip[{k}]", m) for k, m in enumerate(mip or ())),
          ("packed texels", None if packed is None else packed[0]))
    mipmapped = "mipmap" in filter_mode
    if not mipmapped:
        faces = 6 if boundary_mode == "cube" else 1
        h, w = tex.shape[-3], tex.shape[-2]
        texels = tex.reshape(tex.shape[0], faces * h * w, tex.shape[-1])
        tables = ((h,), (w,), (0,))
        return _Texture.apply(texels, uv, None, None, tables, filter_mode, boundary_mode)
    count = None if max_mip_level is None else max_mip_level + 1
    if packed is not None:
        texels, heights, widths, offsets = packed
        tables = (tuple(heights[:count]), tuple(widths[:count]), tuple(offsets[:count]))
    elif mip is not None:
        levels = [tex, *mip][:count]
        texels, heights, widths, offsets = pack(levels)
        tables = (heights, widths, offsets)
    else:
        faces = 6 if tex.ndim == 5 else 1
        heights, widths, offsets, _ = _tables(_chain_sizes(tex.shape[-3], tex.shape[-2],
                                                           max_mip_level), faces)
        return _ChainTexture.apply(tex, uv, uv_da, mip_level_bias, (heights, widths, offsets),
                                   filter_mode, boundary_mode)
    return _Texture.apply(texels, uv, uv_da, mip_level_bias, tables, filter_mode, boundary_mode)


# ---------------------------------------------------------------------------------------------
# Antialias
# ---------------------------------------------------------------------------------------------


def edge_neighbours(tri: Tensor) -> Tensor:
    """Partner of each edge, int32 [triangles, 3], -1 when unshared or non-manifold
    (reference.py:768-787), from a GPU hash table."""
    _require("tri", tri, torch.int32)
    tri = tri.contiguous()
    out = torch.empty(tri.shape[0], 3, dtype=torch.int32, device=tri.device)
    if tri.shape[0] == 0:
        return out
    size = ctypes.c_size_t()
    call("dr_edge_hash_workspace_size", tri.shape[0], ctypes.byref(size))
    workspace = torch.empty(size.value, dtype=torch.uint8, device=tri.device)
    call("dr_edge_neighbours", ptr(tri), tri.shape[0], ptr(workspace), size.value, ptr(out),
         _stream(tri))
    return out


def silhouette_mask(pos: Tensor, tri: Tensor, neighbours: Tensor,
                    rast: Tensor | None = None) -> Tensor:
    """Silhouette bits per (pos batch, triangle), uint8 (reference.py:790-814). Given rast,
    only for the triangles it shows (antialiasing reads no others); 0 elsewhere."""
    pos3 = pos if pos.ndim == 3 else pos[None]
    pos3 = pos3.contiguous()
    mask = torch.empty(pos3.shape[0], tri.shape[0], dtype=torch.uint8, device=pos.device)
    batch, height, width = (0, 1, 1) if rast is None else rast.shape[:3]
    if pos3.dtype == torch.float64:  # every triangle's bits, from the float64 positions
        call("dr_silhouette_mask_f64", ptr(pos3), pos3.shape[1] * 4, pos3.shape[0], ptr(tri),
             tri.shape[0], ptr(neighbours), ptr(mask), _stream(pos))
        return mask
    if rast is not None:
        rast = rast.contiguous()
    call("dr_silhouette_mask", ptr(pos3), pos3.shape[1] * 4, pos3.shape[0], ptr(tri),
         tri.shape[0], ptr(neighbours), ptr(rast), batch, height, width, ptr(mask), _stream(pos))
    return mask


def _aa_args(color, rast, pos, tri, mask, boost):
    batch, height, width, channels = color.shape
    per_view = pos.ndim == 3 and pos.shape[0] > 1
    return _lib.AntialiasArgs(
        color=ptr(color), channels=channels, batch=batch, height=height, width=width,
        rast=ptr(rast), pos=ptr(pos), pos_batch_stride=pos.shape[-2] * 4 if per_view else 0,
        tri=ptr(tri), num_tri=tri.shape[0], silhouette=ptr(mask),
        silhouette_batch_stride=tri.shape[0] if per_view else 0, boost=boost)


class _Antialias(torch.autograd.Function):
    """(reference: _triton_antialias.py:271-320, reference.py:202-265)

    The forward pass keeps the per-pixel pair records (crossing and owner bits) for the
    backward pass, which then needs no crossing search of its own."""

    @staticmethod
    def forward(ctx, color, rast, pos, tri, mask, boost):
        color, rast, pos, tri = (t.contiguous() for t in (color, rast, pos, tri))
        out = torch.empty_like(color)
        args = _aa_args(color, rast, pos, tri, mask, boost)
        size = ctypes.c_size_t()
        call(_entry("dr_antialias_workspace_size", color), ref(args), ctypes.byref(size))
        pairs = torch.empty(max(size.value, 1), dtype=torch.uint8, device=color.device)
        call(_entry("dr_antialias_forward", color), ref(args), ptr(pairs), size.value, ptr(out),
             _stream(color))
        ctx.boost = boost
        ctx.save_for_backward(_saveable(color), _saveable(rast), _saveable(pos), tri, mask, pairs)
        return out

    @staticmethod
    @first_order("antialias")
    def backward(ctx, grad_out):
        color, rast, pos, tri, mask, pairs = ctx.saved_tensors
        need_color, _, need_pos = ctx.needs_input_grad[:3]
        grad_color = torch.empty_like(color) if need_color else None
        grad_pos = torch.zeros_like(pos) if need_pos else None
        if grad_color is None and grad_pos is None:
            return None, None, None, None, None, None
        args = _aa_args(color, rast, pos, tri, mask, ctx.boost)
        call(_entry("dr_antialias_backward", color), ref(args), ptr(pairs), pairs.numel(),
             ptr(grad_out.contiguous()), ptr(grad_color), ptr(grad_pos), _stream(color))
        return grad_color, None, grad_pos, None, None, None


def antialias(color: Tensor, rast: Tensor, pos: Tensor, tri: Tensor, pos_gradient_boost: float,
              neighbours: Tensor | None = None) -> Tensor:
    """(reference: triton.py:82-92, reference.py:202-265)"""
    _real(("color", color), ("rast", rast), ("pos", pos))
    _require("tri", tri, torch.int32)
    if tri.shape[0] == 0:
        return color.clone()
    tri = tri.contiguous()
    if neighbours is None:
        neighbours = edge_neighbours(tri)
    neighbours = neighbours.to(torch.int32).contiguous()
    # Antialiasing reads the silhouette bits of the triangles rast shows only. Finding those
    # takes a pass over rast (16 bytes per pixel); classifying a triangle, some 100 bytes of
    # gathers: when the (pos batch, triangle) pairs are fewer than a sixth of the pixels, all
    # are classified and rast is not read (range mode, small meshes at large images).
    pairs = (pos.shape[0] if pos.ndim == 3 else 1) * tri.shape[0]
    shown = rast.detach() if 6 * pairs > rast.shape[0] * rast.shape[1] * rast.shape[2] else None
    with torch.no_grad():
        mask = silhouette_mask(pos.detach(), tri, neighbours, shown)
    return _Antialias.apply(color, rast, pos, tri, mask, float(pos_gradient_boost))
