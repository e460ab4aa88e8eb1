"""ctypes binding of libdiffrast_hip.so (declared in include/diffrast_hip.h).

The library is loaded on first use from the package directory, where
``python -m diffrast_amd._build`` puts it. There is no fallback: if the library is missing or
was built for another ABI, every op raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent.parent / "libdiffrast_hip.so"
ABI_VERSION = 15
MAX_LEVELS = 32

c_float_p = ctypes.POINTER(ctypes.c_float)
c_void_p = ctypes.c_void_p


class RasterGeometry(ctypes.Structure):
    _fields_ = [
        ("pos", c_void_p),
        ("pos_batch_stride", ctypes.c_int64),
        ("tri", c_void_p),
        ("num_tri", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("ranges", c_void_p),
        ("range_prefix", c_void_p),
        ("num_instances", ctypes.c_int64),
        ("num_vertices", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("order", c_void_p),
    ]


class InterpolateArgs(ctypes.Structure):
    _fields_ = [
        ("attr", c_void_p),
        ("attr_batch_stride", ctypes.c_int64),
        ("num_vertices", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("rast", c_void_p),
        ("rast_db", c_void_p),
        ("tri", c_void_p),
        ("num_tri", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("num_diff", ctypes.c_int32),
        ("diff", c_void_p),
    ]


class TextureArgs(ctypes.Structure):
    _fields_ = [
        ("texels", c_void_p),
        ("tex_batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("num_texels", ctypes.c_int64),
        ("num_levels", ctypes.c_int32),
        ("faces", ctypes.c_int32),
        ("level_height", ctypes.c_int32 * MAX_LEVELS),
        ("level_width", ctypes.c_int32 * MAX_LEVELS),
        ("level_offset", ctypes.c_int64 * MAX_LEVELS),
        ("uv", c_void_p),
        ("uv_da", c_void_p),
        ("bias", c_void_p),
        ("batch", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("filter", ctypes.c_int32),
        ("boundary", ctypes.c_int32),
    ]


class AntialiasArgs(ctypes.Structure):
    _fields_ = [
        ("color", c_void_p),
        ("channels", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("rast", c_void_p),
        ("pos", c_void_p),
        ("pos_batch_stride", ctypes.c_int64),
        ("tri", c_void_p),
        ("num_tri", ctypes.c_int32),
        ("silhouette", c_void_p),
        ("silhouette_batch_stride", ctypes.c_int64),
        ("boost", ctypes.c_float),
    ]


STRUCTS = (RasterGeometry, InterpolateArgs, TextureArgs, AntialiasArgs)

# Entry points and their argument types (return type is int for all).
_P = c_void_p
_SIGNATURES = {
    "dr_error_string": ([ctypes.c_int], ctypes.c_char_p),
    "dr_abi_version": ([], ctypes.c_int),
    "dr_struct_size": ([ctypes.c_int], ctypes.c_int),
    "dr_raster_workspace_size": ([_P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "dr_raster_order_size": ([_P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "dr_raster_order": ([_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P], ctypes.c_int),
    "dr_raster_visibility_begin": (
        [_P, _P, _P, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint32), _P], ctypes.c_int),
    "dr_raster_visibility_start": ([_P, _P, _P, _P, ctypes.c_size_t, _P, _P], ctypes.c_int),
    "dr_raster_visibility_bin": (
        [_P, _P, ctypes.c_size_t, _P, ctypes.POINTER(ctypes.c_uint32), _P], ctypes.c_int),
    "dr_raster_visibility_tiles": (
        [_P, _P, _P, _P, ctypes.c_size_t, _P, ctypes.POINTER(ctypes.c_uint32), _P], ctypes.c_int),
    "dr_raster_visibility_overflow": ([_P, _P, _P, _P, ctypes.c_size_t, ctypes.c_uint32, _P],
                                      ctypes.c_int),
    "dr_raster_visibility": ([_P, _P, _P, _P, ctypes.c_size_t, _P, ctypes.c_uint32,
                              ctypes.c_uint32, _P, _P], ctypes.c_int),
    "dr_raster_visibility_static": ([_P, _P, _P, _P], ctypes.c_int),
    "dr_resolve_forward": ([_P, _P, _P, _P, _P], ctypes.c_int),
    "dr_resolve_backward": ([_P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_interpolate_forward": ([_P, _P, _P, _P], ctypes.c_int),
    "dr_interpolate_backward": ([_P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_texture_forward": ([_P, _P, _P], ctypes.c_int),
    "dr_texture_backward": ([_P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_mip_build": ([_P, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                      ctypes.c_int32, _P, _P, _P, _P], ctypes.c_int),
    "dr_mip_build_backward": ([_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                               ctypes.c_int32, ctypes.c_int32, _P, _P, _P, _P], ctypes.c_int),
    "dr_edge_hash_workspace_size": ([ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)],
                                    ctypes.c_int),
    "dr_edge_neighbours": ([_P, ctypes.c_int32, _P, ctypes.c_size_t, _P, _P], ctypes.c_int),
    "dr_silhouette_mask": ([_P, ctypes.c_int64, ctypes.c_int32, _P, ctypes.c_int32, _P, _P,
                            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _P], ctypes.c_int),
    "dr_antialias_workspace_size": ([_P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "dr_antialias_forward": ([_P, _P, ctypes.c_size_t, _P, _P], ctypes.c_int),
    "dr_antialias_backward": ([_P, _P, ctypes.c_size_t, _P, _P, _P, _P], ctypes.c_int),
    "dr_resolve_forward_f64": ([_P, _P, _P, _P, _P], ctypes.c_int),
    "dr_resolve_backward_f64": ([_P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_interpolate_forward_f64": ([_P, _P, _P, _P], ctypes.c_int),
    "dr_interpolate_backward_f64": ([_P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_texture_forward_f64": ([_P, _P, _P], ctypes.c_int),
    "dr_texture_backward_f64": ([_P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "dr_mip_build_f64": ([_P, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                          ctypes.c_int32, ctypes.c_int32, _P, _P, _P, _P], ctypes.c_int),
    "dr_mip_build_backward_f64": ([_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_int32, ctypes.c_int32, _P, _P, _P, _P],
                                  ctypes.c_int),
    "dr_silhouette_mask_f64": ([_P, ctypes.c_int64, ctypes.c_int32, _P, ctypes.c_int32, _P, _P,
                                _P], ctypes.c_int),
    "dr_antialias_workspace_size_f64": ([_P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "dr_antialias_forward_f64": ([_P, _P, ctypes.c_size_t, _P, _P], ctypes.c_int),
    "dr_antialias_backward_f64": ([_P, _P, ctypes.c_size_t, _P, _P, _P, _P], ctypes.c_int),
}
EXPORTS = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """The loaded library, checked against this binding's ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY.exists():
            raise RuntimeError(
                f"{LIBRARY} is missing: the HIP kernels have not been built. Run "
                "'python -m diffrast_amd._build' (hipcc with gfx950 support is required)."
            )
        lib = ctypes.CDLL(str(LIBRARY))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.dr_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{LIBRARY} has ABI {lib.dr_abi_version()}, expected {ABI_VERSION}; rebuild it."
            )
        for index, struct in enumerate(STRUCTS):
            if lib.dr_struct_size(index) != ctypes.sizeof(struct):
                raise RuntimeError(
                    f"{struct.__name__} is {ctypes.sizeof(struct)} bytes here but "
                    f"{lib.dr_struct_size(index)} in {LIBRARY}; rebuild it."
                )
        _lib = lib
    return _lib


def check(code: int, what: str) -> None:
    if code != 0:
        message = load().dr_error_string(code).decode()
        raise RuntimeError(f"{what} failed: {message} (code {code}).")


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise ``RuntimeError`` on a nonzero status."""
    check(getattr(load(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> int:
    """The handle of the device's current stream (the raw query where torch has it: building a
    Stream object per call costs several microseconds)."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def ref(struct: ctypes.Structure):
    return ctypes.byref(struct)
