"""diffrast for MI355X: differentiable mesh rasterization on hand-written HIP kernels.

The public API of diffrast (rasterize, interpolate, texture, antialias, DepthPeeler, range
mode, cube maps, mip stacks and the nvdiffrast-compatible names), running on gfx950 kernels
loaded from libdiffrast_hip.so.
"""

from diffrast_amd.backends import get_backend_name, set_backend
from diffrast_amd.compat import install_as_nvdiffrast, uninstall_as_nvdiffrast
from diffrast_amd.context import RasterizeContext, RasterizeCudaContext, RasterizeGLContext
from diffrast_amd.log import get_log_level, set_log_level
from diffrast_amd.ops import (
    MipStack,
    antialias,
    antialias_construct_topology_hash,
    interpolate,
    rasterize,
    texture,
    texture_construct_mip,
)
from diffrast_amd.peeling import DepthPeeler
from diffrast_amd.topology import TopologyHash

__version__ = "0.1.0.dev0"

__all__ = [
    "DepthPeeler",
    "MipStack",
    "RasterizeContext",
    "RasterizeCudaContext",
    "RasterizeGLContext",
    "TopologyHash",
    "__version__",
    "antialias",
    "antialias_construct_topology_hash",
    "get_backend_name",
    "get_log_level",
    "install_as_nvdiffrast",
    "interpolate",
    "rasterize",
    "set_backend",
    "set_log_level",
    "texture",
    "texture_construct_mip",
    "uninstall_as_nvdiffrast",
]
