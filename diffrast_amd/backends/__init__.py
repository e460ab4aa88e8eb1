"""Backend selection (reference: src/diffrast/backends/__init__.py:1-66).

The backend modules implement the four ops on validated inputs. This package has one: ``hip``,
the MI355X kernels. ``"triton"``, the name of the reference's GPU backend, selects it too, so
that code written for the reference keeps running. The reference's pure-PyTorch backend is not
part of this package; asking for it raises.
"""

from __future__ import annotations

import importlib
import os
from types import ModuleType

import torch

BACKENDS = ("hip",)
OPS = ("rasterize", "interpolate", "texture", "antialias")
# Names the reference accepts that map onto a backend here.
ALIASES = {"triton": "hip"}

_selected = os.environ.get("DIFFRAST_BACKEND", "auto")


def set_backend(name: str) -> None:
    """Select the backend used by all ops.

    Args:
        name: ``"hip"``, ``"auto"`` (the default) or ``"triton"`` (an alias of ``"hip"``). The
            initial value can also be set with the ``DIFFRAST_BACKEND`` environment variable.
    """
    global _selected
    _check_name(name)
    _selected = name


def get_backend_name(device: torch.device | str, op: str) -> str:
    """Return the name of the backend that ``op`` will run on for tensors on ``device``."""
    _check_name(_selected)
    if op not in OPS:
        raise ValueError(f"Unknown op {op!r}; expected one of {OPS}.")
    device = torch.device(device)
    if not _hip_usable(device):
        raise RuntimeError(
            "diffrast_amd runs on ROCm GPUs only (its kernels are HIP code for MI355X); got "
            f"device {str(device)!r}. Move the tensors to a 'cuda' device."
        )
    return "hip"


def get_backend(device: torch.device | str, op: str) -> ModuleType:
    """Return the backend module that ``op`` will run on for tensors on ``device``."""
    return _load(get_backend_name(device, op))


_loaded: dict[str, ModuleType] = {}


def _load(name: str) -> ModuleType:
    # Cached: import_module takes the import lock on every call (~13 us), once per op call.
    module = _loaded.get(name)
    if module is None:
        module = importlib.import_module(f"diffrast_amd.backends.{ALIASES.get(name, name)}")
        _loaded[name] = module
    return module


def _check_name(name: str) -> None:
    if name == "reference":
        raise ValueError(
            "The pure-PyTorch 'reference' backend is not part of diffrast_amd; use 'hip' or "
            "'auto'."
        )
    if name not in ("auto", *BACKENDS, *ALIASES):
        options = ", ".join(repr(n) for n in ("auto", *BACKENDS, *ALIASES))
        raise ValueError(f"Unknown backend {name!r}; expected one of {options}.")


def _hip_usable(device: torch.device) -> bool:
    return device.type == "cuda" and torch.version.hip is not None
