"""Run code written for nvdiffrast unchanged (reference: compat.py:1-74)."""

from __future__ import annotations

import importlib
import importlib.util
import sys
from types import ModuleType

from diffrast_amd import log

_displaced: dict[str, ModuleType] = {}


def install_as_nvdiffrast(force: bool = False) -> None:
    """Make ``import nvdiffrast.torch as dr`` resolve to this package in this process.

    Registers the package and its ``torch`` module in ``sys.modules`` as ``nvdiffrast`` and
    ``nvdiffrast.torch``. Calling it again does nothing; :func:`uninstall_as_nvdiffrast` undoes
    it.

    Args:
        force: Replace a real nvdiffrast that is installed or imported; otherwise that raises
            ``RuntimeError``.
    """
    ours = _modules()
    current = {name: sys.modules.get(name) for name in ours}
    if all(current[name] is module for name, module in ours.items()):
        return
    imported = [name for name, module in ours.items() if current[name] not in (None, module)]
    if not force:
        if imported:
            raise RuntimeError(
                f"{imported[0]} is already imported; pass force=True to replace it with diffrast."
            )
        if current["nvdiffrast"] is None and _is_installed("nvdiffrast"):
            raise RuntimeError(
                "An nvdiffrast package is installed; pass force=True to use diffrast in its place."
            )
    if imported:
        log.warn(
            "Replacing the imported nvdiffrast with diffrast; modules that imported it "
            "earlier keep using it.",
            stacklevel=2,
        )
    for name, module in ours.items():
        if name in imported:
            _displaced[name] = current[name]
        sys.modules[name] = module


def uninstall_as_nvdiffrast() -> None:
    """Undo :func:`install_as_nvdiffrast`, restoring modules it replaced."""
    for name, module in _modules().items():
        previous = _displaced.pop(name, None)
        if sys.modules.get(name) is module:
            del sys.modules[name]
            if previous is not None:
                sys.modules[name] = previous


def _modules() -> dict[str, ModuleType]:
    return {
        "nvdiffrast": importlib.import_module("diffrast_amd"),
        "nvdiffrast.torch": importlib.import_module("diffrast_amd.torch"),
    }


def _is_installed(name: str) -> bool:
    try:
        return importlib.util.find_spec(name) is not None
    except (ImportError, ValueError):
        return False
