"""Run code written for nvdiffrast unchanged: ``import nvdiffrast.torch`` can resolve to this
package (the reference's src/diffrast/compat.py API: ``install_as_nvdiffrast(force=False)`` and
``uninstall_as_nvdiffrast()``, with the same refusals and messages)."""

from __future__ import annotations

import importlib
import importlib.util
import sys
from types import ModuleType

from diffrast_amd import log

# Aliases registered under nvdiffrast's names, and the package each stands for.
_ALIASES = (("nvdiffrast", "diffrast_amd"), ("nvdiffrast.torch", "diffrast_amd.torch"))

# Modules a forced install took the place of, restored by the uninstall.
_displaced: dict[str, ModuleType] = {}


def _ours() -> dict[str, ModuleType]:
    return {alias: importlib.import_module(target) for alias, target in _ALIASES}


def _findable(name: str) -> bool:
    try:
        return importlib.util.find_spec(name) is not None
    except (ImportError, ValueError):
        return False


def install_as_nvdiffrast(force: bool = False) -> None:
    """Register this package and its ``torch`` module as ``nvdiffrast`` and ``nvdiffrast.torch``
    in ``sys.modules``, so that later imports of nvdiffrast get them. Repeating the call does
    nothing; :func:`uninstall_as_nvdiffrast` undoes it.

    Args:
        force: Take the place of a real nvdiffrast that is imported or installed, which
            otherwise raises ``RuntimeError``.
    """
    ours = _ours()
    foreign = {alias: sys.modules[alias] for alias in ours
               if sys.modules.get(alias) not in (None, ours[alias])}
    if not foreign and all(sys.modules.get(alias) is module for alias, module in ours.items()):
        return  # already in place
    if not force:
        if foreign:
            raise RuntimeError(
                f"{next(iter(foreign))} is already imported; pass force=True to replace it "
                "with diffrast."
            )
        if "nvdiffrast" not in sys.modules and _findable("nvdiffrast"):
            raise RuntimeError(
                "An nvdiffrast package is installed; pass force=True to use diffrast in its place."
            )
    if foreign:
        log.warn("Replacing the imported nvdiffrast with diffrast; modules that imported it "
                 "earlier keep using it.", stacklevel=2)
        _displaced.update(foreign)
    sys.modules.update(ours)


def uninstall_as_nvdiffrast() -> None:
    """Remove the aliases of :func:`install_as_nvdiffrast` and put back what they replaced."""
    for alias, module in _ours().items():
        before = _displaced.pop(alias, None)
        if sys.modules.get(alias) is not module:
            continue
        if before is None:
            del sys.modules[alias]
        else:
            sys.modules[alias] = before
