"""``import diffrast`` for code written against the reference package: this is diffrast_amd.

The submodules a user may import by name (``diffrast.ops``, ``diffrast.torch`` and the rest)
are the ones of diffrast_amd.
"""

import sys as _sys

import diffrast_amd as _impl
from diffrast_amd import *  # noqa: F403
from diffrast_amd import __all__, __version__  # noqa: F401

for _name in ("ops", "context", "peeling", "topology", "backends", "compat", "log", "torch",
              "_cache"):
    _module = __import__(f"diffrast_amd.{_name}", fromlist=["_"])
    _sys.modules[f"{__name__}.{_name}"] = _module
    setattr(_sys.modules[__name__], _name, _module)
del _impl
