"""The public API under nvdiffrast's module path: ``import diffrast_amd.torch as dr``.

Inside this package the name ``torch`` refers to this module only; ``import torch`` elsewhere is
PyTorch, since imports are absolute (reference: torch.py:1-19).
"""

if __name__ == "torch":
    raise ImportError(
        "'import torch' found diffrast_amd/torch.py instead of PyTorch, because the package "
        "directory is the working directory or is on sys.path. Put its parent directory on "
        "sys.path instead."
    )

from diffrast_amd import *  # noqa: F403,E402
from diffrast_amd import __all__ as __all__  # noqa: E402
