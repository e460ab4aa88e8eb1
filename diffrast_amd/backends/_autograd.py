"""Guard for backward passes that are kernels (reference: src/diffrast/backends/_autograd.py)."""

from __future__ import annotations

import functools
from collections.abc import Callable

import torch


def first_order(op: str) -> Callable[[Callable], Callable]:
    """Decorate a ``backward`` so that running it with ``create_graph=True`` raises.

    PyTorch enables gradient tracking inside ``backward`` exactly when a differentiable gradient
    was requested. The kernels here compute first-order gradients only, so that request is
    refused with an error naming ``op`` rather than answered without the second-order terms
    (reference _autograd.py:11-35; the message keeps the reference's wording).
    """

    def decorate(backward: Callable) -> Callable:
        @functools.wraps(backward)
        def guarded(ctx, *grads):
            if torch.is_grad_enabled():
                raise RuntimeError(
                    f"{op} on the HIP backend has no second-order gradients, but its backward "
                    "pass was run with create_graph=True. Gradients of gradients need the "
                    "pure-PyTorch reference diffrast."
                )
            return backward(ctx, *grads)

        return guarded

    return decorate
