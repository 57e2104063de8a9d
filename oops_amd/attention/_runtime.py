"""Small runtime guards shared by the front-ends.

Restates the contract pieces of the reference's runtime helpers
(oops/runtime/dispatch.py:529-636): forward-mode AD is rejected with
``OOpsUnsupportedError``; operands must share one device.
"""

from __future__ import annotations

import torch
from torch._C import _functions as _autograd_nodes
from torch.autograd import forward_ad
from torch.utils._python_dispatch import _get_current_dispatch_mode

from .._errors import unsupported


def is_nested(x) -> bool:
    """Duck-typed DanLing ``NestedTensor`` test (packed ``.concat`` + ``.packed_like``)."""

    return x is not None and not isinstance(x, torch.Tensor) and hasattr(x, "concat") and hasattr(x, "packed_like")


def forward_mode_active(*tensors) -> bool:
    if forward_ad._current_level < 0:
        return False
    try:
        if torch._C._are_functorch_transforms_active():
            return True
    except AttributeError:  # pragma: no cover
        pass
    for t in tensors:
        if isinstance(t, torch.Tensor) and forward_ad.unpack_dual(t).tangent is not None:
            return True
    return False


def require_no_forward_mode(operator: str, *tensors) -> None:
    if forward_mode_active(*tensors):
        raise unsupported(
            operator,
            "does not support forward-mode AD",
            hint="use reverse-mode autograd or the equivalent Torch operation for a Jacobian-vector product",
        )


def require_same_device(operator: str, *tensors) -> None:
    devices = {t.device for t in tensors if isinstance(t, torch.Tensor)}
    if len(devices) > 1:
        raise ValueError(f"{operator} operands must share one device, got {sorted(map(str, devices))}")


def needs_custom_op(tensor) -> bool:
    """True where an operator must go through its ``torch.library`` custom op (fake kernel, traced
    graph): under ``torch.compile``, for fake or subclass tensors and under a Python dispatch mode.
    Elsewhere eager calls may skip the dispatcher."""

    return torch.compiler.is_compiling() or type(tensor) is not torch.Tensor or _get_current_dispatch_mode() is not None


def without_second_derivative(grads, ctx, grad_output):
    """Gradients that a kernel computed have no derivatives of their own.  When a backward runs under
    ``create_graph=True`` and ``grad_output`` or any tensor ``ctx`` saved is differentiable, the non-None ``grads`` come back as outputs of an autograd node that raises if it
    is differentiated, so a second derivative fails loudly instead of silently missing these terms.
    (The custom-op path raises the same way: its backward operator has no autograd formula.)"""

    if not torch.is_grad_enabled():  # (an ordinary backward: the saved tensors are not unpacked)
        return grads
    inputs = (grad_output, *ctx.saved_tensors)
    if not any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs):
        return grads
    present = [g for g in grads if g is not None]
    if not present:
        return grads
    node = _autograd_nodes.DelayedError(b"oops_amd operators have no second derivatives", len(present))
    wrapped = node(*[g.detach().requires_grad_() for g in present])
    wrapped = iter(wrapped if isinstance(wrapped, tuple) else (wrapped,))
    return tuple(None if g is None else next(wrapped) for g in grads)
