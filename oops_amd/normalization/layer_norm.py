"""``layer_norm``: LayerNorm over the last dimension on the HIP row kernels.

Drop-in for the reference's operator
(oops/normalization/layer_norm/layer_norm.py:30-148): dense or DanLing
nested input whose normalized (final) axis is static and physically last,
float16 / bfloat16 / float32 activations, widths 1-8192, optional affine parameters in the
activation dtype (or float32 over half activations).  Forward and backward run
in ``row_norm_*_kernel`` behind ``oops_layer_norm_rows_forward`` and
``oops_layer_norm_rows_backward_affine`` (float32 statistics, biased
variance); the affine gradients are float32 per-wave partials that the library
sums in a fixed order, returned in the parameters' dtype.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
import math
from typing import Iterable, Optional, Tuple, Union

import torch
from torch import Tensor

from .. import _lib
from .._errors import unsupported
from ..attention._runtime import (
    is_nested,
    needs_custom_op,
    require_no_forward_mode,
    require_same_device,
    without_second_derivative,
)

_OPERATOR = "layer_norm"
_HALF = (torch.float16, torch.bfloat16)
_DTYPE_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}
MAX_WIDTH = 8192


def layer_norm(
    input,
    normalized_shape: Union[int, Iterable[int]],
    weight: Optional[Tensor] = None,
    bias: Optional[Tensor] = None,
    eps: float = 1e-5,
):
    r"""Normalize the final feature dimension.

    Args:
        input: CUDA float16 / bfloat16 / float32 ``(..., C)`` tensor, or a
            nested tensor whose final feature axis is static and physically last.
        normalized_shape: ``C`` or ``(C,)`` with ``1 <= C <= 8192``.
        weight, bias: optional ``(C,)`` affine parameters in the activation
            dtype, or float32 for half activations.
        eps: added to the variance before the reciprocal square root.

    Returns the normalized values with the input's shape, dtype and topology.
    """

    if is_nested(input):
        return _nested(input, normalized_shape, weight, bias, eps)
    require_no_forward_mode(_OPERATOR, input, weight, bias)
    require_same_device(_OPERATOR, input, weight, bias)
    shape = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
    if len(shape) != 1:
        raise unsupported(_OPERATOR, "normalizes over the final dimension only", normalized_shape=shape,
                          input_shape=tuple(input.shape))  # fmt: skip
    width = shape[0]
    if torch.is_autocast_enabled("cuda") and input.dtype not in _HALF and any(
        t is not None and t.is_floating_point() and t.dtype != input.dtype for t in (weight, bias)
    ):
        raise unsupported(_OPERATOR, "does not reimplement autocast promotion for a float32 activation with half "
                          "affine", input_dtype=input.dtype)  # fmt: skip
    affine_dtypes = {t.dtype for t in (weight, bias) if t is not None}
    ok = (
        input.is_cuda
        and input.dtype in _DTYPE_CODE
        and input.dim() >= 1
        and input.shape[-1] == width
        and 0 < width <= MAX_WIDTH
        and input.numel() > 0
        and all(t is None or tuple(t.shape) == (width,) for t in (weight, bias))
        and len(affine_dtypes) <= 1
        and affine_dtypes <= {input.dtype, torch.float32}
        and (input.dtype in _HALF or affine_dtypes <= {torch.float32})
    )
    if not ok:
        raise unsupported(
            _OPERATOR,
            "requires a CUDA half/float32 activation with a matching contiguous affine row",
            input_dtype=input.dtype,
            device=input.device,
            normalized_size=width,
            weight_dtype=None if weight is None else weight.dtype,
            bias_dtype=None if bias is None else bias.dtype,
        )
    return _apply(input, weight, bias, float(eps))


def _nested(input, normalized_shape, weight, bias, eps):
    """layer_norm.py:113-143: the packed values carry the static final axis."""

    if is_nested(weight) or is_nested(bias):
        raise ValueError("layer_norm NestedTensor input requires dense affine parameters")
    if input.dim() < 2 or not input.ragged_dims:
        raise unsupported(_OPERATOR, "requires a NestedTensor with explicit packed element topology",
                          ragged_dims=input.ragged_dims)  # fmt: skip
    last = input.dim() - 2
    if last in tuple(input.ragged_dims) or tuple(input.packed_dim_order)[-1] != last:
        raise unsupported(_OPERATOR, "requires the final logical element dimension to be static and physically last",
                          ragged_dims=input.ragged_dims, packed_dim_order=input.packed_dim_order)  # fmt: skip
    if input.concat.dim() < 1:
        raise unsupported(_OPERATOR, "requires packed values with a retained static final dimension")
    return input.packed_like(layer_norm(input.concat, normalized_shape, weight, bias, eps))


@functools.lru_cache(maxsize=256)
def _geometry(dtype, rows: int, width: int, x_row: int, eps: float) -> _lib.RowNormGeometry:
    """The launch geometry (cached: the library only reads it)."""

    g = _lib.RowNormGeometry()
    g.dtype = _DTYPE_CODE[dtype]
    g.width, g.rows, g.x_row, g.y_row, g.eps = width, rows, x_row, width, float(eps)
    return g


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


@functools.lru_cache(maxsize=64)
def _backward_workspace_bytes(lib, dtype, rows: int, width: int, x_row: int) -> int:
    return lib.oops_layer_norm_rows_backward_workspace_bytes(ctypes.byref(_geometry(dtype, rows, width, x_row, 0.0)))


def _stream(device) -> int:
    """The raw handle of the device's current stream."""

    return torch._C._cuda_getCurrentRawStream(device.index)


def _on_device(device):
    """The device context of a launch (a no-op when that device is already current)."""

    return contextlib.nullcontext() if device.index == torch.cuda.current_device() else torch.cuda.device(device)


def _forward_impl(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float) -> Tuple[Tensor, Tensor, Tensor]:
    lib = _lib.load()
    rows, width = x.shape
    y = torch.empty(rows, width, dtype=x.dtype, device=x.device)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    rstd = torch.empty_like(mean)
    geo = _geometry(x.dtype, rows, width, x.stride(0) if rows > 1 else width, eps)
    with _on_device(x.device):
        rc = lib.oops_layer_norm_rows_forward(ctypes.byref(geo), _ptr(x), _ptr(weight), _ptr(bias), _ptr(y),
                                              _ptr(mean), _ptr(rstd), _stream(x.device))
    _lib.check(rc, "layer_norm forward")
    return y, mean, rstd


def _backward_impl(dy: Tensor, x: Tensor, weight: Optional[Tensor], mean: Tensor, rstd: Tensor, eps: float,
                   need_affine: bool) -> Tuple[Tensor, Tensor, Tensor]:  # fmt: skip
    lib = _lib.load()
    rows, width = x.shape
    dev = x.device
    if dy.is_neg():
        dy = dy.resolve_neg()
    if dy.dtype != x.dtype:
        dy = dy.to(x.dtype)
    if dy.dim() != 2 or not dy.is_contiguous():
        dy = dy.reshape(rows, width).contiguous()
    x_row = x.stride(0) if rows > 1 else width
    geo = _geometry(x.dtype, rows, width, x_row, eps)
    # grad_x is written with x's row stride
    dx = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=dev)
    n = width if need_affine else 0
    dw = torch.empty(n, dtype=torch.float32, device=dev)
    db = torch.empty(n, dtype=torch.float32, device=dev)
    ws_bytes = _backward_workspace_bytes(lib, x.dtype, rows, width, x_row) if need_affine else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    # (x, mean, rstd, dy and dx are never empty here)
    args = (ctypes.byref(geo), x.data_ptr(), _ptr(weight), mean.data_ptr(), rstd.data_ptr(), dy.data_ptr(),
            dx.data_ptr(), _ptr(dw), _ptr(db), _ptr(ws), ws_bytes, _stream(dev))  # fmt: skip
    # the affine gradients are summed in the library, in a fixed order
    if dev.index == torch.cuda.current_device():
        rc = lib.oops_layer_norm_rows_backward_affine(*args)
    else:
        with torch.cuda.device(dev):
            rc = lib.oops_layer_norm_rows_backward_affine(*args)
    _lib.check(rc, "layer_norm backward")
    return dx, dw, db


@torch.library.custom_op("oops_amd::layer_norm_forward", mutates_args=(), device_types="cuda")
def layer_norm_forward(
    x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float
) -> Tuple[Tensor, Tensor, Tensor]:
    """Rows ``x`` (rows, width) with unit column stride; float32 affine.  Returns (y, mean, rstd)."""

    return _forward_impl(x, weight, bias, eps)


@layer_norm_forward.register_fake
def _(x, weight, bias, eps):
    rows, width = x.shape
    return x.new_empty(rows, width), x.new_empty(rows, dtype=torch.float32), x.new_empty(rows, dtype=torch.float32)


@torch.library.custom_op("oops_amd::layer_norm_backward", mutates_args=(), device_types="cuda")
def layer_norm_backward(
    dy: Tensor, x: Tensor, weight: Optional[Tensor], mean: Tensor, rstd: Tensor, eps: float, need_affine: bool
) -> Tuple[Tensor, Tensor, Tensor]:
    """(dx, dweight, dbias); the affine gradients are float32 (empty when not needed)."""

    return _backward_impl(dy, x, weight, mean, rstd, eps, need_affine)


@layer_norm_backward.register_fake
def _(dy, x, weight, mean, rstd, eps, need_affine):
    rows, width = x.shape
    n = width if need_affine else 0
    return (torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device),
            x.new_empty(n, dtype=torch.float32), x.new_empty(n, dtype=torch.float32))  # fmt: skip


def _setup_context(ctx, inputs, output):
    x, weight, bias, eps = inputs
    _y, mean, rstd = output
    ctx.save_for_backward(x, weight, mean, rstd)
    ctx.eps = eps
    ctx.has = (weight is not None, bias is not None)
    ctx.mark_non_differentiable(mean, rstd)
    ctx.set_materialize_grads(False)  # no zero-filled gradients for mean and rstd


def _grads(ctx, dy, backward):
    x, weight, mean, rstd = ctx.saved_tensors
    need = ctx.needs_input_grad
    need_affine = bool(need[1] or need[2])
    dx, dw, db = backward(dy, x, weight, mean, rstd, ctx.eps, need_affine)
    return (dx if need[0] else None, dw if ctx.has[0] and need[1] else None,
            db if ctx.has[1] and need[2] else None, None)  # fmt: skip


def _backward(ctx, dy, _dmean, _drstd):
    if dy is None:
        return None, None, None, None
    return _grads(ctx, dy, layer_norm_backward)


layer_norm_forward.register_autograd(_backward, setup_context=_setup_context)


class _EagerLayerNorm(torch.autograd.Function):
    """The same kernels as the custom ops, for eager calls: autograd calls the
    backward directly instead of through the operator dispatcher (about 25 us
    of host time per op).  Traced code (torch.compile) takes the custom ops."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        y, mean, rstd = _forward_impl(x, weight, bias, eps)
        ctx.save_for_backward(x, weight, mean, rstd)
        ctx.eps = eps
        ctx.has = (weight is not None, bias is not None)
        ctx.set_materialize_grads(False)
        return y

    @staticmethod
    def backward(ctx, dy):
        if dy is None:
            return None, None, None, None
        return without_second_derivative(_grads(ctx, dy, _backward_impl), ctx, dy)


def _apply(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float) -> Tensor:
    width = x.shape[-1]
    rows = x.numel() // width
    # (a 2-D input is used as it is: each reshape or view adds an autograd node, about 8 us of host
    # time in the backward)
    x2 = x.resolve_neg()
    if x2.dim() != 2:
        x2 = x2.reshape(rows, width)
    if x2.stride(1) != 1 or (rows > 1 and x2.stride(0) < width):
        x2 = x2.contiguous()
    f32 = lambda t: None if t is None else t.resolve_neg().float().contiguous()  # noqa: E731
    if needs_custom_op(x2):
        y, _, _ = layer_norm_forward(x2, f32(weight), f32(bias), eps)
    else:
        y = _EagerLayerNorm.apply(x2, f32(weight), f32(bias), eps)
    return y if x.dim() == 2 else y.view(x.shape)
