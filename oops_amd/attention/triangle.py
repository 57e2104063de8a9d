"""``triangle_attention``: row-wise attention over the column axis of pair features.

Drop-in for the reference's public operator
(oops/attention/triangle/triangle_attention.py:38-101): same signature, the
same dense and NestedTensor layouts, the same ``ValueError`` /
``OOpsUnsupportedError`` contract, fully masked rows return zero, output in
the query dtype, first-order reverse-mode autograd for q, k, v and the bias.
The compute runs in the gfx950 HIP library through ``_core``.
"""

from __future__ import annotations

from math import prod
from typing import Optional

import torch
from torch import Tensor

from .. import _lib
from .._errors import unsupported
from . import _core
from ._runtime import is_nested, require_no_forward_mode, require_same_device

_OPERATOR = "triangle_attention"


def triangle_attention(
    query,
    key,
    value,
    mask=None,
    triangle_bias=None,
    *,
    scale: Optional[float] = None,
):
    r"""Apply row-wise triangle attention over the column axis of pair features.

    Args:
        query: dense ``(*prefix, R, C, H, D)`` queries (``1 <= D <= 256``) or a
            NestedTensor of square ``(*prefix, N_i, N_i, H, D)`` elements.
        key, value: same shape, dtype, device and nested topology as ``query``.
        mask: optional bool keep-mask broadcastable to ``(*prefix, R, C)``;
            ``False`` excludes a key column.
        triangle_bias: optional additive bias ``(*prefix, R|1, H, C, C)`` in the
            q/k/v dtype or float32.
        scale: multiplies Q.K before the bias; ``None`` uses ``D ** -0.5``.

    Returns the attention values with the query's shape and dtype; rows whose
    keys are all masked are zero.  The ending-node orientation (pair axes
    swapped in memory, e.g. ``x.transpose(-4, -3)`` of a contiguous tensor) is
    read in place.
    """

    if is_nested(query):
        if not is_nested(key) or not is_nested(value):
            raise ValueError("triangle_attention query, key, and value must all use the same NestedTensor layout")
        if mask is not None and not is_nested(mask):
            raise ValueError("triangle_attention mask must use the same NestedTensor layout as nested query/key/value")
        if triangle_bias is not None and not is_nested(triangle_bias):
            raise ValueError(
                "triangle_attention triangle_bias must use a compatible NestedTensor layout with nested query/key/value"
            )
        from .nested import nested_triangle_attention

        return nested_triangle_attention(query, key, value, mask, triangle_bias, scale)
    if is_nested(key) or is_nested(value):
        raise ValueError("triangle_attention query, key, and value must all use the same NestedTensor layout")
    if is_nested(mask) or is_nested(triangle_bias):
        raise ValueError("triangle_attention dense query/key/value cannot use NestedTensor mask or triangle_bias")
    require_no_forward_mode(_OPERATOR, query, key, value, triangle_bias)
    return _dense(query, key, value, mask, triangle_bias, scale)


def _check_dense_shapes(query, key, value, mask, triangle_bias) -> None:
    """Shape contract of the reference's _check_dense_shapes (triangle_attention.py:194-227)."""

    if query.dim() < 4:
        raise ValueError(
            "triangle_attention query must be (*prefix, rows, cols, num_heads, head_size) of rank at least 4, "
            f"got rank {query.dim()}"
        )
    if key.shape != query.shape or value.shape != query.shape:
        raise ValueError("triangle_attention query, key, and value must have the same shape")
    if mask is not None:
        target = tuple(query.shape[:-2])
        if mask.dim() > len(target) or any(
            size not in (1, extent) for size, extent in zip(reversed(mask.shape), reversed(target))
        ):
            raise ValueError(
                f"triangle_attention mask shape {tuple(mask.shape)} must broadcast to the query's "
                f"(*prefix, rows, cols) = {target}"
            )
    if triangle_bias is not None:
        *prefix, rows, cols, num_heads, _ = query.shape
        shape = tuple(triangle_bias.shape)
        if (
            triangle_bias.dim() != query.dim()
            or shape[: len(prefix)] != tuple(prefix)
            or shape[len(prefix)] not in (1, rows)
            or shape[len(prefix) + 1 :] != (num_heads, cols, cols)
        ):
            raise ValueError(
                f"triangle_attention triangle_bias shape {shape} must be {(*prefix, 'rows|1', num_heads, cols, cols)}"
            )


def pair_orientation(tensor: Tensor) -> Optional[bool]:
    """False: row-major; True: swapped pair axes; None: neither (triangle_attention.py:249-258)."""

    if tensor.is_contiguous():
        return False
    batch, rows, cols, heads, head = tensor.shape
    expected = (rows * cols * heads * head, heads * head, rows * heads * head, head, 1)
    if all(size == 1 or stride == want for size, stride, want in zip(tensor.shape, tensor.stride(), expected)):
        return True
    return None


def _describe(t) -> Optional[str]:
    return None if t is None else f"{tuple(t.shape)} {t.dtype} {t.device}"


def _dense(query, key, value, mask, triangle_bias, scale):
    _check_dense_shapes(query, key, value, mask, triangle_bias)
    require_same_device(_OPERATOR, query, key, value, mask, triangle_bias)
    if mask is not None and mask.dtype is not torch.bool:
        raise unsupported(_OPERATOR, "requires a bool keep-mask", mask_dtype=mask.dtype)
    head_size = query.shape[-1]
    if (
        query.device.type != "cuda"
        or query.dtype not in _core.SUPPORTED_DTYPES
        or key.dtype != query.dtype
        or value.dtype != query.dtype
        or not (0 < head_size <= _core.MAX_HEAD_SIZE)
        or query.numel() == 0
        or (triangle_bias is not None and triangle_bias.dtype not in (query.dtype, torch.float32))
    ):
        raise unsupported(
            _OPERATOR,
            "requires CUDA float16/bfloat16/float32 q/k/v of one dtype and shape with head_size <= 256, "
            "a bool mask broadcastable to (*prefix, rows, cols), and a (*prefix, rows|1, num_heads, cols, cols) "
            "bias in the q/k/v dtype or float32",
            query=_describe(query),
            key=_describe(key),
            value=_describe(value),
            mask=_describe(mask),
            triangle_bias=_describe(triangle_bias),
        )
    shape = query.shape
    batchless = query.dim() == 4
    prefixed = query.dim() > 5

    def batched(t: Tensor) -> Tensor:
        return t.unsqueeze(0) if batchless else t.flatten(0, -5)

    if batchless or prefixed:
        bq = batched(query)
        bk = bq if key is query else batched(key)
        bv = bq if value is query else bk if value is key else batched(value)
        query, key, value = bq, bk, bv
        triangle_bias = None if triangle_bias is None else batched(triangle_bias)
    query, key, value = (_core.kernel_operand(t) for t in (query, key, value))
    triangle_bias = _core.kernel_operand(triangle_bias)
    batch, rows, cols, num_heads, head_size = query.shape

    # orientation: read the swapped (ending-node) layout in place, coalesce mixed layouts
    orientations = [pair_orientation(t) for t in (query, key, value)]
    transposed = all(o is True for o in orientations)
    if not transposed and not all(o is False for o in orientations):
        query, key, value = (t.contiguous() for t in (query, key, value))

    if mask is not None:
        mask = mask.expand(shape[:-2]).reshape(batch, rows, cols)
        if mask.stride(-1) != 1:
            mask = mask.contiguous()
    if triangle_bias is not None and triangle_bias.stride(-1) != 1:
        triangle_bias = triangle_bias.contiguous()
    scale = head_size**-0.5 if scale is None else float(scale)

    table = []
    bias_groups = 0 if triangle_bias is None else triangle_bias.shape[1]
    for b in range(batch):
        qs = (b * query.stride(0), query.stride(1), query.stride(3), query.stride(2))
        ks = (b * key.stride(0), key.stride(1), key.stride(3), key.stride(2))
        vs = (b * value.stride(0), value.stride(1), value.stride(3), value.stride(2))
        bias_cols = dbias_cols = None
        mode = _lib.BIAS_NONE
        if triangle_bias is not None:
            shared = bias_groups == 1
            st = triangle_bias.stride()
            bias_cols = (b * st[0], 0 if shared else st[1], st[2], st[3])
            per_b = bias_groups * num_heads * cols * cols
            dbias_cols = (b * per_b, 0 if shared else num_heads * cols * cols, cols * cols, cols)
            mode = _lib.BIAS_SHARED if shared else _lib.BIAS_FULL
        mask_cols = None
        if mask is not None:
            mask_cols = (b * mask.stride(0), mask.stride(1), 0)
        table += _core.table_row(
            groups=rows, len_q=cols, len_k=cols, q=qs, k=ks, v=vs, bias=bias_cols, dbias=dbias_cols,
            bias_mode=mode, mask=mask_cols, lse_off=b * rows * num_heads * cols,
        )
    out = _core.attend(
        query, key, value, mask, triangle_bias, table, num_heads, scale, batch * rows * num_heads * cols
    )
    if batchless:
        return out.squeeze(0)
    return out.reshape(shape) if prefixed else out
