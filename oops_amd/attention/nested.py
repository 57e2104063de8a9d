"""Triangle attention over ragged DanLing ``NestedTensor`` batches.

Drop-in for the reference's nested path (oops/attention/triangle/
triangle_attention.py:261-513 and the sample table of oops/attention/triangle/
nested.py:20-288).  Each element is a square ``(*prefix, N_i, N_i, H, D)`` pair
block; q/k/v are packed either canonically (pair axes ``(N_i, N_i)`` flattened
row-major, ``ragged_dims == (p, p+1)``) or transposed (``ragged_dims ==
(p+1, p)``, the ending-node view of a canonical tensor).  The packed values
``(sum N_i^2, *prefix, H, D)`` are read in place: every (element, prefix
index) pair becomes one geometry-table row whose group/token strides encode
the orientation, so no element is padded to the largest N_i or copied.

The mask and bias are small next to q/k/v; they are repacked once per call
into the kernels' query-major layout (masks ``[p][g][key]``, bias
``[p][g|1][h][q][k]``) with differentiable torch ops, so the bias gradient
flows back to the caller's packed bias through autograd.
"""

from __future__ import annotations

from math import prod
from typing import Optional

import torch
from torch import Tensor

from .. import _lib
from .._errors import unsupported
from . import _core
from ._runtime import require_no_forward_mode, require_same_device

_OPERATOR = "triangle_attention"


def _canonical_qkv(operand: str, nested) -> tuple[Tensor, bool, int]:
    """(packed values, transposed, prefix rank); triangle_attention.py:389-414."""

    if not nested.batch_first or nested.dim() < 5:
        raise ValueError(f"triangle_attention nested {operand} elements must have shape (*prefix, N_i, N_i, H, D)")
    pr = nested.dim() - 5
    tail = (*range(pr), pr + 2, pr + 3)
    canonical = nested.ragged_dims == (pr, pr + 1) and nested.packed_dim_order == (pr, pr + 1, *tail)
    transposed = nested.ragged_dims == (pr + 1, pr) and nested.packed_dim_order == (pr + 1, pr, *tail)
    if not canonical and not transposed:
        raise unsupported(
            _OPERATOR,
            f"requires explicit canonical or transposed (*prefix, N_i, N_i, H, D) nested {operand} packing",
            ragged_dims=nested.ragged_dims,
            packed_dim_order=nested.packed_dim_order,
        )
    values = nested.concat
    if values.dim() != pr + 3 or values.shape[-2] <= 0 or values.shape[-1] <= 0:
        raise ValueError(f"triangle_attention nested {operand} must retain positive num_heads and head_size axes")
    return values, transposed, pr


def _broadcast_prefix(values: Tensor, prefix: tuple, tail_rank: int) -> Tensor:
    """Expand a mask/bias static prefix to the q/k/v prefix (triangle_attention.py:417-433)."""

    own = tuple(values.shape[1 : values.dim() - tail_rank])
    message = "triangle_attention nested mask and bias static prefixes must broadcast to the query prefix"
    try:
        shape = torch.broadcast_shapes(own, prefix)
    except RuntimeError as error:
        raise ValueError(message) from error
    if tuple(shape) != tuple(prefix):
        raise ValueError(message)
    tail = tuple(values.shape[values.dim() - tail_rank :])
    lead = (1,) * (len(prefix) - len(own))
    return values.reshape(values.shape[0], *lead, *own, *tail).expand(values.shape[0], *prefix, *tail)


def _row_sizes(operand: str, rows: list, packed: list, total: int) -> list:
    """N_i per element, validated (nested.py:35-47)."""

    if len(rows) <= 1:
        raise unsupported(_OPERATOR, "does not serve an empty NestedTensor batch")
    if len(packed) != len(rows):
        raise ValueError(f"triangle_attention {operand} packed offsets must contain one boundary per sample")
    sizes = [b - a for a, b in zip(rows[:-1], rows[1:])]
    if any(n <= 0 for n in sizes):
        raise unsupported(_OPERATOR, "requires every nested pair element to have N > 0")
    if any(b - a != n * n for a, b, n in zip(packed[:-1], packed[1:], sizes)):
        raise ValueError(f"triangle_attention {operand} token dims must be square (N, N) per sample")
    if total <= 0:
        raise unsupported(_OPERATOR, "requires non-empty packed pair values")
    return sizes


def _offsets(nested, level=None) -> list:
    t = nested.packed_offsets(dtype=torch.int64) if level is None else nested.ragged_level_offsets(level, dtype=torch.int64)
    return [int(x) for x in t.tolist()]


def _mask_buffer(mask, prefix: tuple, transposed: bool, rows: list, packed: list, sizes: list) -> Tensor:
    """Bool keep-mask repacked to ``[sample][p][g][key]`` (triangle_attention.py:436-463)."""

    if not mask.batch_first or mask.dim() < 3:
        raise ValueError("triangle_attention nested mask elements must have shape (*prefix, N_i, N_i)")
    pr = mask.dim() - 3
    tail = tuple(range(pr))
    canonical = mask.ragged_dims == (pr, pr + 1) and mask.packed_dim_order == (pr, pr + 1, *tail)
    mask_transposed = mask.ragged_dims == (pr + 1, pr) and mask.packed_dim_order == (pr + 1, pr, *tail)
    if not canonical and not mask_transposed:
        raise unsupported(
            _OPERATOR,
            "requires explicit canonical or transposed (*prefix, N_i, N_i) nested mask packing",
            ragged_dims=mask.ragged_dims,
            packed_dim_order=mask.packed_dim_order,
        )
    if mask_transposed != transposed:
        raise ValueError("triangle_attention nested mask must share q/k/v packed pair-axis orientation")
    values = mask.concat
    if values.dim() != pr + 1:
        raise ValueError("triangle_attention nested mask must have flattened square pair storage")
    if values.dtype is not torch.bool:
        raise unsupported(_OPERATOR, "requires a bool keep-mask", mask_dtype=values.dtype)
    if _offsets(mask, 0) != rows or _offsets(mask) != packed:
        raise ValueError("triangle_attention mask layout must match the query layout per sample")
    values = _broadcast_prefix(values, prefix, 0)
    P = prod(prefix)
    pieces = []
    for n, start in zip(sizes, packed[:-1]):
        block = values[start : start + n * n].reshape(n, n, P)  # [g][key] or [key][g]
        if transposed:
            block = block.transpose(0, 1)
        pieces.append(block.permute(2, 0, 1).reshape(-1))
    return torch.cat(pieces)


def _bias_buffer(bias, num_heads: int, prefix: tuple, rows: list, sizes: list):
    """Bias repacked to ``[sample][p][g|1][h][q][k]`` plus per-sample group counts
    (triangle_attention.py:466-509 and the bias orders of nested.py:325-377)."""

    if not bias.batch_first or bias.dim() < 5:
        raise ValueError(
            "triangle_attention nested triangle_bias elements must have shape (*prefix, rows|1, H, N_i, N_i)"
        )
    pr = bias.dim() - 5
    ragged, order = bias.ragged_dims, bias.packed_dim_order
    static = tuple(range(pr))
    shared_tail = (*static, pr, pr + 1)
    full_tail = (*static, pr + 1)
    if ragged == (pr + 2, pr + 3) and order == (*ragged, *shared_tail):
        shared, transposed = True, False
    elif ragged == (pr + 3, pr + 2) and order == (*ragged, *shared_tail):
        shared, transposed = True, True
    elif ragged == (pr, pr + 2, pr + 3) and order == (*ragged, *full_tail):
        shared, transposed = False, False
    elif ragged == (pr, pr + 3, pr + 2) and order == (*ragged, *full_tail):
        shared, transposed = False, True
    else:
        raise unsupported(
            _OPERATOR,
            "requires literal dense-order nested triangle_bias elements with canonical or transposed shared/full "
            "pair-axis ragged dimensions",
            ragged_dims=ragged,
            packed_dim_order=order,
        )
    packed_values = bias.concat
    if shared and packed_values.shape[-2] != 1:
        raise ValueError("triangle_attention row-shared nested triangle_bias must have a unit group axis")
    if packed_values.shape[-1] != num_heads:
        raise unsupported(
            _OPERATOR,
            "requires packed triangle_bias num_heads matching q/k/v",
            triangle_bias=f"{tuple(packed_values.shape)} {packed_values.dtype}",
            num_heads=num_heads,
        )
    values = packed_values.squeeze(-2) if shared else packed_values
    values = _broadcast_prefix(values, prefix, 1)  # (rows, *prefix, H)
    packed = _offsets(bias)
    if len(packed) != len(rows):
        raise ValueError("triangle_attention triangle_bias must have one packed boundary per sample")
    if shared:
        counts = [1] * len(sizes)
        if any(b - a != n * n for a, b, n in zip(packed[:-1], packed[1:], sizes)):
            raise ValueError("triangle_attention shared triangle_bias layout must match query per sample")
    else:
        groups = _offsets(bias, 0)
        counts = [b - a for a, b in zip(groups[:-1], groups[1:])]
        if any(c not in (1, n) for c, n in zip(counts, sizes)):
            raise ValueError("triangle_attention triangle_bias group axis must be 1 or N_i per sample")
        if any(b - a != c * n * n for a, b, c, n in zip(packed[:-1], packed[1:], counts, sizes)):
            raise ValueError("triangle_attention triangle_bias query/key axes must both have length N_i per sample")
    P = prod(prefix)
    pieces = []
    for n, c, start in zip(sizes, counts, packed[:-1]):
        block = values[start : start + c * n * n].reshape(c, n, n, P, num_heads)  # [g][q][k] or [g][k][q]
        if transposed:
            block = block.transpose(1, 2)
        pieces.append(block.permute(3, 0, 4, 1, 2).reshape(-1))
    return torch.cat(pieces), counts


def nested_triangle_attention(query, key, value, mask, triangle_bias, scale: Optional[float]):
    q_values, transposed, pr = _canonical_qkv("query", query)
    k_values, k_transposed, _ = _canonical_qkv("key", key)
    v_values, v_transposed, _ = _canonical_qkv("value", value)
    require_no_forward_mode(_OPERATOR, q_values, k_values, v_values,
                            None if triangle_bias is None else triangle_bias.concat)  # fmt: skip
    if k_values.shape[1:] != q_values.shape[1:] or v_values.shape[1:] != q_values.shape[1:]:
        raise ValueError(
            "triangle_attention nested query, key, and value must share static prefix, num_heads, and head_size"
        )
    if k_transposed != transposed or v_transposed != transposed:
        raise ValueError("triangle_attention nested query, key, and value must share packed pair-axis orientation")
    prefix = tuple(q_values.shape[1:-2])
    P = prod(prefix)
    num_heads, head_size = q_values.shape[-2:]
    rows, packed = _offsets(query, 0), _offsets(query)
    sizes = _row_sizes("query", rows, packed, q_values.shape[0])
    for operand, nested, vals in (("key", key, k_values), ("value", value, v_values)):
        if vals.shape[0] != q_values.shape[0] or _offsets(nested, 0) != rows or _offsets(nested) != packed:
            raise ValueError(f"triangle_attention {operand} layout must match the query layout per sample")

    mask_values = None if mask is None else _mask_buffer(mask, prefix, transposed, rows, packed, sizes)
    bias_values, counts = (None, None) if triangle_bias is None else _bias_buffer(
        triangle_bias, num_heads, prefix, rows, sizes
    )
    require_same_device(_OPERATOR, q_values, k_values, v_values, mask_values, bias_values)
    if (
        q_values.device.type != "cuda"
        or q_values.dtype not in _core.SUPPORTED_DTYPES
        or k_values.dtype != q_values.dtype
        or v_values.dtype != q_values.dtype
        or not (0 < head_size <= _core.MAX_HEAD_SIZE)
        or (bias_values is not None and bias_values.dtype not in (q_values.dtype, torch.float32))
    ):
        raise unsupported(
            _OPERATOR,
            "requires CUDA float16/bfloat16/float32 canonical/transposed packed NestedTensor q/k/v with "
            "head_size <= 256, a matching bool nested mask, and independently canonical/transposed "
            "nested triangle bias in the q/k/v dtype or float32",
            query=f"{tuple(q_values.shape)} {q_values.dtype} {q_values.device}",
        )

    # (cells, *prefix, H, D) -> (cells * P, H, D): row (cell, p) = cell * P + p
    flat = [_core.kernel_operand(t).reshape(t.shape[0] * P, num_heads, head_size) for t in (q_values, k_values, v_values)]
    if key is query:
        flat[1] = flat[0]
    if value is query:
        flat[2] = flat[0]
    elif value is key:
        flat[2] = flat[1]
    qf, kf, vf = (t if t.is_contiguous() else t.contiguous() for t in flat)
    bias_values = _core.kernel_operand(bias_values)
    scale = head_size**-0.5 if scale is None else float(scale)

    hd = num_heads * head_size
    table = []
    lse_off = 0
    mask_off = 0
    bias_off = 0
    for i, (n, start) in enumerate(zip(sizes, packed[:-1])):
        for p in range(P):
            base = (start * P + p) * hd
            if transposed:
                s_g, s_i = P * hd, n * P * hd
            else:
                s_g, s_i = n * P * hd, P * hd
            operand = (base, s_g, head_size, s_i)
            bias_cols = dbias_cols = None
            mode = _lib.BIAS_NONE
            if bias_values is not None:
                c = counts[i]
                shared = c == 1
                cols = (bias_off, 0 if shared else num_heads * n * n, n * n, n)
                bias_cols = dbias_cols = cols
                mode = _lib.BIAS_SHARED if shared else _lib.BIAS_FULL
                bias_off += c * num_heads * n * n
            mask_cols = None
            if mask_values is not None:
                mask_cols = (mask_off, n, 0)
                mask_off += n * n
            table += _core.table_row(
                groups=n, len_q=n, len_k=n, q=operand, k=operand, v=operand, bias=bias_cols, dbias=dbias_cols,
                bias_mode=mode, mask=mask_cols, lse_off=lse_off,
            )  # fmt: skip
            lse_off += n * num_heads * n
    out = _core.attend(qf, kf, vf, mask_values, bias_values, table, num_heads, scale, lse_off)
    return query.packed_like(out.reshape(q_values.shape))
