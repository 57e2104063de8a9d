"""``pair_bias_attention``: head-major attention with an additive pair bias (MSA row attention).

Drop-in for the reference's operator
(oops/attention/pair_bias/pair_bias_attention.py:57-244 and the admission
rules of oops/attention/flash/triton/problem.py:170-274); DanLing
NestedTensor inputs go to ``pair_bias_nested`` (ragged MSA):

* q/k/v ``(*prefix, S, H, Q|K, D)``; rank 3 omits prefix and group, rank 4
  the prefix; query and key lengths may differ.
* mask: bool keep-mask ``(*prefix, S|1, K)`` (key mask), ``(*prefix, S|1,
  Q|1, K)`` (pair mask) or ``(*prefix, S|1, 1, Q|1, K)``.
* pair_bias ``(*prefix, S|1, H|1, Q|1, K|1)`` in the q/k/v dtype, or float32
  over half q/k/v inside CUDA autocast of that dtype.

It lowers to the same attention ops as ``triangle_attention``: one geometry
table row per batch element with groups = S, the query/key strides read in
place, the bias in shared (S|1 = 1) or per-group mode.  Bias axes broadcast
over heads, queries or keys are expanded before the call, so autograd's
expand backward sums the gradient to the bias's own shape.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .. import _lib
from .._errors import unsupported
from . import _core
from ._runtime import is_nested, require_no_forward_mode, require_same_device
from .pair_bias_nested import nested_pair_bias_attention

_OPERATOR = "pair_bias_attention"
_HALF = (torch.float16, torch.bfloat16)


def pair_bias_attention(
    query,
    key,
    value,
    mask=None,
    pair_bias=None,
    *,
    scale: Optional[float] = None,
):
    r"""Scaled dot-product attention over head-major q/k/v with an optional additive pair bias.

    Args:
        query: ``(*prefix, S, H, Q, D)`` queries, ``1 <= D <= 256``; rank 3
            omits prefix and group, rank 4 omits the prefix.
        key, value: ``(*prefix, S, H, K, D)`` with the query's prefix, groups,
            heads, head size, dtype and device.
        mask: optional bool keep-mask ``(*prefix, S|1, K)``,
            ``(*prefix, S|1, Q|1, K)`` or ``(*prefix, S|1, 1, Q|1, K)``;
            ``False`` excludes a key or a (query, key) pair.
        pair_bias: optional additive bias ``(*prefix, S|1, H|1, Q|1, K|1)``.
        scale: multiplies Q.K before the bias; ``None`` uses ``D ** -0.5``.

    Returns the attention values with the query's shape and dtype; fully
    masked query rows are zero.  First-order reverse mode differentiates
    q, k, v and the bias (broadcast bias gradients are summed to its shape).
    """

    if is_nested(query):
        if not (is_nested(key) and is_nested(value)):
            raise ValueError("pair_bias_attention query, key, and value must all use NestedTensor")
        if mask is not None and not is_nested(mask):
            raise ValueError("pair_bias_attention nested query/key/value require a NestedTensor mask")
        if pair_bias is not None and not is_nested(pair_bias):
            raise ValueError("pair_bias_attention nested query/key/value require a NestedTensor pair_bias")
        return nested_pair_bias_attention(query, key, value, mask, pair_bias, scale)
    if is_nested(key) or is_nested(value):
        raise ValueError("pair_bias_attention query, key, and value must all use NestedTensor")
    if is_nested(mask) or is_nested(pair_bias):
        raise ValueError("pair_bias_attention dense query/key/value cannot use NestedTensor mask or pair_bias")
    require_no_forward_mode(_OPERATOR, query, key, value, pair_bias)
    if mask is not None and mask.dim() == query.dim():
        if mask.shape[-3] != 1:
            raise unsupported(
                _OPERATOR,
                "serves a mask head axis only of size 1",
                mask_shape=tuple(mask.shape),
                query_shape=tuple(query.shape),
            )
        mask = mask.squeeze(-3)
    if mask is not None and mask.dim() == query.dim() - 1 and mask.shape[-2] == 1:
        mask = mask.squeeze(-2)
    _check_head_major(query, key, value)
    require_same_device(_OPERATOR, query, key, value, mask, pair_bias)
    rank = query.dim()
    if rank == 3:
        unit = lambda t: None if t is None else t.unsqueeze(0)  # noqa: E731
        bq = query.unsqueeze(0)
        bk = bq if key is query else key.unsqueeze(0)
        bv = bq if value is query else bk if value is key else value.unsqueeze(0)
        return _grouped(bq, bk, bv, unit(mask), unit(pair_bias), scale).squeeze(0)
    if rank > 5:
        return _prefixed(query, key, value, mask, pair_bias, scale)
    return _grouped(query, key, value, mask, pair_bias, scale)


def _check_head_major(query, key, value) -> None:
    """Shape contract of check_head_major_qkv (oops/attention/flash/qkv.py:38-52)."""

    if query.dim() < 3:
        raise ValueError("query must have layout (num_heads, query_length, head_size) under an optional prefix")
    if key.dim() != query.dim() or value.dim() != query.dim():
        raise ValueError("query, key, and value must have the same rank")
    if key.shape[:-2] != query.shape[:-2] or value.shape[:-2] != key.shape[:-2]:
        raise ValueError("query, key, and value must share prefix and num_heads dimensions")
    if key.shape[-1] != query.shape[-1]:
        raise ValueError("query and key head_size dimensions must match")
    if value.shape[-1] != query.shape[-1]:
        raise ValueError("query and value head_size dimensions must match")
    if value.shape[-2] != key.shape[-2]:
        raise ValueError("key and value key_len dimensions must match")


def _mask_is_key(query: Tensor, mask: Tensor) -> bool:
    return mask.dim() == query.dim() - 2


def _prefixed(query, key, value, mask, pair_bias, scale):
    """Flatten ``*prefix`` into one batch axis (pair_bias_attention.py:174-244)."""

    batch_prefix = query.shape[:-4]
    groups = query.shape[-4]
    if mask is not None:
        if mask.dim() == query.dim() - 2:
            ok = mask.shape[:-2] == batch_prefix and mask.shape[-2] in (1, groups) and mask.shape[-1] == key.shape[-2]
        elif mask.dim() == query.dim() - 1:
            ok = (
                mask.shape[:-3] == batch_prefix
                and mask.shape[-3] in (1, groups)
                and mask.shape[-2:] == (query.shape[-2], key.shape[-2])
            )
        else:
            ok = False
        if not ok:
            raise ValueError(
                "pair_bias_attention mask must have shape "
                "(*batch_prefix, group|1, key_len) or "
                "(*batch_prefix, group|1, query_length|1, key_len), optionally with a unit head "
                "axis before query_length, matching query/key"
            )
    if pair_bias is not None and (
        pair_bias.dim() != query.dim()
        or pair_bias.shape[:-4] != batch_prefix
        or pair_bias.shape[-4] not in (1, groups)
        or pair_bias.shape[-3] not in (1, query.shape[-3])
        or pair_bias.shape[-2] not in (1, query.shape[-2])
        or pair_bias.shape[-1] not in (1, key.shape[-2])
    ):
        raise ValueError(
            "pair_bias_attention pair_bias must have shape "
            "(*batch_prefix, group|1, num_heads|1, query_length|1, key_len|1) matching query/key"
        )
    gq = query.flatten(0, -5)
    gk = gq if key is query else key.flatten(0, -5)
    gv = gq if value is query else gk if value is key else value.flatten(0, -5)
    if mask is not None:
        mask = mask.flatten(0, -3) if _mask_is_key(query, mask) else mask.flatten(0, -4)
    gb = None if pair_bias is None else pair_bias.flatten(0, -5)
    return _grouped(gq, gk, gv, mask, gb, scale).reshape(query.shape)


def _unit_batch(t: Tensor, rank: int) -> Tensor:
    """Prepend unit axes up to ``rank`` (the reference's degenerate_shape)."""

    while t.dim() < rank:
        t = t.unsqueeze(0)
    return t


def _describe(t) -> Optional[str]:
    return None if t is None else f"{tuple(t.shape)} {t.dtype} {t.device}"


def _raise_unsupported(query, key, value, mask, pair_bias):
    raise unsupported(
        _OPERATOR,
        "requires CUDA float16/bfloat16/float32 query/key/value sharing one dtype with "
        f"head_size <= {_core.MAX_HEAD_SIZE}, a pair bias in that dtype -- or a same-device "
        "float32 bias over half-precision Q/K/V inside matching CUDA autocast -- at the query's own rank "
        "shaped (batch, sample|1, num_heads|1, query_length|1, key_len|1) whose batch axis is the query's own "
        "and not expanded over a zero stride, and a bool keep mask shaped (batch, sample|1, key_len) or "
        "(batch, sample|1, query_length|1, key_len), optionally with a unit head axis before query_length",
        query=_describe(query),
        key=_describe(key),
        value=_describe(value),
        mask=_describe(mask),
        pair_bias=_describe(pair_bias),
        pair_bias_stride=None if pair_bias is None else tuple(pair_bias.stride()),
    )


def _supported(query, key, value, mask, pair_bias) -> bool:
    """Admission rules of supports_head_major_qkv / supports_pair_mask / supports_pair_bias
    (oops/attention/flash/triton/problem.py:170-263)."""

    if not (
        query.device.type == "cuda"
        and query.dim() in (4, 5)
        and query.dtype in _core.SUPPORTED_DTYPES
        and key.dtype == query.dtype
        and value.dtype == query.dtype
        and query.shape[-3] > 0
        and query.shape[-2] > 0
        and key.shape[-2] > 0
        and 0 < query.shape[-1] <= _core.MAX_HEAD_SIZE
        and query.numel() > 0
    ):
        return False
    q5 = _unit_batch(query, 5)
    batch, samples = q5.shape[:2]
    if mask is not None:
        if mask.dtype is not torch.bool:
            return False
        if _mask_is_key(query, mask):
            trailing = (key.shape[-2],)
        elif mask.dim() == query.dim() - 1:
            trailing = (query.shape[-2], key.shape[-2])
        else:
            return False
        shape = _unit_batch(mask, len(trailing) + 2).shape
        if not (shape[0] == batch and shape[1] in (1, samples) and tuple(shape[2:]) == trailing):
            return False
    if pair_bias is not None:
        if pair_bias.dim() != query.dim():
            return False
        autocast_f32 = (
            query.dtype in _HALF
            and pair_bias.dtype == torch.float32
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == query.dtype
        )
        if not (pair_bias.dtype == query.dtype or autocast_f32):
            return False
        b5 = _unit_batch(pair_bias, 5)
        target = (batch, samples, q5.shape[2], q5.shape[3], key.shape[-2])
        if b5.shape[0] != batch or (batch != 1 and b5.stride(0) == 0):
            return False
        if any(size not in (1, want) for size, want in zip(b5.shape[1:], target[1:])):
            return False
    return True


def _grouped(query, key, value, mask, pair_bias, scale):
    """Rank-4 ``(S, H, Q, D)`` or rank-5 ``(B, S, H, Q, D)`` call."""

    if not _supported(query, key, value, mask, pair_bias):
        _raise_unsupported(query, key, value, mask, pair_bias)
    rank = query.dim()
    shape = query.shape
    key_is_query, value_is_query, value_is_key = key is query, value is query, value is key
    query = _core.kernel_operand(_unit_batch(query, 5))
    key = query if key_is_query else _core.kernel_operand(_unit_batch(key, 5))
    value = query if value_is_query else key if value_is_key else _core.kernel_operand(_unit_batch(value, 5))
    # the kernels read the head dim with unit stride
    if query.stride(-1) != 1:
        query = query.contiguous()
    if key.stride(-1) != 1:
        key = key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    batch, samples, num_heads, len_q, head_size = query.shape
    len_k = key.shape[3]

    pair_mask = False
    if mask is not None:
        if mask.dim() == rank - 2:  # key mask
            mask = _unit_batch(mask, 3)  # (B, S|1, K)
        else:
            mask = _unit_batch(mask, 4)  # (B, S|1, Q|1, K)
            pair_mask = mask.shape[2] != 1
            if not pair_mask:
                mask = mask.squeeze(2)
        if mask.stride(-1) != 1:
            mask = mask.contiguous()

    bias = None
    if pair_bias is not None:
        bias = _core.kernel_operand(_unit_batch(pair_bias, 5))
        target = (batch, bias.shape[1], num_heads, len_q, len_k)
        if tuple(bias.shape) != target or bias.stride(-1) != 1:
            # heads/queries/keys broadcast: materialise so the kernels read unit key
            # strides and write one gradient cell per (head, query, key)
            bias = bias.expand(target).contiguous()
    scale = head_size**-0.5 if scale is None else float(scale)

    table = []
    for b in range(batch):
        qs = (b * query.stride(0), query.stride(1), query.stride(2), query.stride(3))
        ks = (b * key.stride(0), key.stride(1), key.stride(2), key.stride(3))
        vs = (b * value.stride(0), value.stride(1), value.stride(2), value.stride(3))
        bias_cols = dbias_cols = None
        mode = _lib.BIAS_NONE
        if bias is not None:
            shared = bias.shape[1] == 1
            st = bias.stride()
            bias_cols = (b * st[0], 0 if shared else st[1], st[2], st[3])
            per_b = bias.shape[1] * num_heads * len_q * len_k
            dbias_cols = (b * per_b, 0 if shared else num_heads * len_q * len_k, len_q * len_k, len_k)
            mode = _lib.BIAS_SHARED if shared else _lib.BIAS_FULL
        mask_cols = None
        if mask is not None:
            ms = mask.stride()
            m_sg = 0 if mask.shape[1] == 1 else ms[1]
            mask_cols = (b * ms[0], m_sg, ms[2] if pair_mask else 0)
        table += _core.table_row(
            groups=samples, len_q=len_q, len_k=len_k, q=qs, k=ks, v=vs, bias=bias_cols, dbias=dbias_cols,
            bias_mode=mode, mask=mask_cols, lse_off=b * samples * num_heads * len_q,
        )
    out = _core.attend(query, key, value, mask, bias, table, num_heads, scale, batch * samples * num_heads * len_q)
    return out.squeeze(0) if rank == 4 else out

