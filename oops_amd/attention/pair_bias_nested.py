"""Pair-bias attention over ragged DanLing ``NestedTensor`` batches (ragged MSA).

Drop-in for the reference's nested path
(oops/attention/pair_bias/pair_bias_attention.py:247-597, with the metadata
rules of oops/attention/pair_bias/nested.py:35-467).  Each element is one
sample's head-major MSA block.  q/k/v use one of five packings:

==================  ===================  ==========================  ===============================
packing             element              ragged dims / packed order  packed values
==================  ===================  ==========================  ===============================
implicit            ``(H, Q_i, D)``      ``(1,)`` / ``(1, 0, 2)``    ``(sum Q_i, H, D)``
static groups       ``(S, H, Q_i, D)``   ``(2,)`` / ``(2, 0, 1, 3)`` ``(sum Q_i, S, H, D)``
group-outer         ``(S_i, H, Q_i, D)`` ``(0, 2)`` / ``(0,2,1,3)``  ``(sum S_i Q_i, H, D)``, s major
token-outer         ``(S_i, H, Q_i, D)`` ``(2, 0)`` / ``(2,0,1,3)``  ``(sum Q_i S_i, H, D)``, q major
ragged groups       ``(S_i, H, Q, D)``   ``(0,)`` / ``(0,1,2,3)``    ``(sum S_i, H, Q, D)``
                                         or ``(0, 2, 1, 3)``         or ``(sum S_i, Q, H, D)``
==================  ===================  ==========================  ===============================

q/k/v are read in place: every sample becomes one geometry-table row whose
group/head/token strides encode its packing, and the output is written with
the query's packing.  Keys may be longer or shorter than queries per sample.
The mask and the bias are small next to q/k/v; where their packing puts the
key axis at a non-unit stride they are repacked once per call into the
kernels' key-contiguous layouts (mask ``[g|1][q|-][k]``, bias
``[g|1][h][q][k]`` over the packed cells) with differentiable torch ops, so
the bias gradient reaches the caller's packed values through autograd.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch
from torch import Tensor

from .. import _lib
from .._errors import unsupported
from . import _core
from ._runtime import require_no_forward_mode, require_same_device

_OPERATOR = "pair_bias_attention"
_HALF = (torch.float16, torch.bfloat16)

IMPLICIT, STATIC, GROUP_OUTER, TOKEN_OUTER, RAGGED_GROUPS = "implicit", "static", "group_outer", "token_outer", "ragged"


def _offsets(nested, level=None) -> List[int]:
    t = nested.packed_offsets(dtype=torch.int64) if level is None else nested.ragged_level_offsets(level, dtype=torch.int64)
    return [int(x) for x in t.tolist()]


def _element_sizes(nested) -> List[tuple]:
    sizes = nested.element_sizes()
    if isinstance(sizes, Tensor):
        sizes = sizes.tolist()
    return [tuple(int(x) for x in s) for s in sizes]


class _Operand:
    """One of q/k/v: the values the kernels read and each sample's geometry."""

    def __init__(self, values: Tensor, kind: str, groups: List[int], lengths: List[int], cols: List[tuple],
                 heads: int, head_size: int):  # fmt: skip
        self.values, self.kind = values, kind
        self.groups, self.lengths, self.cols = groups, lengths, cols
        self.heads, self.head_size = heads, head_size


def _operand(operand: str, nested) -> _Operand:
    """Packing detection (pair_bias_attention.py:394-430) and per-sample strides."""

    if not nested.batch_first:
        raise ValueError(f"pair_bias_attention nested {operand} must be batch-first")
    rd, order, nd = tuple(nested.ragged_dims), tuple(nested.packed_dim_order), nested.dim()
    if nd == 4 and rd == (1,) and order == (1, 0, 2):
        kind = IMPLICIT
    elif nd == 5 and rd == (2,) and order == (2, 0, 1, 3):
        kind = STATIC
    elif nd == 5 and rd == (0, 2) and order == (0, 2, 1, 3):
        kind = GROUP_OUTER
    elif nd == 5 and rd == (2, 0) and order == (2, 0, 1, 3):
        kind = TOKEN_OUTER
    elif nd == 5 and rd == (0,) and order in ((0, 1, 2, 3), (0, 2, 1, 3)):
        kind = RAGGED_GROUPS
    else:
        raise unsupported(
            _OPERATOR,
            f"requires nested {operand} with (H, Q_i, D) or (S_i, H, Q_i, D) elements "
            "and ragged group and/or token axes",
            ragged_dims=rd,
            packed_dim_order=order,
        )
    values = _core.kernel_operand(nested.concat)
    want_rank = 4 if kind in (STATIC, RAGGED_GROUPS) else 3
    if values.dim() != want_rank or any(size <= 0 for size in values.shape[1:]):
        raise ValueError(f"pair_bias_attention nested {operand} must retain positive group, token, H, and D axes")
    if values.stride(-1) != 1:
        values = values.contiguous()
    packed = _offsets(nested)
    if len(packed) <= 1:
        raise unsupported(_OPERATOR, "does not serve an empty NestedTensor batch")
    if packed[0] != 0 or any(b < a for a, b in zip(packed[:-1], packed[1:])):
        raise ValueError(f"pair_bias_attention {operand} packed offsets must be monotonic and start at zero")
    if packed[-1] != values.shape[0]:
        raise ValueError(
            f"pair_bias_attention {operand} packed layout covers {packed[-1]} tokens, "
            f"but packed values contain {values.shape[0]}"
        )
    counts = [b - a for a, b in zip(packed[:-1], packed[1:])]
    if any(c <= 0 for c in counts):
        raise unsupported(_OPERATOR, f"requires every nested {operand} element to have length > 0")
    st = values.stride()
    starts = packed[:-1]
    if kind == IMPLICIT:
        heads, head_size = values.shape[1:]
        groups, lengths = [1] * len(counts), counts
        cols = [(a * st[0], 0, st[1], st[0]) for a in starts]
    elif kind == STATIC:
        s, heads, head_size = values.shape[1:]
        groups, lengths = [s] * len(counts), counts
        cols = [(a * st[0], st[1], st[2], st[0]) for a in starts]
    elif kind in (GROUP_OUTER, TOKEN_OUTER):
        heads, head_size = values.shape[1:]
        sizes = _element_sizes(nested)
        groups, lengths = [s[0] for s in sizes], [s[2] for s in sizes]
        if any(s[1] != heads or s[3] != head_size for s in sizes):
            raise ValueError("pair_bias_attention grouped head sizes must match packed Q/K/V")
        if any(c != g * n for c, g, n in zip(counts, groups, lengths)):
            raise ValueError(f"pair_bias_attention {operand} packed offsets must cover groups * tokens per sample")
        if kind == GROUP_OUTER:
            cols = [(a * st[0], n * st[0], st[1], st[0]) for a, n in zip(starts, lengths)]
        else:
            cols = [(a * st[0], st[0], st[1], g * st[0]) for a, g in zip(starts, groups)]
    else:
        if order == (0, 1, 2, 3):
            heads, length, head_size = values.shape[1:]
            s_h, s_i = st[1], st[2]
        else:
            length, heads, head_size = values.shape[1:]
            s_h, s_i = st[2], st[1]
        groups, lengths = counts, [length] * len(counts)
        cols = [(a * st[0], st[0], s_h, s_i) for a in starts]
    return _Operand(values, kind, groups, lengths, cols, heads, head_size)


def _mask_plan(mask, q: _Operand, k: _Operand):
    """Key-contiguous mask buffer and per-sample (offset, s_g, s_q) columns
    (pair_bias_attention.py:433-528, nested.py:60-89 and :400-448)."""

    if not mask.batch_first:
        raise ValueError("pair_bias_attention nested mask must be batch-first")
    rd, order, nd = tuple(mask.ragged_dims), tuple(mask.packed_dim_order), mask.dim()
    values = mask.concat
    if values.dtype is not torch.bool:
        raise unsupported(_OPERATOR, "requires a bool keep-mask", mask_dtype=values.dtype)
    n = len(q.groups)
    packed = _offsets(mask)
    if len(packed) != n + 1:
        raise ValueError("pair_bias_attention mask must have one packed boundary per sample")
    grouped = q.kind in (GROUP_OUTER, TOKEN_OUTER, RAGGED_GROUPS)
    lq, lk, groups = q.lengths, k.lengths, q.groups

    # per-group key masks of ragged-group batches, (S_i, 1, K_i) elements
    per_group = None
    if nd == 4 and rd == (0,) and order in ((0, 1, 2), (0, 2, 1)):
        per_group = RAGGED_GROUPS
    elif nd == 4 and rd == (0, 2) and order == (0, 2, 1):
        per_group = GROUP_OUTER
    elif nd == 4 and rd == (2, 0) and order == (2, 0, 1):
        per_group = TOKEN_OUTER
    if per_group is not None:
        if not grouped or per_group != q.kind:
            raise ValueError("pair_bias_attention ragged Q/K/V and per-group key mask must share packed axis order")
        if per_group == RAGGED_GROUPS:
            singleton = 1 if order == (0, 1, 2) else 2
            if values.dim() != 3 or values.shape[singleton] != 1:
                raise ValueError("pair_bias_attention ragged-group key mask elements must have shape (S_i, 1, K)")
            width = values.shape[3 - singleton]
            if width != lk[0] or [b - a for a, b in zip(packed[:-1], packed[1:])] != groups:
                raise ValueError("pair_bias_attention per-group key mask must match groups and static key lengths")
            buf = values.reshape(-1)
            cols = [(a * width, width, 0) for a in packed[:-1]]
            return buf.contiguous(), cols
        if values.dim() != 2 or values.shape[1] != 1:
            raise ValueError("pair_bias_attention ragged-group key mask elements must have shape (S_i, 1, K_i)")
        if any(b - a != g * m for a, b, g, m in zip(packed[:-1], packed[1:], groups, lk)):
            raise ValueError("pair_bias_attention group key mask query/key axes must match Q_i and K_i for every sample")
        flat = values.reshape(-1)
        if per_group == GROUP_OUTER:
            buf = flat
        else:  # token-major (K_i, S_i) blocks -> (S_i, K_i)
            buf = torch.cat([flat[a : a + g * m].view(m, g).t().reshape(-1)
                             for a, g, m in zip(packed[:-1], groups, lk)])  # fmt: skip
        cols = [(a, m, 0) for a, m in zip(packed[:-1], lk)]
        return buf.contiguous(), cols

    if nd == 2 and rd == (0,) and order == (0,):
        pair, implicit = False, True
    elif nd == 3 and rd == (0, 1) and order == (0, 1):
        pair, implicit = True, True
    elif nd == 3 and rd == (1,) and order == (1, 0):
        pair, implicit = False, False
    elif nd == 4 and rd == (1, 2) and order == (1, 2, 0):
        pair, implicit = True, False
    elif nd == 4 and rd == (2,) and order == (2, 0, 1):
        pair, implicit = False, False
        if values.dim() != 3 or values.shape[2] != 1:
            raise unsupported(
                _OPERATOR,
                "requires a nested mask query axis that is ragged as Q_i or a singleton",
                packed_shape=tuple(values.shape),
            )
        values = values.squeeze(2)
    else:
        raise unsupported(
            _OPERATOR,
            "requires a key/pair mask with an implicit unit sample axis or a uniformly shared/full "
            "explicit sample axis; per-element mixed sample sharing is not served",
            ragged_dims=rd,
            packed_dim_order=order,
        )
    if implicit:
        if values.dim() != 1:
            raise ValueError("pair_bias_attention implicit-sample nested mask must have flattened packed storage")
        values = values.unsqueeze(1)
    elif values.dim() != 2:
        raise ValueError("pair_bias_attention nested mask must retain one static sample axis")
    mask_groups = values.shape[1]
    if grouped:
        if mask_groups != 1 and any(g != mask_groups for g in groups):
            raise ValueError("pair_bias_attention mask group axis must be shared or match S_i for every sample")
    elif mask_groups not in (1, groups[0]):
        raise ValueError("pair_bias_attention mask sample axis must be uniformly 1 or S")
    cells = [(a * m if pair else m) for a, m in zip(lq, lk)]
    if [b - a for a, b in zip(packed[:-1], packed[1:])] != cells:
        if pair:
            raise ValueError("pair_bias_attention pair mask query/key axes must match Q_i and K_i for every sample")
        raise ValueError("pair_bias_attention key mask lengths must match K_i per sample")
    total = values.shape[0]
    buf = (values.t() if mask_groups > 1 else values[:, 0]).contiguous().reshape(-1)  # [g][cell]
    s_g = total if mask_groups > 1 else 0
    cols = [(a, s_g, m if pair else 0) for a, m in zip(packed[:-1], lk)]
    return buf, cols


def _bias_plan(pair_bias, q: _Operand, k: _Operand):
    """Bias buffer ``[S|1][H][cells]`` and per-sample columns (pair_bias_attention.py:531-566,
    nested.py:96-118 and :450-462)."""

    if not pair_bias.batch_first:
        raise ValueError("pair_bias_attention nested pair_bias must be batch-first")
    rd, order, nd = tuple(pair_bias.ragged_dims), tuple(pair_bias.packed_dim_order), pair_bias.dim()
    implicit = nd == 4 and rd == (1, 2) and order == (1, 2, 0)
    explicit = nd == 5 and rd == (2, 3) and order == (2, 3, 0, 1)
    if not implicit and not explicit:
        raise unsupported(
            _OPERATOR,
            "requires a literal full-Q/K pair_bias with an implicit unit sample axis or uniform explicit "
            "sample/head sharing; per-element mixed S/H sharing and singleton Q/K broadcast are not served",
            ragged_dims=rd,
            packed_dim_order=order,
        )
    values = _core.kernel_operand(pair_bias.concat)
    if implicit:
        if values.dim() != 2 or values.shape[1] <= 0:
            raise ValueError("pair_bias_attention implicit-sample nested pair_bias must retain a positive head axis")
        values = values.unsqueeze(1)
    elif values.dim() != 3 or values.shape[1] <= 0 or values.shape[2] <= 0:
        raise ValueError("pair_bias_attention nested pair_bias must retain positive sample and head axes")
    bias_groups, bias_heads = values.shape[1], values.shape[2]
    grouped = q.kind in (GROUP_OUTER, TOKEN_OUTER, RAGGED_GROUPS)
    if grouped and bias_groups != 1:
        raise unsupported(_OPERATOR, "requires pair_bias shared across ragged attention groups")
    if not grouped and bias_groups not in (1, q.groups[0]):
        raise ValueError("pair_bias_attention pair_bias sample axis must be uniformly 1 or S")
    if bias_heads not in (1, q.heads):
        raise ValueError("pair_bias_attention pair_bias head axis must be uniformly 1 or H")
    packed = _offsets(pair_bias)
    if len(packed) != len(q.groups) + 1:
        raise ValueError("pair_bias_attention pair_bias must have one packed boundary per sample")
    if [b - a for a, b in zip(packed[:-1], packed[1:])] != [a * m for a, m in zip(q.lengths, k.lengths)]:
        raise ValueError("pair_bias_attention pair_bias query/key axes must match Q_i and K_i for every sample")
    cells = values.shape[0]
    # (cells, S|1, H|1) -> [S|1][H][cells]: heads expanded so every head owns its gradient cells
    buf = values.expand(cells, bias_groups, q.heads).permute(1, 2, 0).contiguous()
    s_g = q.heads * cells if bias_groups > 1 else 0
    cols = [(a, s_g, cells, m) for a, m in zip(packed[:-1], k.lengths)]
    return buf, cols, bias_groups == 1


def nested_pair_bias_attention(query, key, value, mask, pair_bias, scale: Optional[float]):
    q = _operand("query", query)
    k = q if key is query else _operand("key", key)
    v = q if value is query else k if value is key else _operand("value", value)
    require_no_forward_mode(_OPERATOR, q.values, k.values, v.values,
                            None if pair_bias is None else pair_bias.concat)  # fmt: skip
    if k.kind != q.kind or v.kind != q.kind:
        raise ValueError("pair_bias_attention nested Q/K/V must share their group packing")
    if (k.heads, k.head_size) != (q.heads, q.head_size) or (v.heads, v.head_size) != (q.heads, q.head_size):
        raise ValueError("pair_bias_attention nested Q/K/V must share group counts, heads, and channels")
    if len(k.groups) != len(q.groups) or len(v.groups) != len(q.groups):
        raise ValueError("pair_bias_attention query and key must contain the same number of samples")
    if k.groups != q.groups or v.groups != q.groups:
        raise ValueError("pair_bias_attention nested Q/K/V must share group counts, heads, and channels")
    if v.lengths != k.lengths or v.values.shape[0] != k.values.shape[0]:
        raise ValueError("pair_bias_attention value layout must match the key layout per sample")

    mask_buf, mask_cols = (None, None) if mask is None else _mask_plan(mask, q, k)
    if pair_bias is None:
        bias_buf, bias_cols, shared = None, None, True
    else:
        bias_buf, bias_cols, shared = _bias_plan(pair_bias, q, k)
    require_same_device(_OPERATOR, q.values, k.values, v.values, mask_buf, bias_buf)
    dtype = q.values.dtype
    autocast_f32 = (
        bias_buf is not None
        and dtype in _HALF
        and bias_buf.dtype == torch.float32
        and torch.is_autocast_enabled("cuda")
        and torch.get_autocast_dtype("cuda") == dtype
    )
    if (
        q.values.device.type != "cuda"
        or dtype not in _core.SUPPORTED_DTYPES
        or k.values.dtype != dtype
        or v.values.dtype != dtype
        or not (0 < q.head_size <= _core.MAX_HEAD_SIZE)
        or (bias_buf is not None and bias_buf.dtype != dtype and not autocast_f32)
    ):
        raise unsupported(
            _OPERATOR,
            "requires CUDA float16/bfloat16/float32 supported packed NestedTensor Q/K/V with "
            f"head_size <= {_core.MAX_HEAD_SIZE}, a matching bool key/pair mask, and a literal full-Q/K "
            "uniform sample/head pair bias in the Q/K/V dtype or matching-autocast float32",
            query=f"{tuple(q.values.shape)} {dtype} {q.values.device}",
            key=f"{tuple(k.values.shape)} {k.values.dtype}",
            pair_bias=None if bias_buf is None else f"{tuple(bias_buf.shape)} {bias_buf.dtype}",
        )
    table = plan_table(q, k, v, mask_cols, bias_cols, shared)
    lse_numel = sum(g * q.heads * n for g, n in zip(q.groups, q.lengths))
    scale = q.head_size**-0.5 if scale is None else float(scale)
    out = _core.attend(q.values, k.values, v.values, mask_buf, bias_buf, table, q.heads, scale, lse_numel)
    if out.shape != query.concat.shape:
        out = out.reshape(query.concat.shape)
    return query.packed_like(out)


def plan_table(q: _Operand, k: _Operand, v: _Operand, mask_cols: Optional[Sequence[tuple]],
               bias_cols: Optional[Sequence[tuple]], shared: bool) -> List[int]:  # fmt: skip
    """One geometry-table row per sample."""

    table: List[int] = []
    lse_off = 0
    for i, (g, lq, lk) in enumerate(zip(q.groups, q.lengths, k.lengths)):
        bias = None if bias_cols is None else bias_cols[i]
        table += _core.table_row(
            groups=g, len_q=lq, len_k=lk, q=q.cols[i], k=k.cols[i], v=v.cols[i], bias=bias, dbias=bias,
            bias_mode=(_lib.BIAS_SHARED if shared else _lib.BIAS_FULL) if bias is not None else _lib.BIAS_NONE,
            mask=None if mask_cols is None else mask_cols[i], lse_off=lse_off,
        )  # fmt: skip
        lse_off += g * q.heads * lq
    return table
