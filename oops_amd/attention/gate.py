"""``gate_attention_output`` and ``gated_pair_bias_attention``: the gated output stage after attention.

Drop-in for the reference's operators
(oops/attention/gate/gate_attention_output.py:36-185 and
oops/attention/pair_bias/gated_pair_bias_attention.py:33-126):

    out = linear(round(sigmoid(linear(single, gate_weight))) * attention_flat, output_weight)

``attention`` is head-major ``(*prefix, H, Q, D)``; its ``(Q, H, D)`` view is
read in place through its strides (no transposed copy).  On the GPU the gate
projection, the sigmoid and the product run in one HIP kernel for 16-bit
operands (MFMA, the logits kept for the backward); other dtypes and layouts
compute the logits with ``F.linear`` and apply the gate with the HIP
elementwise kernel.  The output projection and the ``single``/``gate_weight``
gradients are plain GEMMs, as in the reference
(gate/triton/generic.py:265-327, gate/composed.py:31-53).  Where the reference
composes Torch operations instead of launching its kernel (CPU tensors,
mixed dtypes outside autocast, forward-mode AD, functorch transforms), so
does this module.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor
from torch.nn import functional as F

from .. import _lib
from .._errors import unsupported
from ._runtime import forward_mode_active, is_nested, require_no_forward_mode, require_same_device
from .pair_bias import pair_bias_attention

_OPERATOR = "gate_attention_output"
_DTYPE_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


# ----------------------------------------------------------------- C ABI


def _gate_geometry(att5: Tensor, single_rows: Optional[Tensor], weight: Optional[Tensor]) -> _lib.GateGeometry:
    b, s, t, h, d = att5.shape
    g = _lib.GateGeometry()
    g.dtype = _DTYPE_CODE[att5.dtype]
    g.heads, g.width = h, d
    g.channels = single_rows.shape[1] if single_rows is not None else 0
    g.rows = b * s * t
    g.tokens = max(t, 1)
    g.groups = max(s, 1)
    g.a_sb, g.a_sg, g.a_st, g.a_sh, g.a_sd = att5.stride()
    g.s_row = single_rows.stride(0) if single_rows is not None else 0
    g.w_row = weight.stride(0) if weight is not None else 0
    return g


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _fused_ok(att5: Tensor, single_rows: Tensor, weight: Tensor) -> bool:
    """Layouts the fused projection kernel takes (mirrors gate_projection_ok in gate.hip)."""

    if att5.dtype == torch.float32 or att5.shape[-1] % 16 or single_rows.shape[1] % 8:
        return False
    if att5.stride(-1) != 1 or single_rows.stride(1) != 1 or weight.stride(1) != 1:
        return False
    if single_rows.stride(0) % 8 or weight.stride(0) % 8 or any(s % 8 for s in att5.stride()[:4]):
        return False
    return all(t.data_ptr() % 16 == 0 for t in (att5, single_rows, weight))


@torch.library.custom_op("oops_amd::gate_forward", mutates_args=(), device_types="cuda")
def gate_forward(attention: Tensor, single: Tensor, weight: Tensor, save_logits: bool) -> Tuple[Tensor, Tensor]:
    """(gated, logits) for attention ``(B, S, Q, H, D)`` (any strides), single ``(rows, C)``, weight ``(H*D, C)``."""

    lib = _lib.load()
    rows = single.shape[0]
    n = weight.shape[0]
    gated = torch.empty(rows, n, dtype=attention.dtype, device=attention.device)
    with torch.cuda.device(attention.device):
        if _fused_ok(attention, single, weight):
            logits = torch.empty_like(gated) if save_logits else gated.new_empty(0)
            geo = _gate_geometry(attention, single, weight)
            rc = lib.oops_gate_projection_forward(
                ctypes.byref(geo), _ptr(single), _ptr(weight), _ptr(attention), _ptr(gated), _ptr(logits),
                _stream(attention.device),
            )
            _lib.check(rc, "gate projection")
        else:
            logits = F.linear(single, weight).contiguous()
            geo = _gate_geometry(attention, None, None)
            rc = lib.oops_gate_multiply_forward(
                ctypes.byref(geo), _ptr(attention), _ptr(logits), _ptr(gated), _stream(attention.device)
            )
            _lib.check(rc, "gate multiply")
            if not save_logits:
                logits = gated.new_empty(0)
    return gated, logits


@gate_forward.register_fake
def _(attention, single, weight, save_logits):
    gated = attention.new_empty(single.shape[0], weight.shape[0])
    return gated, (torch.empty_like(gated) if save_logits else gated.new_empty(0))


@torch.library.custom_op("oops_amd::gate_backward", mutates_args=(), device_types="cuda")
def gate_backward(
    grad: Tensor, attention: Tensor, logits: Tensor, need_attention: bool, need_logits: bool
) -> Tuple[Tensor, Tensor]:
    """(grad_attention, grad_logits), each ``(rows, H*D)`` or empty when not needed."""

    lib = _lib.load()
    grad = grad.contiguous()
    grad_attention = torch.empty_like(logits) if need_attention else logits.new_empty(0)
    grad_logits = torch.empty_like(logits) if need_logits else logits.new_empty(0)
    if need_attention or need_logits:
        geo = _gate_geometry(attention, None, None)
        with torch.cuda.device(attention.device):
            rc = lib.oops_gate_multiply_backward(
                ctypes.byref(geo), _ptr(attention), _ptr(logits), _ptr(grad), _ptr(grad_attention),
                _ptr(grad_logits), _stream(attention.device),
            )
        _lib.check(rc, "gate multiply backward")
    return grad_attention, grad_logits


@gate_backward.register_fake
def _(grad, attention, logits, need_attention, need_logits):
    return (
        torch.empty_like(logits) if need_attention else logits.new_empty(0),
        torch.empty_like(logits) if need_logits else logits.new_empty(0),
    )


def _weight_grad(g_rows: Tensor, x_rows: Tensor) -> Tensor:
    """``g^T x`` over a long row axis (weight gradients of the projections).

    The library picks a kernel for one (256 x rows) x (rows x 256) GEMM that
    leaves the GPU nearly idle (0.46 ms at rows = 196608); the same product as
    a batched GEMM over up to 64 row chunks with float32 partial products,
    summed in float32, rounds once at the end like the single GEMM.
    """

    rows = g_rows.shape[0]
    chunks = min(64, rows // 1024)
    if chunks < 2:
        return g_rows.t().mm(x_rows)
    g_rows, x_rows = g_rows.contiguous(), x_rows.contiguous()
    main = rows // chunks * chunks
    out = torch.bmm(
        g_rows[:main].view(chunks, main // chunks, -1).transpose(1, 2),
        x_rows[:main].view(chunks, main // chunks, -1),
        out_dtype=torch.float32,
    ).sum(0)
    if main < rows:
        out = out + g_rows[main:].t().float().mm(x_rows[main:].float())
    return out.to(g_rows.dtype)


class _OutputProjection(torch.autograd.Function):
    """``linear(gated, output_weight)`` whose weight gradient uses _weight_grad."""

    @staticmethod
    def forward(ctx, gated: Tensor, weight: Tensor) -> Tensor:
        ctx.save_for_backward(gated, weight)
        return F.linear(gated, weight)

    @staticmethod
    def backward(ctx, grad: Tensor):
        gated, weight = ctx.saved_tensors
        grad_gated = grad @ weight if ctx.needs_input_grad[0] else None
        grad_weight = None
        if ctx.needs_input_grad[1]:
            grad_weight = _weight_grad(grad.reshape(-1, grad.shape[-1]), gated.reshape(-1, gated.shape[-1]))
        return grad_gated, grad_weight


class _Relabel(torch.autograd.Function):
    """Value of ``values``, derivatives of ``source`` (double backward through composed ops)."""

    @staticmethod
    def forward(ctx, values: Tensor, source: Tensor) -> Tensor:
        return values.detach()

    @staticmethod
    def backward(ctx, grad: Tensor):
        return None, grad


def _setup_context(ctx, inputs, output):
    attention, single, weight, save_logits = inputs
    _gated, logits = output
    ctx.save_for_backward(attention, single, weight, logits)
    ctx.mark_non_differentiable(logits)
    ctx.set_materialize_grads(False)  # no zero-filled gradient for the logits output


def _backward(ctx, grad_gated, _grad_logits):
    if grad_gated is None:
        return None, None, None, None
    attention, single, weight, logits = ctx.saved_tensors
    need_att, need_single, need_weight = ctx.needs_input_grad[:3]
    need_logits = need_single or need_weight
    ga, gl = gate_backward(grad_gated, attention, logits, need_att, need_logits)
    if torch.is_grad_enabled():
        # differentiable backward: kernel values, derivatives of the composed form
        gate = torch.sigmoid(F.linear(single, weight) if need_logits else logits)
        if need_att:
            ga = _Relabel.apply(ga, grad_gated * gate)
        if need_logits:
            att_rows = attention.reshape(logits.shape)
            gl = _Relabel.apply(gl, torch.ops.aten.sigmoid_backward(grad_gated * att_rows, gate))
    grad_attention = ga.view(attention.shape) if need_att else None
    grad_single = gl @ weight if need_single else None
    grad_weight = _weight_grad(gl, single) if need_weight else None
    return grad_attention, grad_single, grad_weight, None


torch.library.register_autograd("oops_amd::gate_forward", _backward, setup_context=_setup_context)


# ----------------------------------------------------------------- front-end


def _check_gate_output(attention: Tensor, single: Tensor, gate_weight: Tensor, output_weight: Tensor) -> None:
    """Shape contract of the reference's _check_gate_output (gate/_contract.py:27-45)."""

    if attention.dim() not in (3, 4, 5):
        raise ValueError(
            "attention must have layout (num_heads, query_length, head_size) under optional batch and sample axes"
        )
    if single.dim() != attention.dim() - 1:
        raise ValueError("single must have layout (..., query_length, single_channels)")
    if gate_weight.dim() != 2 or output_weight.dim() != 2:
        raise ValueError("gate_weight and output_weight must be rank-2 matrices")
    *prefix, num_heads, query_length, head_size = attention.shape
    gate_channels = num_heads * head_size
    if tuple(single.shape[:-1]) != (*prefix, query_length):
        raise ValueError("single must share the attention leading axes and its query_length")
    if gate_weight.shape != (gate_channels, single.shape[-1]):
        raise ValueError("gate_weight must have shape (num_heads * head_size, single_channels)")
    if output_weight.shape[1] != gate_channels:
        raise ValueError("output_weight input channels must equal num_heads * head_size")


def _composed(att_qhd: Tensor, single: Tensor, gate_weight: Tensor) -> Tensor:
    """The reference's Torch composition (gate/composed.py:44-52), gated values ``(..., Q, H*D)``."""

    gate = torch.sigmoid(F.linear(single, gate_weight))
    return (gate.unflatten(-1, att_qhd.shape[-2:]) * att_qhd).flatten(-2)


def _kernel_eligible(att_qhd: Tensor, single: Tensor, gate_weight: Tensor) -> Tuple[bool, torch.dtype]:
    autocast = torch.is_autocast_enabled("cuda")
    dtype = torch.get_autocast_dtype("cuda") if autocast else single.dtype
    ok = (
        att_qhd.is_cuda
        and dtype in _DTYPE_CODE
        and att_qhd.dtype == dtype
        and (gate_weight.dtype == dtype or autocast)
        and single.dtype in _DTYPE_CODE
        and gate_weight.dtype in _DTYPE_CODE
        and att_qhd.shape[-1] > 0
        and att_qhd.shape[-2] > 0
        and single.shape[-1] > 0
        and not forward_mode_active(att_qhd, single, gate_weight)
    )
    try:
        ok = ok and not torch._C._are_functorch_transforms_active()
    except AttributeError:  # pragma: no cover
        pass
    return ok, dtype


def _gate_output(att_qhd: Tensor, single: Tensor, gate_weight: Tensor, output_weight: Tensor) -> Tensor:
    """The stage's output ``(*prefix, Q, O)`` for attention viewed ``(*prefix, Q, H, D)`` (prefix rank 1 or 2)."""

    ok, dtype = _kernel_eligible(att_qhd, single, gate_weight)
    if not ok:
        return F.linear(_composed(att_qhd, single, gate_weight), output_weight)
    gated = _gate_values(att_qhd, single, gate_weight, dtype)
    if not torch.is_grad_enabled() or output_weight.dtype != gated.dtype:
        return F.linear(gated, output_weight)
    return _OutputProjection.apply(gated, output_weight)


def _gate_values(att_qhd: Tensor, single: Tensor, gate_weight: Tensor, dtype: torch.dtype) -> Tensor:
    """Gated values ``(*prefix, Q, H*D)`` from the HIP kernels."""

    single = single if single.dtype == dtype else single.to(dtype)
    weight = gate_weight if gate_weight.dtype == dtype else gate_weight.to(dtype)
    att5 = att_qhd if att_qhd.dim() == 5 else att_qhd.unsqueeze(0)
    channels = single.shape[-1]
    single_rows = single.reshape(-1, channels)
    if single_rows.stride(1) != 1:
        single_rows = single_rows.contiguous()
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (att_qhd, single_rows, weight))
    gated, _ = gate_forward(att5, single_rows, weight, needs_grad)
    return gated.view(*att_qhd.shape[:-2], att_qhd.shape[-2] * att_qhd.shape[-1])


def gate_attention_output(attention, single, gate_weight: Tensor, output_weight: Tensor):
    r"""Apply a sigmoid gate and output projection to head-major attention values.

    Args:
        attention: Dense ``(*prefix, H, Q, D)`` values with rank 3, 4 or 5, or a
            ``NestedTensor`` of ``(H, Q_i, D)`` or ``(S, H, Q_i, D)`` elements.
        single: Gating input ``(*prefix, Q, C)`` or matching nested ``(Q_i, C)``
            or ``(S, Q_i, C)`` elements, on the attention device.
        gate_weight: ``(H * D, C)``.
        output_weight: ``(O, H * D)``.

    Returns ``linear(sigmoid(linear(single, gate_weight)) * attention_flat,
    output_weight)`` shaped ``(*prefix, Q, O)``; a nested result keeps the
    single topology with channel width ``O``.
    """

    if is_nested(attention):
        if not is_nested(single):
            raise ValueError("gate_attention_output nested attention requires a NestedTensor single")
        return _gate_nested(attention, single, gate_weight, output_weight)
    if is_nested(single):
        raise ValueError("gate_attention_output dense attention cannot use a NestedTensor single")
    _check_gate_output(attention, single, gate_weight, output_weight)
    require_same_device(_OPERATOR, attention, single, gate_weight, output_weight)
    if attention.dim() == 3:
        return gate_attention_output(attention.unsqueeze(0), single.unsqueeze(0), gate_weight, output_weight).squeeze(0)
    return _gate_output(attention.transpose(-3, -2), single, gate_weight, output_weight)


def _gate_nested(attention, single, gate_weight: Tensor, output_weight: Tensor):
    """Nested values with token-major packing (gate_attention_output.py:103-177)."""

    if not getattr(attention, "batch_first", True):
        raise ValueError("gate_attention_output nested attention must be batch-first")
    implicit_att = attention.dim() == 4 and tuple(attention.ragged_dims) == (1,) and tuple(
        attention.packed_dim_order) == (1, 0, 2)
    explicit_att = attention.dim() == 5 and tuple(attention.ragged_dims) == (2,) and tuple(
        attention.packed_dim_order) == (2, 0, 1, 3)
    if not implicit_att and not explicit_att:
        raise unsupported(
            _OPERATOR,
            "requires token-major nested attention elements shaped (H, N_i, D) or (S, H, N_i, D)",
            ragged_dims=attention.ragged_dims,
            packed_dim_order=attention.packed_dim_order,
        )
    if not getattr(single, "batch_first", True):
        raise ValueError("gate_attention_output nested single must be batch-first")
    implicit_single = single.dim() == 3 and tuple(single.ragged_dims) == (0,) and tuple(single.packed_dim_order) == (
        0, 1)
    explicit_single = single.dim() == 4 and tuple(single.ragged_dims) == (1,) and tuple(
        single.packed_dim_order) == (1, 0, 2)
    if not implicit_single and not explicit_single:
        raise unsupported(
            _OPERATOR,
            "requires token-major nested single elements shaped (N_i, C) or (S, N_i, C)",
            ragged_dims=single.ragged_dims,
            packed_dim_order=single.packed_dim_order,
        )
    if implicit_att != implicit_single:
        raise ValueError("gate_attention_output nested single and attention must both include or omit S")
    att = attention.concat
    sgl = single.concat
    if implicit_att:
        if att.dim() != 3 or sgl.dim() != 2:
            raise ValueError("gate_attention_output implicit-sample nested packed values have invalid ranks")
        att, sgl = att.unsqueeze(1), sgl.unsqueeze(1)
    elif att.dim() != 4 or sgl.dim() != 3:
        raise ValueError("gate_attention_output explicit-sample nested packed values have invalid ranks")
    num_groups, num_heads, head_size = att.shape[1:]
    if sgl.shape[1] != num_groups:
        raise ValueError("gate_attention_output nested single and attention must share S")
    if gate_weight.dim() != 2 or output_weight.dim() != 2:
        raise ValueError("gate_weight and output_weight must be rank-2 matrices")
    gate_channels = num_heads * head_size
    if tuple(gate_weight.shape) != (gate_channels, sgl.shape[-1]):
        raise ValueError("gate_weight must have shape (num_heads * head_size, single_channels)")
    if output_weight.shape[1] != gate_channels:
        raise ValueError("output_weight input channels must equal num_heads * head_size")
    require_same_device(_OPERATOR, att, sgl, gate_weight, output_weight)
    a_off = attention.packed_offsets(dtype=torch.int64)
    s_off = single.packed_offsets(dtype=torch.int64)
    if a_off.shape != s_off.shape or not torch.equal(a_off.cpu(), s_off.cpu()) or att.shape[0] != sgl.shape[0]:
        raise ValueError("gate_attention_output nested single and attention must share their token topology")
    # packed (tokens, S, H, D) values read as a dense (prefix = tokens, Q = S, H, D)
    # problem: the gate acts on each (token, s) row independently
    out = _gate_output(att, sgl, gate_weight, output_weight)  # (tokens, S, O)
    if implicit_single:
        out = out.squeeze(1)
    return single.packed_with_static_tail(out)


def gated_pair_bias_attention(
    single,
    query,
    key,
    value,
    mask=None,
    pair_bias=None,
    gate_weight: Optional[Tensor] = None,
    output_weight: Optional[Tensor] = None,
    *,
    scale: Optional[float] = None,
):
    r"""Pair-bias attention, sigmoid gating and an output projection.

    Composes ``pair_bias_attention`` with ``gate_attention_output``
    (reference: oops/attention/pair_bias/gated_pair_bias_attention.py:33-126).
    ``pair_bias``, ``gate_weight`` and ``output_weight`` are required.
    """

    if pair_bias is None:
        raise ValueError("pair_bias is required")
    if gate_weight is None:
        raise ValueError("gate_weight is required")
    if output_weight is None:
        raise ValueError("output_weight is required")
    if (type(query) is not Tensor or type(single) is not Tensor) and is_nested(query) != is_nested(single):
        raise ValueError("gated_pair_bias_attention query and single must both be dense or both NestedTensor")
    unpack = (lambda t: t.concat if is_nested(t) else t)
    require_no_forward_mode("gated_pair_bias_attention", *(unpack(t) for t in (query, key, value, pair_bias)))
    require_same_device(
        "gated_pair_bias_attention",
        *(unpack(t) for t in (query, key, value, mask, pair_bias, single)),
        gate_weight,
        output_weight,
    )
    attention = pair_bias_attention(query, key, value, mask, pair_bias, scale=scale)
    return gate_attention_output(attention, single, gate_weight, output_weight)
