"""Custom ops and autograd around the C-ABI attention library.

Every front-end (dense triangle attention, nested triangle attention, MSA-row
pair-bias attention) lowers its call to the same two operators:

* ``oops_amd::attention_forward(q, k, v, mask, bias, table, ...) -> (out, lse)``
* ``oops_amd::attention_backward(dout, q, k, v, mask, bias, out, lse, table, ...)``

``table`` is the flattened int64 geometry table of ``include/oops_amd.h``
(``TABLE_WIDTH`` ints per sample), built from shapes and strides only, so the
ops are opaque to ``torch.compile`` and traceable under ``FakeTensorMode``.
The output, dQ, dK and dV are allocated with the strides of Q, K and V, so
their table columns are those of Q/K/V; dBias is a float32 buffer laid out as
the contiguous bias values.

This plays the role of the reference's ``triton_triangle_attention`` /
``_TriangleAttention`` and the ``ooperators::_triangle_attention_*`` custom ops
(oops/attention/triangle/triton/ops.py:102-423).
"""

from __future__ import annotations

import contextlib
import ctypes
from collections import OrderedDict
from typing import List, Optional, Sequence, Tuple

import torch
from torch import Tensor

from .. import _lib
from ._runtime import needs_custom_op, without_second_derivative

_DTYPE_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}
SUPPORTED_DTYPES = tuple(_DTYPE_CODE)
MAX_HEAD_SIZE = 256

# Backward kernels to run (OR of _lib.PHASE_*; 0 = all).  Only for profiling
# single kernels; see ``profile_phases``.
_PHASES = 0


class profile_phases:
    """Context manager restricting backward calls to a subset of kernels (profiling only)."""

    def __init__(self, phases: int):
        self.phases = phases

    def __enter__(self):
        global _PHASES
        self.saved, _PHASES = _PHASES, self.phases
        return self

    def __exit__(self, *exc):
        global _PHASES
        _PHASES = self.saved
        return False


_FORCE_GENERIC = 0


class force_generic:
    """Context manager routing calls to the generic kernels instead of the fast paths (testing)."""

    def __enter__(self):
        global _FORCE_GENERIC
        self.saved, _FORCE_GENERIC = _FORCE_GENERIC, 1
        return self

    def __exit__(self, *exc):
        global _FORCE_GENERIC
        _FORCE_GENERIC = self.saved
        return False


class separate_dkv_dbias:
    """Context manager keeping the 16-bit fast kernels but running dK/dV and the shared dBias in
    separate kernels instead of the fused one (testing)."""

    def __enter__(self):
        global _FORCE_GENERIC
        self.saved, _FORCE_GENERIC = _FORCE_GENERIC, 2
        return self

    def __exit__(self, *exc):
        global _FORCE_GENERIC
        _FORCE_GENERIC = self.saved
        return False


_DBIAS_SINK: Optional[list] = None


class capture_dbias_f32:
    """Context manager collecting each backward's float32 dBias (the kernels' output, before the
    cast to the bias dtype) in ``.values``, in call order (accuracy reporting and tests)."""

    def __enter__(self):
        global _DBIAS_SINK
        self.saved, _DBIAS_SINK = _DBIAS_SINK, []
        self.values = _DBIAS_SINK
        return self

    def __exit__(self, *exc):
        global _DBIAS_SINK
        _DBIAS_SINK = self.saved
        return False


# ----------------------------------------------------------------- tables

class _TableCache:
    """Least-recently-used cache of geometry tables, except that an entry used
    while the current stream is being captured into a graph is pinned for the
    life of the process: the graph holds the device copy's address and replays
    read it long after the call that built it."""

    def __init__(self, size: int, make):
        self.size = size
        self.make = make  # key -> (host copy, device copy)
        self.lru: "OrderedDict[tuple, tuple]" = OrderedDict()
        self.pinned: dict = {}

    def get(self, key: tuple, capturing: bool) -> tuple:
        hit = self.pinned.get(key)
        if hit is not None:
            return hit
        hit = self.lru.get(key)
        if hit is None:
            hit = self.make(key)
        else:
            del self.lru[key]
        if capturing:
            self.pinned[key] = hit
            return hit
        self.lru[key] = hit
        while len(self.lru) > self.size:
            self.lru.popitem(last=False)
        return hit


def _make_table(key: tuple) -> tuple:
    device = torch.device("cuda", key[0])
    host = torch.tensor(key[1], dtype=torch.int64).pin_memory()
    dev = torch.empty(host.shape, dtype=torch.int64, device=device)
    dev.copy_(host, non_blocking=True)
    # (host, device copy, streams the device copy is recorded on)
    return host, dev, {_stream(device)}


_TABLES = _TableCache(512, _make_table)


def device_table(table: Sequence[int], device: torch.device) -> tuple[Tensor, Tensor]:
    """(pinned host copy, device copy) of a geometry table, cached by value.

    The device copy is filled from pinned memory with an async copy, which is
    legal under CUDA-graph capture.  Entries are reused unchanged; one used
    under capture is never evicted, and the device copy is recorded on every
    stream that reads it, so its memory is not handed out again while a
    launch on another stream may still read it.
    """

    key = (device.index, tuple(map(int, table)))
    host, dev, streams = _TABLES.get(key, torch.cuda.is_current_stream_capturing())
    raw = _stream(device)
    if raw not in streams:
        dev.record_stream(torch.cuda.current_stream(device))
        streams.add(raw)
    return host, dev


def _vec_ok(table: Sequence[int], tensors: Sequence[Optional[Tensor]], bias: Optional[Tensor]) -> bool:
    """True when every row of every operand starts on a 16-byte boundary."""

    for t in (*tensors, bias):
        if t is not None and t.data_ptr() % 16:
            return False
    width = _lib.TABLE_WIDTH
    q = tensors[0]
    ce = 16 // q.element_size()
    cols = (
        _lib.T_Q_OFF, _lib.T_Q_SG, _lib.T_Q_SH, _lib.T_Q_SI,
        _lib.T_K_OFF, _lib.T_K_SG, _lib.T_K_SH, _lib.T_K_SI,
        _lib.T_V_OFF, _lib.T_V_SG, _lib.T_V_SH, _lib.T_V_SI,
        _lib.T_DO_OFF, _lib.T_DO_SG, _lib.T_DO_SH, _lib.T_DO_SI,
    )  # fmt: skip
    bce = 16 // bias.element_size() if bias is not None else 1
    bcols = (_lib.T_B_OFF, _lib.T_B_SG, _lib.T_B_SH, _lib.T_B_SI)
    for s in range(len(table) // width):
        row = table[s * width : (s + 1) * width]
        if any(int(row[c]) % ce for c in cols):
            return False
        if bias is not None and int(row[_lib.T_B_OFF]) >= 0 and any(int(row[c]) % bce for c in bcols):
            return False
    return True


def _geometry(q: Tensor, bias: Optional[Tensor], mask: Optional[Tensor], table: Sequence[int],
              num_heads: int, scale: float, vec_ok: bool) -> tuple[_lib.Geometry, tuple]:
    host, dev = device_table(table, q.device)
    geo = _lib.Geometry()
    geo.dtype = _DTYPE_CODE[q.dtype]
    geo.bias_dtype = _DTYPE_CODE[bias.dtype] if bias is not None else geo.dtype
    geo.num_heads = num_heads
    geo.head_size = q.shape[-1]
    geo.num_samples = len(table) // _lib.TABLE_WIDTH
    geo.has_bias = int(bias is not None)
    geo.has_mask = int(mask is not None)
    geo.vec_ok = int(vec_ok)
    geo.scale = float(scale)
    geo.phases = _PHASES
    geo.force_generic = _FORCE_GENERIC
    geo.table_host = host.data_ptr()
    geo.table_device = dev.data_ptr()
    return geo, (host, dev)


def _remap_dout(table: List[int], out: Tensor, dout: Tensor, num_heads: int) -> Optional[List[int]]:
    """``table`` with its dO columns rewritten for ``dout``'s strides, or None.

    The rows address the output (dense in some dimension order) as
    ``off + g*s_g + h*s_h + i*s_i + d``.  Each of those terms is decomposed
    into coordinates of the output's dimensions; when no row's index box
    carries across a dimension, the same coordinates give dO's offsets with
    dO's strides (zero strides of an expanded gradient included).  Returns
    None when that does not hold or dO's last dimension is not unit-stride.
    """

    if dout.shape != out.shape or out.dim() == 0 or (dout.size(-1) > 1 and dout.stride(-1) != 1):
        return None
    sizes, ost, dst = out.shape, out.stride(), dout.stride()
    order = sorted((d for d in range(out.dim()) if sizes[d] > 1), key=lambda d: -ost[d])
    expect = 1
    for d in reversed(order):  # dense, non-overlapping over the non-trivial dims
        if ost[d] != expect:
            return None
        expect *= sizes[d]

    def coords(x: int) -> Optional[List[int]]:
        c = []
        for d in order:
            q, x = divmod(x, ost[d])
            c.append(q)
        return c if x == 0 else None

    width = _lib.TABLE_WIDTH
    new = list(table)
    for s in range(len(table) // width):
        row = table[s * width : (s + 1) * width]
        counts = (1, row[_lib.T_GROUPS] - 1, num_heads - 1, row[_lib.T_LEN_Q] - 1)
        terms = row[_lib.T_O_OFF : _lib.T_O_OFF + 4]
        cols = []
        span = [0] * len(order)
        for value, n in zip(terms, counts):
            if n == 0:
                cols.append(0)
                continue
            c = coords(int(value))
            if c is None:
                return None
            for k in range(len(order)):
                span[k] += c[k] * n
            cols.append(sum(ck * dst[d] for ck, d in zip(c, order)))
        unit = coords(1)  # the head-dim step (d = 0 .. D-1)
        if unit is None:
            return None
        for k in range(len(order)):
            span[k] += unit[k] * (sizes[-1] - 1)
        if any(span[k] >= sizes[d] for k, d in enumerate(order)):
            return None
        new[s * width + _lib.T_DO_OFF : s * width + _lib.T_DO_OFF + 4] = cols
    return new


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(device: torch.device) -> int:
    """The raw handle of the device's current stream."""

    return torch._C._cuda_getCurrentRawStream(device.index)


def _on_device(device: torch.device):
    """The device context of a launch (a no-op when that device is already current)."""

    return contextlib.nullcontext() if device.index == torch.cuda.current_device() else torch.cuda.device(device)


# ----------------------------------------------------------------- ops


def _forward_impl(q: Tensor, k: Tensor, v: Tensor, mask: Optional[Tensor], bias: Optional[Tensor], table: List[int],
                  num_heads: int, scale: float, lse_numel: int, save_residual: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """The forward launch: (out, out_lo, lse)."""

    lib = _lib.load()
    out = torch.empty_strided(q.size(), q.stride(), dtype=q.dtype, device=q.device)
    out_lo = _residual_like(out, save_residual)
    lse = torch.empty(lse_numel, dtype=torch.float32, device=q.device)
    vec = _vec_ok(table, (q, k, v, out), bias)
    geo, keep = _geometry(q, bias, mask, table, num_heads, scale, vec)
    ws_bytes = lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with _on_device(q.device):
        rc = lib.oops_attn_forward(
            ctypes.byref(geo), _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(bias), _ptr(out), _ptr(out_lo),
            _ptr(lse), _ptr(workspace), ws_bytes, _stream(q.device),
        )
    _lib.check(rc, "attention forward")
    del keep
    return out, out_lo, lse


@torch.library.custom_op("oops_amd::attention_forward", mutates_args=(), device_types="cuda")
def attention_forward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Optional[Tensor],
    bias: Optional[Tensor],
    table: List[int],
    num_heads: int,
    scale: float,
    lse_numel: int,
    save_residual: bool,
) -> Tuple[Tensor, Tensor, Tensor]:
    return _forward_impl(q, k, v, mask, bias, table, num_heads, scale, lse_numel, save_residual)


def _residual_like(out: Tensor, save: bool) -> Tensor:
    """Buffer for out - round(out) (16-bit outputs of a differentiable call), else empty."""

    if save and out.dtype != torch.float32:
        return torch.empty_strided(out.size(), out.stride(), dtype=out.dtype, device=out.device)
    return out.new_empty(0)


@attention_forward.register_fake
def _(q, k, v, mask, bias, table, num_heads, scale, lse_numel, save_residual):
    out = torch.empty_strided(q.size(), q.stride(), dtype=q.dtype, device=q.device)
    return out, _residual_like(out, save_residual), q.new_empty(lse_numel, dtype=torch.float32)


def _backward_impl(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, mask: Optional[Tensor], bias: Optional[Tensor],
                   out: Tensor, out_lo: Tensor, lse: Tensor, table: List[int], num_heads: int, scale: float,
                   dbias_numel: int, needs: List[bool]) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """The backward launch: (dq, dk, dv, float32 dbias)."""

    lib = _lib.load()
    dout = dout.resolve_neg().resolve_conj()
    if dout.dtype != out.dtype:
        dout = dout.to(out.dtype)
    if dout.stride() != out.stride():
        # the kernels read dO through its own table columns: re-express them
        # for dO's strides, or copy dO into the output's layout
        remapped = _remap_dout(table, out, dout, num_heads)
        if remapped is None:
            dout = torch.empty_strided(out.size(), out.stride(), dtype=out.dtype, device=out.device).copy_(dout)
        else:
            table = remapped
    need_q, need_k, need_v, need_b = needs

    def like(t: Tensor, need: bool) -> Tensor:
        if not need:
            return t.new_empty(0)
        return torch.empty_strided(t.size(), t.stride(), dtype=t.dtype, device=t.device)

    dq, dk, dv = like(q, need_q), like(k, need_k), like(v, need_v)
    dbias = (
        torch.empty(dbias_numel, dtype=torch.float32, device=q.device)
        if need_b and bias is not None
        else q.new_empty(0, dtype=torch.float32)
    )
    vec = _vec_ok(table, (q, k, v, out, dout), bias)
    geo, keep = _geometry(q, bias, mask, table, num_heads, scale, vec)
    ws_bytes = lib.oops_attn_backward_workspace_bytes(ctypes.byref(geo))
    if ws_bytes == 0:
        _lib.check(1, "attention backward workspace sizing")
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with _on_device(q.device):
        rc = lib.oops_attn_backward(
            ctypes.byref(geo), _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(bias), _ptr(out), _ptr(out_lo),
            _ptr(lse), _ptr(dout), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dbias), _ptr(workspace), ws_bytes,
            _stream(q.device),
        )
    _lib.check(rc, "attention backward")
    del keep
    return dq, dk, dv, dbias


@torch.library.custom_op("oops_amd::attention_backward", mutates_args=(), device_types="cuda")
def attention_backward(
    dout: Tensor,
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Optional[Tensor],
    bias: Optional[Tensor],
    out: Tensor,
    out_lo: Tensor,
    lse: Tensor,
    table: List[int],
    num_heads: int,
    scale: float,
    dbias_numel: int,
    needs: List[bool],
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    return _backward_impl(dout, q, k, v, mask, bias, out, out_lo, lse, table, num_heads, scale, dbias_numel, needs)


@attention_backward.register_fake
def _(dout, q, k, v, mask, bias, out, out_lo, lse, table, num_heads, scale, dbias_numel, needs):
    def like(t, need):
        return torch.empty_strided(t.size(), t.stride(), dtype=t.dtype, device=t.device) if need else t.new_empty(0)

    need_q, need_k, need_v, need_b = needs
    dbias = q.new_empty(dbias_numel if (need_b and bias is not None) else 0, dtype=torch.float32)
    return like(q, need_q), like(k, need_k), like(v, need_v), dbias


def _save(ctx, q, k, v, mask, bias, table, num_heads, scale, out, out_lo, lse):
    ctx.save_for_backward(q, k, v, mask, bias, out, out_lo, lse)
    ctx.table = table
    ctx.num_heads = num_heads
    ctx.scale = scale
    ctx.bias_shape = None if bias is None else bias.shape
    ctx.bias_dtype = None if bias is None else bias.dtype
    ctx.set_materialize_grads(False)  # no zero-filled gradients for the residual and LSE outputs


def _setup_context(ctx, inputs, output):
    q, k, v, mask, bias, table, num_heads, scale, lse_numel, save_residual = inputs
    out, out_lo, lse = output
    _save(ctx, q, k, v, mask, bias, table, num_heads, scale, out, out_lo, lse)
    ctx.mark_non_differentiable(out_lo, lse)


def _backward(ctx, dout, dout_lo, dlse):
    return _grads(ctx, dout, attention_backward)


def _grads(ctx, dout, backward):
    """Gradients of (q, k, v, mask, bias, table, num_heads, scale, lse_numel, save_residual)."""

    q, k, v, mask, bias, out, out_lo, lse = ctx.saved_tensors
    need_q, need_k, need_v, _, need_b = ctx.needs_input_grad[:5]
    need_b = bool(need_b and bias is not None)
    if dout is None or not (need_q or need_k or need_v or need_b):
        return (None,) * 10
    dbias_numel = 0 if bias is None else bias.numel()
    dq, dk, dv, dbias = backward(
        dout, q, k, v, mask, bias, out, out_lo, lse, ctx.table, ctx.num_heads, ctx.scale, dbias_numel,
        [bool(need_q), bool(need_k), bool(need_v), need_b],
    )
    grad_bias = dbias.view(ctx.bias_shape).to(ctx.bias_dtype) if need_b else None
    if need_b and _DBIAS_SINK is not None:
        _DBIAS_SINK.append(dbias.view(ctx.bias_shape))
    return (
        dq if need_q else None,
        dk if need_k else None,
        dv if need_v else None,
        None,
        grad_bias,
        None,
        None,
        None,
        None,
        None,
    )


attention_forward.register_autograd(_backward, setup_context=_setup_context)


class _EagerAttention(torch.autograd.Function):
    """The same implementations as the custom ops, for eager calls: autograd
    calls the backward directly instead of through the operator dispatcher
    (about 100 us less host time per forward and backward on a slow host).
    Traced code (torch.compile) takes the custom ops."""

    @staticmethod
    def forward(ctx, q, k, v, mask, bias, table, num_heads, scale, lse_numel):
        out, out_lo, lse = _forward_impl(q, k, v, mask, bias, table, num_heads, scale, lse_numel, True)
        _save(ctx, q, k, v, mask, bias, table, num_heads, scale, out, out_lo, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        return without_second_derivative(_grads(ctx, dout, _backward_impl)[:9], ctx, dout)


# ----------------------------------------------------------------- table rows


def table_row(
    *,
    groups: int,
    len_q: int,
    len_k: int,
    q: Sequence[int],
    k: Sequence[int],
    v: Sequence[int],
    bias: Optional[Sequence[int]] = None,
    dbias: Optional[Sequence[int]] = None,
    bias_mode: int = _lib.BIAS_NONE,
    mask: Optional[Sequence[int]] = None,
    lse_off: int = 0,
) -> list:
    """One geometry-table row.  q/k/v/bias/dbias are (off, s_g, s_h, s_i); mask is (off, s_g, s_i).

    The output and dO columns repeat the query's, matching how the ops
    allocate the output.
    """

    row = [0] * _lib.TABLE_WIDTH
    row[_lib.T_GROUPS], row[_lib.T_LEN_Q], row[_lib.T_LEN_K] = groups, len_q, len_k
    row[_lib.T_Q_OFF : _lib.T_Q_OFF + 4] = list(q)
    row[_lib.T_K_OFF : _lib.T_K_OFF + 4] = list(k)
    row[_lib.T_V_OFF : _lib.T_V_OFF + 4] = list(v)
    row[_lib.T_O_OFF : _lib.T_O_OFF + 4] = list(q)
    row[_lib.T_DO_OFF : _lib.T_DO_OFF + 4] = list(q)
    row[_lib.T_B_OFF : _lib.T_B_OFF + 4] = list(bias) if bias is not None else [-1, 0, 0, 0]
    row[_lib.T_M_OFF : _lib.T_M_OFF + 3] = list(mask) if mask is not None else [-1, 0, 0]
    row[_lib.T_L_OFF] = lse_off
    row[_lib.T_DB_OFF : _lib.T_DB_OFF + 4] = list(dbias) if dbias is not None else [0, 0, 0, 0]
    row[_lib.T_BIAS_MODE] = bias_mode if bias is not None else _lib.BIAS_NONE
    return row


def kernel_operand(tensor: Optional[Tensor]) -> Optional[Tensor]:
    """Resolve lazy neg/conj view bits; raw pointers cannot observe them."""

    if tensor is None:
        return None
    return tensor.resolve_neg().resolve_conj()


def attend(q, k, v, mask, bias, table, num_heads, scale, lse_numel) -> Tensor:
    """Run the forward op (autograd-aware) and return the output tensor."""

    save = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, bias)
    )
    if needs_custom_op(q):
        out, _, _ = attention_forward(q, k, v, mask, bias, table, num_heads, scale, lse_numel, save)
    elif save:
        out = _EagerAttention.apply(q, k, v, mask, bias, table, num_heads, scale, lse_numel)
    else:
        out, _, _ = _forward_impl(q, k, v, mask, bias, table, num_heads, scale, lse_numel, False)
    return out
