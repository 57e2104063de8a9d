"""``triangle_multiplication``: the incoming / outgoing triangle multiplicative update.

Drop-in for the reference's operator
(oops/pair/triangle_multiplication/triangle_multiplication.py:42-443):

    xn    = LayerNorm_C(pair)
    left  = mask * (xn W_lv^T + b_lv) * sigmoid(xn W_lg^T + b_lg)     (right likewise)
    X[i,j] = sum_k left[i,k] right[j,k]   (outgoing)  or  sum_k left[k,i] right[k,j]   (incoming)
    out   = (LayerNorm_H(X) W_o^T + b_o) * sigmoid(xn W_og^T + b_og)

per hidden channel and prefix element.  The pipeline is the reference's
(triton/generic.py:111-200, 657-1092): the input LayerNorm, the two gated
factor projections (one fused MFMA kernel writing the channel-major factors),
the contraction as a batched GEMM per (group, channel) on the factors in
place, the channel-major output LayerNorm and the fused gated output
projection are HIP kernels behind the ``oops_layer_norm_rows_*`` /
``oops_trimul_*`` C entry points; the backward recomputes the projections in
the same kernels and uses library GEMMs for the weight and input gradients.
Nested (DanLing) pairs run every ragged ``N_i x N_i`` block of the packed
values through the same kernels, with one GEMM batch per element for the
contraction.
"""

from __future__ import annotations

import ctypes
from typing import List, Literal, Optional, Sequence, Tuple

import torch
from torch import Tensor
from torch.nn import functional as F

from .. import _lib
from .._errors import unsupported
from .._partials import PartialSums
from ..attention._runtime import (
    is_nested,
    needs_custom_op,
    require_no_forward_mode,
    require_same_device,
    without_second_derivative,
)

_OPERATOR = "triangle_multiplication"
_KERNEL_DTYPES = (torch.bfloat16, torch.float16)
_SERVED_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_DTYPE_CODE = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}
MAX_FUSED_WIDTH = 1024

_WEIGHT_NAMES = (
    "input_norm_weight",
    "input_norm_bias",
    "left_value_weight",
    "left_gate_weight",
    "right_value_weight",
    "right_gate_weight",
    "output_norm_weight",
    "output_norm_bias",
    "output_weight",
    "output_gate_weight",
)
_BIAS_NAMES = ("left_value_bias", "left_gate_bias", "right_value_bias", "right_gate_bias", "output_bias",
               "output_gate_bias")  # fmt: skip


def triangle_multiplication(
    pair,
    pair_mask=None,
    *,
    direction: Literal["incoming", "outgoing"] = "outgoing",
    input_norm_weight: Tensor,
    input_norm_bias: Tensor,
    left_value_weight: Tensor,
    left_gate_weight: Tensor,
    right_value_weight: Tensor,
    right_gate_weight: Tensor,
    output_norm_weight: Tensor,
    output_norm_bias: Tensor,
    output_weight: Tensor,
    output_gate_weight: Tensor,
    left_value_bias: Optional[Tensor] = None,
    left_gate_bias: Optional[Tensor] = None,
    right_value_bias: Optional[Tensor] = None,
    right_gate_bias: Optional[Tensor] = None,
    output_bias: Optional[Tensor] = None,
    output_gate_bias: Optional[Tensor] = None,
    input_norm_eps: float = 1e-5,
    output_norm_eps: float = 1e-5,
):
    r"""Incoming or outgoing triangle multiplicative update of pair features.

    Args:
        pair: dense ``(*prefix, N, N, C)`` or a DanLing ``NestedTensor`` with
            ``(*prefix, N_i, N_i, C)`` elements.
        pair_mask: optional multiplicative mask broadcastable to ``(*prefix, N, N)``
            (or matching nested elements); floating masks are differentiable.
        direction: ``"outgoing"`` (``X[i,j] = sum_k left[i,k] right[j,k]``) or
            ``"incoming"`` (``X[i,j] = sum_k left[k,i] right[k,j]``).
        input_norm_weight, input_norm_bias: ``(C,)``; output_norm_weight,
            output_norm_bias: ``(H,)``; projections ``(H, C)``; output_weight
            ``(C, H)``; output_gate_weight ``(C, C)``; optional biases of the
            projections' output widths.

    Returns the update with the pair's shape and dtype (no residual added).
    """

    if direction not in ("incoming", "outgoing"):
        raise ValueError("direction must be 'incoming' or 'outgoing'")
    weights = (input_norm_weight, input_norm_bias, left_value_weight, left_gate_weight, right_value_weight,
               right_gate_weight, output_norm_weight, output_norm_bias, output_weight, output_gate_weight)  # fmt: skip
    biases = (left_value_bias, left_gate_bias, right_value_bias, right_gate_bias, output_bias, output_gate_bias)
    if is_nested(pair):
        if pair_mask is not None and not is_nested(pair_mask):
            raise ValueError("triangle_multiplication pair and pair_mask must both use the same NestedTensor layout")
        return _nested(pair, pair_mask, direction, weights, biases, input_norm_eps, output_norm_eps)
    if is_nested(pair_mask):
        raise ValueError("triangle_multiplication pair and pair_mask must both use the same NestedTensor layout")
    require_no_forward_mode(_OPERATOR, pair, pair_mask, *weights, *biases)
    _check_shapes(pair, pair_mask, weights)
    _check_bias_shapes(pair.shape[-1], weights[2].shape[0], biases)
    require_same_device(_OPERATOR, pair, pair_mask, *weights, *biases)
    pair, weights, biases = _prepare_autocast(pair, weights, biases)
    n = pair.shape[-2]
    grouped = pair.reshape(-1, n * n, pair.shape[-1])
    mask = None
    if pair_mask is not None:
        mask = pair_mask.to(torch.float32) if not pair_mask.is_floating_point() else pair_mask
        mask = mask.expand(pair.shape[:-1]).reshape(grouped.shape[:2])
    blocks = [(0, n)]
    out = _run(grouped, mask, blocks, direction, weights, biases, input_norm_eps, output_norm_eps)
    return out.reshape(pair.shape)


# ----------------------------------------------------------------- contracts


def _broadcasts_to(shape, target) -> bool:
    return len(shape) <= len(target) and all(s in (1, t) for s, t in zip(reversed(shape), reversed(target)))


def _check_weight_shapes(pair_size: int, weights: Sequence[Tensor]) -> None:
    """triangle_multiplication.py:426-443."""

    hidden = weights[2].shape[0]
    projection = (hidden, pair_size)
    expected = ((pair_size,), (pair_size,), projection, projection, projection, projection, (hidden,), (hidden,),
                (pair_size, hidden), (pair_size, pair_size))  # fmt: skip
    for name, weight, shape in zip(_WEIGHT_NAMES, weights, expected):
        if tuple(weight.shape) != shape:
            raise ValueError(f"{name} must have shape {shape}; got {tuple(weight.shape)}")


def _check_shapes(pair: Tensor, pair_mask: Optional[Tensor], weights) -> None:
    """triangle_multiplication.py:403-415."""

    if pair.dim() < 3:
        raise ValueError(f"pair must have shape (..., N, N, pair_size); got rank {pair.dim()}")
    if pair.shape[-2] != pair.shape[-3]:
        raise ValueError(f"pair token dims must be square (N, N); got {tuple(pair.shape[-3:-1])}")
    if pair_mask is not None and not _broadcasts_to(pair_mask.shape, pair.shape[:-1]):
        raise ValueError(
            f"pair_mask shape {tuple(pair_mask.shape)} must broadcast to pair[..., N, N] = {tuple(pair.shape[:-1])}"
        )
    _check_weight_shapes(pair.shape[-1], weights)


def _check_bias_shapes(pair_size: int, hidden: int, biases) -> None:
    """triangle_multiplication.py:396-400."""

    widths = (hidden, hidden, hidden, hidden, pair_size, pair_size)
    for name, bias, width in zip(_BIAS_NAMES, biases, widths):
        if bias is not None and tuple(bias.shape) != (width,):
            raise ValueError(f"{name} must have shape {(width,)}; got {tuple(bias.shape)}")


def _prepare_autocast(pair: Tensor, weights, biases):
    """Inside CUDA autocast the pair and projections take the autocast dtype
    (triangle_multiplication.py:296-316)."""

    if pair.is_cuda and torch.is_autocast_enabled("cuda"):
        dtype = torch.get_autocast_dtype("cuda")
        pair = pair.to(dtype)
        weights = tuple(w.to(dtype) if i in (2, 3, 4, 5, 8, 9) else w for i, w in enumerate(weights))
        biases = tuple(None if b is None else b.to(dtype) for b in biases)
    return pair, weights, biases


def _describe(t: Optional[Tensor]) -> Optional[str]:
    return None if t is None else f"{tuple(t.shape)} {t.dtype} {t.device}"


def _admit(pair: Tensor, weights, biases) -> None:
    """Admission rules of supports_triangle_multiplication (triton/ops.py:68-103)."""

    hidden = weights[2].shape[0]
    affine = (weights[6], weights[7])
    ok = (
        pair.is_cuda
        and pair.dtype in _SERVED_DTYPES
        and 0 < pair.shape[-1] <= MAX_FUSED_WIDTH
        and 0 < hidden <= MAX_FUSED_WIDTH
        and all(w.device == pair.device for w in weights)
        and all(weights[i].dtype == pair.dtype for i in (2, 3, 4, 5, 8, 9))
        and weights[0].dtype in (pair.dtype, torch.float32)
        and weights[1].dtype == weights[0].dtype
        and affine[0].dtype == affine[1].dtype
        and affine[0].dtype in (pair.dtype, torch.float32)
    )
    if not ok:
        raise unsupported(
            _OPERATOR,
            "requires a CUDA float16/bfloat16/float32 pair, channel widths within the fused launch domain, and weights on "
            "the pair's device in the pair's dtype (float32 allowed for the two LayerNorms)",
            pair=_describe(pair),
            hidden_size=hidden,
            weight_dtypes=tuple(sorted({str(w.dtype) for w in weights})),
        )
    for name, b in zip(_BIAS_NAMES, biases):
        if b is not None and b.dtype != pair.dtype:
            raise unsupported(_OPERATOR, "requires projection biases in the pair's dtype", bias=name,
                              operand=_describe(b))  # fmt: skip


# ----------------------------------------------------------------- execution


def _round8(x: int) -> int:
    return (x + 7) // 8 * 8


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _long_k_partials(a: Tensor, b: Tensor) -> Tensor:
    """float32 partial products of ``a (M, K) @ b (K, N)`` for a long K (weight gradients over every pair
    cell), (parts, M, N): their sum is the product.

    K is split into up to 64 chunks as one batched GEMM with float32 outputs (the library's single GEMM of
    this shape leaves most of the GPU idle); a remainder of K past the chunks is one more part.
    """

    k = a.shape[1]
    chunks = min(64, k // 1024)
    if chunks < 2:
        return a.float().mm(b.float())[None]
    main = k // chunks * chunks
    step = main // chunks
    a_c = a[:, :main].unflatten(1, (chunks, step)).transpose(0, 1)  # (chunks, M, step), strided view
    b_c = b[:main].view(chunks, step, b.shape[1]) if b.is_contiguous() else b[:main].reshape(chunks, step, -1)
    parts = torch.bmm(a_c, b_c, out_dtype=torch.float32)
    if main < k:
        parts = torch.cat([parts, a[:, main:].float().mm(b[main:].float())[None]])
    return parts


def _column_partials(x: Tensor) -> Tensor:
    """float32 partial column sums of ``x (K, N)`` (bias gradients), (parts, 1, N): a ones-row GEMM with
    float32 outputs, faster than a float32 reduction of the 16-bit rows."""

    return _long_k_partials(x.new_ones(1, x.shape[0]), x)


def _geometry(pair: Tensor, hidden: int, has_mask: bool, eps: float) -> _lib.TrimulGeometry:
    g = _lib.TrimulGeometry()
    g.dtype = _DTYPE_CODE[pair.dtype]
    g.channels = pair.shape[-1]
    g.hidden = hidden
    g.has_mask = int(has_mask)
    g.groups, g.positions = pair.shape[0], pair.shape[1]
    g.c_row = _round8(g.channels)
    g.h_row = _round8(hidden)
    g.eps = float(eps)
    return g


def _row_geometry(dtype, rows: int, width: int, x_row: int, y_row: int, eps: float) -> _lib.RowNormGeometry:
    g = _lib.RowNormGeometry()
    g.dtype = _DTYPE_CODE[dtype]
    g.width, g.rows, g.x_row, g.y_row, g.eps = width, rows, x_row, y_row, float(eps)
    return g


def _contract(factors: Tensor, out: Tensor, blocks, direction: str, grad: bool = False, grad_out=None) -> None:
    """Per (group, channel) and ragged block: out = L R^T (outgoing) or L^T R (incoming)."""

    G, H = factors.shape[1], factors.shape[2]
    whole = len(blocks) == 1 and blocks[0][1] ** 2 == factors.shape[3]
    with torch.autocast("cuda", enabled=False):
        if whole and not grad:
            n = blocks[0][1]
            left, right = factors[0].view(G * H, n, n), factors[1].view(G * H, n, n)
            if direction == "outgoing":
                torch.bmm(left, right.transpose(1, 2), out=out.view(G * H, n, n))
            else:
                torch.bmm(left.transpose(1, 2), right, out=out.view(G * H, n, n))
            return
        if whole:
            n = blocks[0][1]
            left, right = factors[0].view(G * H, n, n), factors[1].view(G * H, n, n)
            dx = grad_out.view(G * H, n, n)
            d_left, d_right = out[0].view(G * H, n, n), out[1].view(G * H, n, n)
            if direction == "outgoing":
                torch.bmm(dx, right, out=d_left)
                torch.bmm(dx.transpose(1, 2), left, out=d_right)
            else:
                torch.bmm(right, dx.transpose(1, 2), out=d_left)
                torch.bmm(left, dx, out=d_right)
            return
        for off, n in blocks:
            cells = slice(off, off + n * n)
            left = factors[0, :, :, cells].reshape(G * H, n, n)
            right = factors[1, :, :, cells].reshape(G * H, n, n)
            if not grad:
                res = torch.bmm(left, right.transpose(1, 2)) if direction == "outgoing" else torch.bmm(
                    left.transpose(1, 2), right)  # fmt: skip
                out[:, :, cells].copy_(res.view(G, H, n * n))
                continue
            dx = grad_out[:, :, cells].reshape(G * H, n, n)
            if direction == "outgoing":  # X = L R^T: dL = dX R, dR = dX^T L
                d_left, d_right = torch.bmm(dx, right), torch.bmm(dx.transpose(1, 2), left)
            else:  # X = L^T R: dL = R dX^T, dR = L dX
                d_left, d_right = torch.bmm(right, dx.transpose(1, 2)), torch.bmm(left, dx)
            out[0, :, :, cells].copy_(d_left.view(G, H, n * n))
            out[1, :, :, cells].copy_(d_right.view(G, H, n * n))


def _pairs(blocks: List[int]):
    return [(blocks[i], blocks[i + 1]) for i in range(0, len(blocks), 2)]


# The small float32 parameters travel as one buffer ``small`` with ``spans`` = [start, end] per entry of
# _SMALL (-1, -1 when absent): one operand and one gradient instead of seven slices, whose separate
# gradients autograd would each scatter into a zero-filled copy of the buffer.
_SMALL = ("b4", "bo", "bog", "in_w", "in_b", "on_w", "on_b")


def _small_views(small: Tensor, spans: List[int]) -> List[Optional[Tensor]]:
    return [None if spans[2 * i] < 0 else small[spans[2 * i] : spans[2 * i + 1]] for i in range(len(_SMALL))]


def _forward_impl(pair: Tensor, mask: Optional[Tensor], w_cat: Tensor, wo: Tensor, wog: Tensor, small: Tensor,
                  spans: List[int], blocks: List[int], direction: str, eps_in: float, eps_out: float):
    """Forward on prepared operands: pair (G, P, C); float32 mask (G, P); w_cat [4H][c_row]; wo [C][h_row];
    wog [C][c_row]; the float32 biases and LayerNorm affines in ``small`` (``spans``).  Returns (out, xn,
    mean_in, rstd_in, factors, combined, nrm, mean_out, rstd_out); all but ``out`` are kept for the backward."""

    b_cat, bo, bog, in_w, in_b, on_w, on_b = _small_views(small, spans)
    lib = _lib.load()
    G, P, C = pair.shape
    H = w_cat.shape[0] // 4
    R = G * P
    dtype, dev = pair.dtype, pair.device
    geo = _geometry(pair, H, mask is not None, eps_out)
    cp, hp = geo.c_row, geo.h_row
    stream = _stream(dev)
    with torch.cuda.device(dev):
        xn = torch.empty(R, cp, dtype=dtype, device=dev)
        mean_in = torch.empty(R, dtype=torch.float32, device=dev)
        rstd_in = torch.empty_like(mean_in)
        rg = _row_geometry(dtype, R, C, C, cp, eps_in)
        _lib.check(lib.oops_layer_norm_rows_forward(ctypes.byref(rg), _ptr(pair), _ptr(in_w), _ptr(in_b), _ptr(xn),
                                                    _ptr(mean_in), _ptr(rstd_in), stream),
                   "triangle_multiplication input LayerNorm")  # fmt: skip
        factors = torch.empty(2, G, H, P, dtype=dtype, device=dev)
        _lib.check(lib.oops_trimul_factors_forward(ctypes.byref(geo), _ptr(xn), _ptr(w_cat), _ptr(b_cat),
                                                   _ptr(mask), _ptr(factors), stream),
                   "triangle_multiplication factors")  # fmt: skip
        combined = torch.empty(G, H, P, dtype=dtype, device=dev)
        _contract(factors, combined, _pairs(blocks), direction)
        nrm = torch.empty(R, hp, dtype=dtype, device=dev)
        mean_out = torch.empty(R, dtype=torch.float32, device=dev)
        rstd_out = torch.empty_like(mean_out)
        _lib.check(lib.oops_trimul_output_norm_forward(ctypes.byref(geo), _ptr(combined), _ptr(on_w), _ptr(on_b),
                                                       _ptr(nrm), _ptr(mean_out), _ptr(rstd_out), stream),
                   "triangle_multiplication output LayerNorm")  # fmt: skip
        out = torch.empty(G, P, C, dtype=dtype, device=dev)
        _lib.check(lib.oops_trimul_output_forward(ctypes.byref(geo), _ptr(nrm), _ptr(xn), _ptr(wo), _ptr(wog),
                                                  _ptr(bo), _ptr(bog), _ptr(out), stream),
                   "triangle_multiplication output")  # fmt: skip
    return out, xn, mean_in, rstd_in, factors, combined, nrm, mean_out, rstd_out


@torch.library.custom_op("oops_amd::trimul_forward", mutates_args=(), device_types="cuda")
def trimul_forward(
    pair: Tensor,
    mask: Optional[Tensor],
    w_cat: Tensor,
    wo: Tensor,
    wog: Tensor,
    small: Tensor,
    spans: List[int],
    blocks: List[int],
    direction: str,
    eps_in: float,
    eps_out: float,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    return _forward_impl(pair, mask, w_cat, wo, wog, small, spans, blocks, direction, eps_in, eps_out)


@trimul_forward.register_fake
def _(pair, mask, w_cat, wo, wog, small, spans, blocks, direction, eps_in, eps_out):
    G, P, C = pair.shape
    H = w_cat.shape[0] // 4
    R = G * P
    f32 = dict(dtype=torch.float32, device=pair.device)
    return (pair.new_empty(G, P, C), pair.new_empty(R, w_cat.shape[1]), pair.new_empty(R, **f32),
            pair.new_empty(R, **f32), pair.new_empty(2, G, H, P), pair.new_empty(G, H, P),
            pair.new_empty(R, wo.shape[1]), pair.new_empty(R, **f32), pair.new_empty(R, **f32))  # fmt: skip


def _backward_impl(dout: Tensor, pair: Tensor, mask: Optional[Tensor], w_cat: Tensor, wo: Tensor, wog: Tensor,
                   small: Tensor, spans: List[int], xn: Tensor, mean_in: Tensor, rstd_in: Tensor, factors: Tensor,
                   combined: Tensor, nrm: Tensor, mean_out: Tensor, rstd_out: Tensor, blocks: List[int],
                   direction: str, eps_in: float, eps_out: float, need_mask: bool):  # fmt: skip
    """Gradients of the prepared operands: (pair, mask, w_cat, wo, wog, small); the mask gradient is empty
    when not needed."""

    b_cat, bo, bog, in_w, _in_b, on_w, _on_b = _small_views(small, spans)
    d_small = torch.empty_like(small)
    d_views = _small_views(d_small, spans)
    lib = _lib.load()
    G, P, C = pair.shape
    H = factors.shape[2]
    R = G * P
    dtype, dev = pair.dtype, pair.device
    geo = _geometry(pair, H, mask is not None, eps_out)
    cp, hp = geo.c_row, geo.h_row
    stream = _stream(dev)
    dout = dout.resolve_neg().to(dtype).contiguous()

    def empty():  # a fresh tensor per absent gradient: custom-op outputs may not alias
        return pair.new_empty(0, dtype=torch.float32)

    with torch.cuda.device(dev):
        g_val = torch.empty(R, cp, dtype=dtype, device=dev)
        g_gate = torch.empty(R, cp, dtype=dtype, device=dev)
        _lib.check(lib.oops_trimul_output_backward(ctypes.byref(geo), _ptr(nrm), _ptr(xn), _ptr(wo), _ptr(wog),
                                                   _ptr(bo), _ptr(bog), _ptr(dout), _ptr(g_val), _ptr(g_gate),
                                                   stream),
                   "triangle_multiplication output backward")  # fmt: skip
        gv, gg = g_val[:, :C], g_gate[:, :C]
        # every float32 partial (K-chunk products, per-workgroup sums) is summed by one launch at the end
        sums = PartialSums()
        parts = lib.oops_trimul_output_grad_parts(ctypes.byref(geo))
        if parts:
            # C = H = 128: one pass over each gradient gives its GEMM with the weight, its weight-gradient
            # and bias-gradient partials (oops_trimul_output_grad_products)
            d_nrm = torch.empty(R, H, dtype=dtype, device=dev)
            d_xn = torch.empty(R, C, dtype=dtype, device=dev)
            g_parts = torch.empty(2, parts, C, C, dtype=torch.float32, device=dev)
            s_parts = torch.empty(2, parts, C, dtype=torch.float32, device=dev)
            for i, (x, w, y, d) in enumerate(((g_val, wo, nrm, d_nrm), (g_gate, wog, xn, d_xn))):
                _lib.check(lib.oops_trimul_output_grad_products(
                    ctypes.byref(geo), _ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(y), y.stride(0), _ptr(d),
                    d.stride(0), _ptr(g_parts[i]), _ptr(s_parts[i]), stream), "triangle_multiplication output gradients")  # fmt: skip
            d_wo, d_wog = sums.add(g_parts[0], dtype), sums.add(g_parts[1], dtype)
            if bo is not None:
                sums.add(s_parts[0], out=d_views[1])
            if bog is not None:
                sums.add(s_parts[1], out=d_views[2])
        else:
            d_nrm = gv.mm(wo[:, :H]).contiguous()  # (R, H)
            d_xn = gg.mm(wog[:, :C])  # (R, C)
            d_wo = sums.add(_long_k_partials(gv.t(), nrm[:, :H]), dtype)
            d_wog = sums.add(_long_k_partials(gg.t(), xn[:, :C]), dtype)
            if bo is not None:
                sums.add(_column_partials(gv), out=d_views[1])
            if bog is not None:
                sums.add(_column_partials(gg), out=d_views[2])

        d_comb = torch.empty(G, H, P, dtype=dtype, device=dev)
        on_parts = torch.empty(2, lib.oops_trimul_output_norm_parts(ctypes.byref(geo)), H, dtype=torch.float32,
                               device=dev)  # fmt: skip
        _lib.check(lib.oops_trimul_output_norm_backward(ctypes.byref(geo), _ptr(combined), _ptr(on_w),
                                                        _ptr(mean_out), _ptr(rstd_out), _ptr(d_nrm), _ptr(d_comb),
                                                        _ptr(on_parts[0]), _ptr(on_parts[1]), stream),
                   "triangle_multiplication output LayerNorm backward")  # fmt: skip
        d_factors = torch.empty_like(factors)
        _contract(factors, d_factors, _pairs(blocks), direction, grad=True, grad_out=d_comb)
        d_proj = torch.empty(4 * H, R, dtype=dtype, device=dev)
        want_mask = mask is not None and need_mask
        mparts = torch.empty(lib.oops_trimul_mask_parts(ctypes.byref(geo)), R, dtype=torch.float32,
                             device=dev) if want_mask else None  # fmt: skip
        bparts = torch.empty(lib.oops_trimul_bias_parts(ctypes.byref(geo)), 4 * H, dtype=torch.float32, device=dev)
        _lib.check(lib.oops_trimul_factors_backward(ctypes.byref(geo), _ptr(xn), _ptr(w_cat), _ptr(b_cat),
                                                    _ptr(mask), _ptr(d_factors), _ptr(d_proj), _ptr(mparts),
                                                    _ptr(bparts), stream),
                   "triangle_multiplication factor backward")  # fmt: skip
        d_xn = d_xn.addmm_(d_proj.t(), w_cat[:, :C])  # in place: no copy of d_xn into a new result
        d_wcat = sums.add(_long_k_partials(d_proj, xn[:, :C]), dtype)
        if b_cat is not None:
            sums.add(bparts, out=d_views[0])

        d_pair = torch.empty(G, P, C, dtype=dtype, device=dev)
        rg = _row_geometry(dtype, R, C, C, C, eps_in)
        in_parts = torch.empty(2, lib.oops_layer_norm_rows_parts(ctypes.byref(rg)), C, dtype=torch.float32,
                               device=dev)  # fmt: skip
        _lib.check(lib.oops_layer_norm_rows_backward(ctypes.byref(rg), _ptr(pair), _ptr(in_w), _ptr(mean_in),
                                                     _ptr(rstd_in), _ptr(d_xn), _ptr(d_pair), _ptr(in_parts[0]),
                                                     _ptr(in_parts[1]), stream),
                   "triangle_multiplication input LayerNorm backward")  # fmt: skip
        d_mask = sums.add(mparts).view(G, P) if want_mask else empty()
        for i, parts in ((3, in_parts[0]), (4, in_parts[1]), (5, on_parts[0]), (6, on_parts[1])):
            sums.add(parts, out=d_views[i])
        sums.run(stream)
    # projection gradients padded back to the operands' 16-byte rows
    if cp != C:
        d_wog, d_wcat = F.pad(d_wog, (0, cp - C)), F.pad(d_wcat, (0, cp - C))
    if hp != H:
        d_wo = F.pad(d_wo, (0, hp - H))
    return d_pair, d_mask, d_wcat, d_wo, d_wog, d_small


@torch.library.custom_op("oops_amd::trimul_backward", mutates_args=(), device_types="cuda")
def trimul_backward(
    dout: Tensor,
    pair: Tensor,
    mask: Optional[Tensor],
    w_cat: Tensor,
    wo: Tensor,
    wog: Tensor,
    small: Tensor,
    spans: List[int],
    xn: Tensor,
    mean_in: Tensor,
    rstd_in: Tensor,
    factors: Tensor,
    combined: Tensor,
    nrm: Tensor,
    mean_out: Tensor,
    rstd_out: Tensor,
    blocks: List[int],
    direction: str,
    eps_in: float,
    eps_out: float,
    need_mask: bool,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    return _backward_impl(dout, pair, mask, w_cat, wo, wog, small, spans, xn, mean_in, rstd_in, factors, combined,
                          nrm, mean_out, rstd_out, blocks, direction, eps_in, eps_out, need_mask)  # fmt: skip


@trimul_backward.register_fake
def _(dout, pair, mask, w_cat, wo, wog, small, spans, xn, mean_in, rstd_in, factors, combined, nrm, mean_out,
      rstd_out, blocks, direction, eps_in, eps_out, need_mask):  # fmt: skip
    G, P, C = pair.shape
    d_mask = pair.new_empty(G, P, dtype=torch.float32) if mask is not None and need_mask else pair.new_empty(
        0, dtype=torch.float32)
    return (pair.new_empty(G, P, C), d_mask, torch.empty_like(w_cat), torch.empty_like(wo), torch.empty_like(wog),
            torch.empty_like(small))  # fmt: skip


def _save(ctx, inputs, output):
    pair, mask, w_cat, wo, wog, small, spans, blocks, direction, eps_in, eps_out = inputs
    _out, xn, mean_in, rstd_in, factors, combined, nrm, mean_out, rstd_out = output
    ctx.save_for_backward(pair, mask, w_cat, wo, wog, small, xn, mean_in, rstd_in, factors, combined, nrm,
                          mean_out, rstd_out)  # fmt: skip
    ctx.args = (spans, blocks, direction, eps_in, eps_out)
    ctx.has_mask = mask is not None
    ctx.set_materialize_grads(False)  # no zero-filled gradients for the saved intermediates


def _setup_context(ctx, inputs, output):
    _save(ctx, inputs, output)
    for t in output[1:]:
        ctx.mark_non_differentiable(t)


def _grads(ctx, dout, backward):
    """Gradients of trimul_forward's 11 inputs."""

    if dout is None:
        return (None,) * 11
    pair, mask, w_cat, wo, wog, small, *rest = ctx.saved_tensors
    spans, blocks, direction, eps_in, eps_out = ctx.args
    need = ctx.needs_input_grad
    d_pair, d_mask, d_wcat, d_wo, d_wog, d_small = backward(
        dout, pair, mask, w_cat, wo, wog, small, spans, *rest, blocks, direction, eps_in, eps_out, bool(need[1])
    )
    d_mask = d_mask if ctx.has_mask and need[1] else None
    return d_pair, d_mask, d_wcat, d_wo, d_wog, d_small, None, None, None, None, None


def _backward(ctx, dout, *_unused):
    return _grads(ctx, dout, trimul_backward)


trimul_forward.register_autograd(_backward, setup_context=_setup_context)


class _EagerTrimul(torch.autograd.Function):
    """The same implementations as the custom ops, for eager calls: autograd
    calls the backward directly instead of through the operator dispatcher.
    Traced code (torch.compile), fake and subclass tensors take the custom ops."""

    @staticmethod
    def forward(ctx, *inputs):
        output = _forward_impl(*inputs)
        _save(ctx, inputs, output)
        return output[0]

    @staticmethod
    def backward(ctx, dout):
        return without_second_derivative(_grads(ctx, dout, _backward_impl), ctx, dout)


def _prepare(grouped: Tensor, mask: Optional[Tensor], weights, biases):
    """Kernel operands (pair, mask, w_cat, wo, wog, small, spans) from the caller's tensors, with
    differentiable torch ops (their autograd maps the operands' gradients back): projections concatenated and
    zero-padded to 16-byte rows; the small parameters (biases, LayerNorm affines) concatenated into one
    float32 buffer, one conversion for all, located by ``spans`` (in _SMALL order)."""

    in_w, in_b, wlv, wlg, wrv, wrg, on_w, on_b, wo, wog = weights
    blv, blg, brv, brg, bo, bog = biases
    C, H = grouped.shape[-1], wlv.shape[0]
    cp, hp = _round8(C), _round8(H)
    small = (((blv, blg, brv, brg), H), ((bo,), C), ((bog,), C), ((in_w,), C), ((in_b,), C), ((on_w,), H),
             ((on_b,), H))  # fmt: skip
    pieces, spans, off = [], [], 0
    for tensors, n in small:
        if all(t is None for t in tensors):
            spans += [-1, -1]
            continue
        for t in tensors:
            pieces.append(torch.zeros(n, device=grouped.device) if t is None else t.resolve_neg().reshape(-1))
        spans += [off, off + n * len(tensors)]
        off += n * len(tensors)
    buf = torch.cat(pieces).float() if pieces else torch.zeros(1, device=grouped.device)

    def padded(w: Tensor, width: int) -> Tensor:
        w = w.resolve_neg()
        return (F.pad(w, (0, width - w.shape[1])) if width != w.shape[1] else w).contiguous()

    pair = grouped.resolve_neg().contiguous()
    mask32 = None if mask is None else mask.resolve_neg().float().contiguous()
    return pair, mask32, padded(torch.cat([wlv, wlg, wrv, wrg]), cp), padded(wo, hp), padded(wog, cp), buf, spans


def _run(grouped: Tensor, mask: Optional[Tensor], blocks, direction, weights, biases, eps_in, eps_out) -> Tensor:
    """One fused pipeline for every served dtype: 16-bit pairs on the bf16/f16 MFMA kernels, float32 pairs
    on their exact float32 MFMA counterparts (csrc/trimul_f32.hip), the contraction as library GEMMs."""

    _admit(grouped, weights, biases)
    flat = [v for block in blocks for v in block]
    operands = _prepare(grouped, mask, weights, biases)
    args = (*operands, flat, direction, float(eps_in), float(eps_out))
    if needs_custom_op(grouped):
        return trimul_forward(*args)[0]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in operands[:6]):
        return _EagerTrimul.apply(*args)
    return _forward_impl(*args)[0]


# ----------------------------------------------------------------- nested


def _offsets(nested, level=None):
    t = nested.packed_offsets(dtype=torch.int64) if level is None else nested.ragged_level_offsets(level, dtype=torch.int64)
    return [int(v) for v in t.tolist()]


def _nested(pair, pair_mask, direction, weights, biases, eps_in, eps_out):
    """Canonical nested pairs (triangle_multiplication.py:170-223, :319-393)."""

    values = pair.concat
    require_no_forward_mode(_OPERATOR, values, None if pair_mask is None else pair_mask.concat, *weights, *biases)
    if not pair.batch_first:
        raise ValueError("triangle_multiplication NestedTensor batch must be the leading logical dimension")
    if pair.dim() < 4:
        raise ValueError(
            "triangle_multiplication nested pair elements must have shape (*prefix, N_i, N_i, pair_size); "
            f"got logical rank {pair.dim()}"
        )
    pr = pair.dim() - 4
    token_dims = (pr, pr + 1)
    if tuple(pair.packed_dim_order) != (*token_dims, *range(pr), pr + 2):
        raise unsupported(_OPERATOR, "requires token-pair-major nested (*prefix, N_i, N_i, pair_size) packing",
                          packed_dim_order=pair.packed_dim_order)  # fmt: skip
    if tuple(pair.ragged_dims) != token_dims:
        raise unsupported(_OPERATOR, "requires both nested token axes to be declared ragged",
                          ragged_dims=pair.ragged_dims)  # fmt: skip
    if values.dim() != pr + 2 or values.shape[-1] <= 0:
        raise ValueError(
            "triangle_multiplication nested pair elements must retain their static prefix and channel axis"
        )
    C = values.shape[-1]
    _check_weight_shapes(C, weights)
    _check_bias_shapes(C, weights[2].shape[0], biases)
    rows, packed = _offsets(pair, 0), _offsets(pair)
    if len(rows) <= 1:
        raise unsupported(_OPERATOR, "does not serve an empty NestedTensor batch")
    sizes = [b - a for a, b in zip(rows[:-1], rows[1:])]
    if any(n <= 0 for n in sizes):
        raise unsupported(_OPERATOR, "requires every nested pair element to have N > 0")
    if any(b - a != n * n for a, b, n in zip(packed[:-1], packed[1:], sizes)):
        raise ValueError("triangle_multiplication pair token dims must be square (N, N) per sample")
    if packed[-1] != values.shape[0]:
        raise ValueError(
            f"triangle_multiplication pair packed layout covers {packed[-1]} positions, "
            f"but packed values contain {values.shape[0]}"
        )
    prefix = tuple(values.shape[1:-1])
    mask_values = None
    if pair_mask is not None:
        if not pair_mask.batch_first or pair_mask.dim() != pair.dim() - 1:
            raise ValueError(
                "triangle_multiplication nested pair_mask elements must have shape (*prefix, N_i, N_i) "
                "with a leading wrapper batch"
            )
        if tuple(pair_mask.packed_dim_order) != (*token_dims, *range(pr)):
            raise unsupported(_OPERATOR, "requires token-pair-major nested (*prefix, N_i, N_i) mask packing",
                              packed_dim_order=pair_mask.packed_dim_order)  # fmt: skip
        if tuple(pair_mask.ragged_dims) != token_dims:
            raise unsupported(_OPERATOR, "requires both nested pair_mask token axes to be declared ragged",
                              ragged_dims=pair_mask.ragged_dims)  # fmt: skip
        mask_values = pair_mask.concat
        if tuple(mask_values.shape[1:]) != prefix:
            raise unsupported(_OPERATOR, "requires a nested pair_mask with the pair's complete static prefix")
        if _offsets(pair_mask, 0) != rows or _offsets(pair_mask) != packed:
            raise ValueError("triangle_multiplication pair_mask layout must match the pair layout per sample")
    require_same_device(_OPERATOR, values, mask_values, *weights, *biases)
    values, weights, biases = _prepare_autocast(values, weights, biases)
    # (cells, *prefix, C) -> (prefix groups, cells, C): each static prefix element is one group
    pr_n = len(prefix)
    grouped = values.permute(*range(1, pr_n + 1), 0, pr_n + 1).reshape(-1, values.shape[0], C)
    mask = None
    if mask_values is not None:
        m = mask_values.to(torch.float32) if not mask_values.is_floating_point() else mask_values
        mask = m.permute(*range(1, pr_n + 1), 0).reshape(-1, values.shape[0])
    blocks = [(a, n) for a, n in zip(packed[:-1], sizes)]
    out = _run(grouped, mask, blocks, direction, weights, biases, eps_in, eps_out)
    out = out.reshape(*prefix, values.shape[0], C).permute(pr_n, *range(pr_n), pr_n + 1)
    return pair.packed_like(out.contiguous())
