"""CPU oracle for the triangle multiplicative update — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker.  The product
(``oops_amd``) never imports it.

It restates in numpy the update the reference's tests define
(tests/pair/triangle_multiplication/test_triangle_multiplication.py:48-80
``_reference`` and :166-198 ``_biased_reference``; operator docstring
oops/pair/triangle_multiplication/triangle_multiplication.py:67-146):

    xn    = LayerNorm_C(pair)
    left  = mask * (xn W_lv^T + b_lv) * sigmoid(xn W_lg^T + b_lg)      (likewise right)
    X[i,j,h] = sum_k left[i,k,h] right[j,k,h]        (outgoing)
             = sum_k left[k,i,h] right[k,j,h]        (incoming)
    out   = (LayerNorm_H(X) W_o^T + b_o) * sigmoid(xn W_og^T + b_og)

and its derivative written out (the reference's kernels implement the same
chain, oops/pair/triangle_multiplication/triton/kernel.py:190-628).

With ``rounding`` ("bf16" / "f16") the tensors the reference stores in the
pair dtype between its kernels are rounded there: xn, the two factors, X and
LayerNorm_H(X) (generic.py:351-503).

Parity pins (tests/test_oracle.py): the operator's docstring example, torch
float64 autograd of the reference test's own formulation (F.layer_norm,
F.linear, permuted matmul), and central finite differences.
"""

from __future__ import annotations

import numpy as np

from .gate import _rounder


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _layer_norm(x, w, b, eps):
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (x - mean) * rstd
    return xhat * w + b, xhat, rstd


def _layer_norm_backward(dy, xhat, rstd, w):
    wdy = dy * w
    n = xhat.shape[-1]
    dx = rstd * (wdy - wdy.sum(-1, keepdims=True) / n - xhat * (wdy * xhat).sum(-1, keepdims=True) / n)
    lead = tuple(range(dy.ndim - 1))
    return dx, (dy * xhat).sum(lead), dy.sum(lead)


def _linear(x, w, b):
    y = x @ w.T
    return y if b is None else y + b


def _as64(xs):
    return [None if x is None else np.asarray(x, np.float64) for x in xs]


def _contract(left, right, direction):
    """left/right (..., N, N, H) -> X (..., N, N, H)."""

    if direction == "outgoing":
        return np.einsum("...ikh,...jkh->...ijh", left, right)
    return np.einsum("...kih,...kjh->...ijh", left, right)


def triangle_multiplication_forward(pair, mask, weights, biases=(None,) * 6, direction="outgoing", input_eps=1e-5,
                                    output_eps=1e-5, rounding=None):  # fmt: skip
    """Returns the update (..., N, N, C) in float64.

    weights = (in_w, in_b, W_lv, W_lg, W_rv, W_rg, out_norm_w, out_norm_b, W_o, W_og);
    biases = (b_lv, b_lg, b_rv, b_rg, b_o, b_og), each may be None."""

    r = _rounder(rounding)
    pair = np.asarray(pair, np.float64)
    in_w, in_b, wlv, wlg, wrv, wrg, on_w, on_b, wo, wog = _as64(weights)
    blv, blg, brv, brg, bo, bog = _as64(biases)
    m = 1.0 if mask is None else np.broadcast_to(np.asarray(mask, np.float64), pair.shape[:-1])[..., None]
    xn = r(_layer_norm(pair, in_w, in_b, input_eps)[0])
    left = r(m * _linear(xn, wlv, blv) * _sigmoid(_linear(xn, wlg, blg)))
    right = r(m * _linear(xn, wrv, brv) * _sigmoid(_linear(xn, wrg, brg)))
    x = r(_contract(left, right, direction))
    y = r(_layer_norm(x, on_w, on_b, output_eps)[0])
    return _linear(y, wo, bo) * _sigmoid(_linear(xn, wog, bog))


def triangle_multiplication_backward(pair, mask, weights, biases, d_out, direction="outgoing", input_eps=1e-5,
                                     output_eps=1e-5):  # fmt: skip
    """float64 gradients: (d_pair, d_mask or None, d_weights (10), d_biases (6, None where absent))."""

    pair = np.asarray(pair, np.float64)
    dy_out = np.asarray(d_out, np.float64)
    in_w, in_b, wlv, wlg, wrv, wrg, on_w, on_b, wo, wog = _as64(weights)
    blv, blg, brv, brg, bo, bog = _as64(biases)
    shape = pair.shape[:-1]
    m = np.ones(shape + (1,)) if mask is None else np.broadcast_to(np.asarray(mask, np.float64), shape)[..., None]

    xn, xhat_in, rstd_in = _layer_norm(pair, in_w, in_b, input_eps)
    lv, lg = _linear(xn, wlv, blv), _linear(xn, wlg, blg)
    rv, rg = _linear(xn, wrv, brv), _linear(xn, wrg, brg)
    sl, sr = _sigmoid(lg), _sigmoid(rg)
    left, right = m * lv * sl, m * rv * sr
    x = _contract(left, right, direction)
    y, xhat_out, rstd_out = _layer_norm(x, on_w, on_b, output_eps)
    a = _linear(y, wo, bo)
    sg = _sigmoid(_linear(xn, wog, bog))

    flat = lambda t: t.reshape(-1, t.shape[-1])  # noqa: E731
    da = dy_out * sg
    dgl = dy_out * a * sg * (1 - sg)
    d_wo, d_bo = flat(da).T @ flat(y), flat(da).sum(0)
    d_wog, d_bog = flat(dgl).T @ flat(xn), flat(dgl).sum(0)
    dy = da @ wo
    dxn = dgl @ wog
    dx, d_on_w, d_on_b = _layer_norm_backward(dy, xhat_out, rstd_out, on_w)
    if direction == "outgoing":  # X[i,j] = sum_k L[i,k] R[j,k]
        d_left = np.einsum("...ijh,...jkh->...ikh", dx, right)
        d_right = np.einsum("...ijh,...ikh->...jkh", dx, left)
    else:  # X[i,j] = sum_k L[k,i] R[k,j]
        d_left = np.einsum("...ijh,...kjh->...kih", dx, right)
        d_right = np.einsum("...ijh,...kih->...kjh", dx, left)
    grads_w, grads_b = [], []
    d_mask = np.zeros(shape)
    for d_f, v, s, wv, wg in ((d_left, lv, sl, wlv, wlg), (d_right, rv, sr, wrv, wrg)):
        dv = d_f * m * s
        dg = d_f * m * v * s * (1 - s)
        d_mask += (d_f * v * s).sum(-1)
        dxn += dv @ wv + dg @ wg
        grads_w += [flat(dv).T @ flat(xn), flat(dg).T @ flat(xn)]
        grads_b += [flat(dv).sum(0), flat(dg).sum(0)]
    d_pair, d_in_w, d_in_b = _layer_norm_backward(dxn, xhat_in, rstd_in, in_w)
    d_weights = (d_in_w, d_in_b, *grads_w, d_on_w, d_on_b, d_wo, d_wog)
    d_biases = tuple(g if b is not None else None for g, b in zip((*grads_b, d_bo, d_bog), (blv, blg, brv, brg, bo, bog)))
    if mask is None:
        d_m = None
    else:
        mshape = np.shape(mask)
        d_m = d_mask
        while d_m.ndim > len(mshape):
            d_m = d_m.sum(0)
        for ax, n in enumerate(mshape):
            if n == 1 and d_m.shape[ax] != 1:
                d_m = d_m.sum(ax, keepdims=True)
    return d_pair, d_m, d_weights, d_biases
