"""CPU oracle for the gated output stage — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker.  The product
(``oops_amd``) never imports it.

It restates in numpy the equation of the reference's
``gate_attention_output`` (oops/attention/gate/gate_attention_output.py:57-58
and its ``_gate_attention_output_reference``, :178-185):

    attention_flat = attention (*prefix, H, Q, D) moved to (*prefix, Q, H*D)
    gated = sigmoid(single @ gate_weight^T) * attention_flat
    out   = gated @ output_weight^T

and its derivative, written out (the reference takes it with autograd through
the same composition, oops/attention/gate/triton/ops.py:50-83):

    d_gated  = d_out @ output_weight,      d_output_weight = d_out^T gated
    d_att    = d_gated * g,                g = sigmoid(logits)
    d_logits = d_gated * attention_flat * g * (1 - g)
    d_single = d_logits @ gate_weight,     d_gate_weight = d_logits^T single

With ``rounding`` ("bf16" / "f16") the intermediates the reference stores in
the operand dtype are rounded there, as its kernel and its Torch composition
do (gate/triton/kernel.py:62-66, :104-113): the logits, the gate, the gated
values, dO @ W_o, and each step of the sigmoid backward.  The comparison then
measures the implementation, not the dtype's own storage rounding.

Parity pins (tests/test_oracle.py): the reference's own docstring example
(zero gate logits halve the attention values), torch autograd of the
composition in float64 (and in bfloat16 for the rounding points), and central
finite differences.
"""

from __future__ import annotations

import numpy as np


def _flat(attention: np.ndarray) -> np.ndarray:
    """(*prefix, H, Q, D) -> (*prefix, Q, H*D)."""

    *prefix, h, q, d = attention.shape
    return np.swapaxes(attention, -3, -2).reshape(*prefix, q, h * d)


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def _rounder(rounding):
    """float64 -> nearest value of the storage dtype (round-to-nearest-even), as float64."""

    if rounding is None:
        return lambda x: x
    if rounding == "f16":
        return lambda x: np.asarray(x).astype(np.float16).astype(np.float64)
    if rounding == "bf16":

        def bf16(x):
            f = np.ascontiguousarray(np.asarray(x, np.float64).astype(np.float32))
            u = f.view(np.uint32).astype(np.uint64)
            u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
            return u.astype(np.uint32).view(np.float32).astype(np.float64)

        return bf16
    raise ValueError(f"unknown rounding {rounding!r}")


def gate_attention_output_forward(attention, single, gate_weight, output_weight, rounding=None):
    """Returns (out, gated, logits) in float64."""

    r = _rounder(rounding)
    a = _flat(np.asarray(attention, np.float64))
    s = np.asarray(single, np.float64)
    logits = r(s @ np.asarray(gate_weight, np.float64).T)
    gated = r(r(_sigmoid(logits)) * a)
    out = gated @ np.asarray(output_weight, np.float64).T
    return out, gated, logits


def gate_attention_output_backward(attention, single, gate_weight, output_weight, d_out, rounding=None):
    """Gradients (attention, single, gate_weight, output_weight) in float64."""

    r = _rounder(rounding)
    attention = np.asarray(attention, np.float64)
    *prefix, h, q, d = attention.shape
    a = _flat(attention)
    s = np.asarray(single, np.float64)
    w = np.asarray(gate_weight, np.float64)
    wo = np.asarray(output_weight, np.float64)
    dy = np.asarray(d_out, np.float64)
    logits = r(s @ w.T)
    g = r(_sigmoid(logits))
    gated = r(g * a)
    d_gated = r(dy @ wo)
    d_wo = dy.reshape(-1, dy.shape[-1]).T @ gated.reshape(-1, gated.shape[-1])
    d_a = d_gated * g
    d_logits = r(r(r(d_gated * a) * r(1.0 - g)) * g)
    d_s = d_logits @ w
    d_w = d_logits.reshape(-1, d_logits.shape[-1]).T @ s.reshape(-1, s.shape[-1])
    d_att = np.swapaxes(d_a.reshape(*prefix, q, h, d), -3, -2)
    return d_att, d_s, d_w, d_wo
