"""CPU oracle for LayerNorm over the last axis — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker.  It restates
the reference's operator (oops/normalization/layer_norm/layer_norm.py:30-110:
biased variance, ``(x - mean) / sqrt(var + eps) * weight + bias``) and its
derivative in numpy float64.  Pinned in tests/test_oracle.py against torch's
float64 ``F.layer_norm`` and its autograd.
"""

from __future__ import annotations

import numpy as np


def layer_norm_forward(x, weight=None, bias=None, eps=1e-5):
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def layer_norm_backward(x, dy, weight=None, eps=1e-5):
    """(dx, dweight, dbias) of sum(y * dy)."""

    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    n = x.shape[-1]
    mean = x.mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(((x - mean) ** 2).mean(-1, keepdims=True) + eps)
    xhat = (x - mean) * rstd
    w = 1.0 if weight is None else np.asarray(weight, np.float64)
    g = dy * w
    dx = rstd * (g - g.sum(-1, keepdims=True) / n - xhat * (g * xhat).sum(-1, keepdims=True) / n)
    lead = tuple(range(x.ndim - 1))
    return dx, (dy * xhat).sum(lead), dy.sum(lead)
