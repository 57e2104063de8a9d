"""Second derivatives are not provided: differentiating a gradient of the
eager operators raises instead of returning values that silently miss the
kernels' own derivatives (first derivatives taken with ``create_graph=True``
are still correct)."""

import pytest
import torch

from oops_amd import layer_norm, triangle_attention, triangle_multiplication

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _r(*shape, dtype=torch.bfloat16, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(DEV).requires_grad_(True)


def _second_raises(out, x):
    dout = torch.randn_like(out)
    plain = torch.autograd.grad(out, x, dout, retain_graph=True)[0]
    (first,) = torch.autograd.grad(out, x, dout, create_graph=True)
    torch.testing.assert_close(first, plain)
    with pytest.raises(RuntimeError, match="no second derivatives"):
        first.float().sum().backward()


def test_triangle_attention_second_derivative_raises():
    q, k, v = (_r(1, 6, 40, 2, 32, seed=s) for s in range(3))
    bias = _r(1, 1, 2, 40, 40, seed=3)
    _second_raises(triangle_attention(q, k, v, None, bias), q)


def test_layer_norm_second_derivative_raises():
    x = _r(20, 96)
    w, b = _r(96, dtype=torch.float32, seed=1), _r(96, dtype=torch.float32, seed=2)
    _second_raises(layer_norm(x, 96, w, b), x)


def test_triangle_multiplication_second_derivative_raises():
    c, h = 32, 32
    pair = _r(1, 12, 12, c, seed=4)
    names = ("input_norm_weight", "input_norm_bias", "left_value_weight", "left_gate_weight",
             "right_value_weight", "right_gate_weight", "output_norm_weight", "output_norm_bias",
             "output_weight", "output_gate_weight")  # fmt: skip
    shapes = ((c,), (c,), (h, c), (h, c), (h, c), (h, c), (h,), (h,), (c, h), (c, c))
    weights = {n: _r(*s, scale=0.2, seed=10 + i) for i, (n, s) in enumerate(zip(names, shapes))}
    _second_raises(triangle_multiplication(pair, None, **weights), pair)
