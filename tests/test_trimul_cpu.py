"""Host-side contract of triangle_multiplication and layer_norm (no GPU needed).

Shape and topology errors are ValueError and unsupported devices, dtypes and
packings OOpsUnsupportedError, with the reference's rules
(oops/pair/triangle_multiplication/triangle_multiplication.py:153-443,
oops/normalization/layer_norm/layer_norm.py:69-143).
"""

import pytest
import torch

from nested_standin import NestedTensor
from oops_amd import OOpsUnsupportedError, layer_norm, triangle_multiplication

_NAMES = ("input_norm_weight", "input_norm_bias", "left_value_weight", "left_gate_weight", "right_value_weight",
          "right_gate_weight", "output_norm_weight", "output_norm_bias", "output_weight", "output_gate_weight")


def _weights(c=8, h=4):
    shapes = ((c,), (c,), (h, c), (h, c), (h, c), (h, c), (h,), (h,), (c, h), (c, c))
    return {n: torch.zeros(s) for n, s in zip(_NAMES, shapes)}


def test_trimul_contract_errors():
    w = _weights()
    pair = torch.zeros(2, 5, 5, 8)
    with pytest.raises(ValueError, match="direction"):
        triangle_multiplication(pair, direction="sideways", **w)
    with pytest.raises(ValueError, match="square"):
        triangle_multiplication(torch.zeros(5, 4, 8), **w)
    with pytest.raises(ValueError, match="rank"):
        triangle_multiplication(torch.zeros(5, 8), **w)
    with pytest.raises(ValueError, match="broadcast"):
        triangle_multiplication(pair, torch.ones(3, 5, 5), **w)
    bad = dict(w, left_gate_weight=torch.zeros(3, 8))
    with pytest.raises(ValueError, match="left_gate_weight"):
        triangle_multiplication(pair, **bad)
    with pytest.raises(ValueError, match="output_bias"):
        triangle_multiplication(pair, output_bias=torch.zeros(3), **w)
    with pytest.raises(OOpsUnsupportedError):
        triangle_multiplication(pair, **w)  # CPU pair
    with pytest.raises(ValueError, match="NestedTensor"):
        triangle_multiplication(pair, NestedTensor([torch.ones(5, 5)], ragged_dims=(0, 1)), **w)


def test_trimul_nested_contract_errors():
    w = _weights()
    nt = NestedTensor([torch.zeros(3, 3, 8), torch.zeros(5, 5, 8)], ragged_dims=(0, 1))
    with pytest.raises(ValueError, match="NestedTensor"):
        triangle_multiplication(nt, torch.ones(8, 8), **w)
    with pytest.raises(OOpsUnsupportedError, match="ragged"):
        triangle_multiplication(NestedTensor([torch.zeros(3, 3, 8)], ragged_dims=(0,)), **w)
    mismatched = NestedTensor([torch.ones(3, 3), torch.ones(4, 4)], ragged_dims=(0, 1))
    with pytest.raises(ValueError, match="layout"):
        triangle_multiplication(nt, mismatched, **w)
    with pytest.raises(OOpsUnsupportedError):
        triangle_multiplication(nt, **w)  # CPU values


def test_layer_norm_contract_errors():
    x = torch.zeros(4, 8)
    with pytest.raises(OOpsUnsupportedError, match="final dimension"):
        layer_norm(x, (2, 4))
    with pytest.raises(OOpsUnsupportedError):
        layer_norm(x, 8)  # CPU input
    nt = NestedTensor([torch.zeros(3, 8), torch.zeros(5, 8)], ragged_dims=(0,))
    with pytest.raises(ValueError, match="dense affine"):
        layer_norm(nt, 8, NestedTensor([torch.zeros(8)], ragged_dims=(0,)))
    ragged_last = NestedTensor([torch.zeros(3, 2), torch.zeros(3, 4)], ragged_dims=(1,))
    with pytest.raises(OOpsUnsupportedError, match="static"):
        layer_norm(ragged_last, 4)
