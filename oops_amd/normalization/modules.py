"""``LayerNorm``: the ``torch.nn.LayerNorm`` module on the HIP row kernels.

Drop-in for the reference's module (oops/normalization/layer_norm/modules.py:31-70,
exported as ``oops.LayerNorm``): the constructor, parameters and state dict are
``torch.nn.LayerNorm``'s; a call goes through ``layer_norm`` and, when that
operator declines the input with ``OOpsUnsupportedError`` (CPU tensors, float64,
several normalized dimensions, widths above 8192, ...), through PyTorch's own
LayerNorm instead.  Call ``layer_norm`` directly where unsupported inputs should
raise.
"""

from __future__ import annotations

from torch import Tensor, nn

from .._errors import OOpsUnsupportedError
from .layer_norm import layer_norm


class LayerNorm(nn.LayerNorm):
    """``torch.nn.LayerNorm`` whose served calls run ``oops_amd.layer_norm``."""

    def forward(self, input: Tensor) -> Tensor:
        try:
            return layer_norm(input, self.normalized_shape, self.weight, self.bias, self.eps)
        except OOpsUnsupportedError:
            return super().forward(input)
