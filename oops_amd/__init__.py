"""oops_amd: MI355X-native pair-biased triangle attention (and the operators beside it) with the OOps API.

``from oops_amd import triangle_attention, pair_bias_attention, OOpsUnsupportedError``
is the drop-in for ``from oops import ...`` on the attention path.
"""

from ._errors import OOpsUnsupportedError
from .attention import gate_attention_output, gated_pair_bias_attention, pair_bias_attention, triangle_attention
from .normalization import LayerNorm, layer_norm
from .pair import triangle_multiplication

__all__ = [
    "LayerNorm",
    "OOpsUnsupportedError",
    "gate_attention_output",
    "gated_pair_bias_attention",
    "layer_norm",
    "pair_bias_attention",
    "triangle_attention",
    "triangle_multiplication",
]
