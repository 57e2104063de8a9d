"""Pair-biased attention operators (gfx950 HIP kernels behind the reference's API)."""

from .gate import gate_attention_output, gated_pair_bias_attention
from .pair_bias import pair_bias_attention
from .triangle import triangle_attention

__all__ = ["gate_attention_output", "gated_pair_bias_attention", "pair_bias_attention", "triangle_attention"]
