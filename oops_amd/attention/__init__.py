"""Pair-biased attention operators (gfx950 HIP kernels behind the reference's API)."""

from .pair_bias import pair_bias_attention
from .triangle import triangle_attention

__all__ = ["pair_bias_attention", "triangle_attention"]
