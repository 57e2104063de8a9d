"""Pair-biased attention operators (gfx950 HIP kernels behind the reference's API)."""

from .triangle import triangle_attention

__all__ = ["triangle_attention"]
