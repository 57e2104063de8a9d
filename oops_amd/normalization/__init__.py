"""Normalization operators (the reference's ``oops.normalization``)."""

from .layer_norm import layer_norm
from .modules import LayerNorm

__all__ = ["LayerNorm", "layer_norm"]
