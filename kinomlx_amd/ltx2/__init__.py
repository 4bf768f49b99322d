"""LTX-2 DiT block on MI355X (mirror of ``kinomlx/models/ltx2/transformer`` and
``kinomlx/models/ltx2/kernels/dense_attention.py``)."""

from . import attention, dense_attention, feed_forward, rope, transformer
from .attention import Attention, Linear, RMSNorm
from .feed_forward import FeedForward, GELUApprox
from .rope import LTXRopeType, apply_rotary_emb, apply_split_rotary_emb, precompute_freqs_cis
from .transformer import BasicAVTransformerBlock, TransformerArgs, TransformerConfig

__all__ = [
    "Attention",
    "BasicAVTransformerBlock",
    "FeedForward",
    "GELUApprox",
    "LTXRopeType",
    "Linear",
    "RMSNorm",
    "TransformerArgs",
    "TransformerConfig",
    "apply_rotary_emb",
    "apply_split_rotary_emb",
    "attention",
    "dense_attention",
    "feed_forward",
    "precompute_freqs_cis",
    "rope",
    "transformer",
]
