"""Krea 2 block surface on MI355X: mirror of ``kinomlx/models/krea2/transformer/model.py`` over
the kx355 kernels."""

from . import transformer  # noqa: F401
from .transformer import (  # noqa: F401
    Krea2Attention,
    Krea2BlockConfig,
    Krea2RMSNorm,
    Krea2RotaryEmbedding,
    Krea2SwiGLU,
    Krea2TransformerBlock,
    apply_rotary_embedding,
    split_six_way_modulation,
)
