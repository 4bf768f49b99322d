"""FLUX.2 blocks on MI355X: mirror of ``kinomlx/models/flux2/transformer.py`` and
``kinomlx/models/flux2/kv.py:48-54`` over the kx355 kernels."""

from . import kv, transformer  # noqa: F401
from .kv import attend  # noqa: F401
from .transformer import (  # noqa: F401
    DoubleAttention,
    DoubleBlock,
    FeedForward,
    Modulation,
    QKNorm,
    SingleAttention,
    SingleBlock,
    joint_attention,
    normalized,
    rotary_positions,
    rotate,
    swiglu,
)
