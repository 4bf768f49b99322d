"""MI355X kernels behind the reference's ``kinomlx.kernels`` surface
(``kinomlx/kernels/__init__.py``): FP32-opmath norms and activations, split RoPE, MFMA linear
products and the affine quantized linear."""

from . import mpp_linear, quantized, split_rope
from .fused_ops import gelu_approx, layer_norm, rms_norm, silu, swiglu

__all__ = [
    "gelu_approx",
    "layer_norm",
    "mpp_linear",
    "quantized",
    "rms_norm",
    "silu",
    "split_rope",
    "swiglu",
]
