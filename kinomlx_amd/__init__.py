"""kinomlx_amd — MI355X-native (gfx950) implementation of the KinoMLX DiT-block hot path.

The reference's operator surface for the diffusion-transformer block (modulated norms, RoPE,
attention, dense and affine-quantized linear layers, and the LTX-2 / FLUX.2 / Krea 2 block
compositions that call them) on PyTorch-ROCm tensors, backed by hand-written HIP kernels in
``libkx355.so`` (C ABI: ``include/kx355.h``). There is no CPU or PyTorch fallback: operators
raise when the library or a GPU is missing.
"""

from . import _lib

__version__ = "0.1.0"


def library_available() -> bool:
    """Whether ``libkx355.so`` is built and a GPU is visible."""
    return _lib.available()


__all__ = ["library_available"]
