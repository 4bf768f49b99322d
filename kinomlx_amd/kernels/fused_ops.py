"""FP32-opmath norms and activations on MI355X.

Mirror of ``kinomlx/kernels/fused_ops.py``: same names, arguments and dtype-preserving
semantics, on torch tensors. Every function runs a hand-written gfx950 kernel from
``libkx355.so``; there is no CPU or PyTorch fallback. Activations are bf16 or fp16 (the
reference's two transformer dtypes; the output keeps the input's); other dtypes raise
``ValueError``.
"""

from __future__ import annotations

import torch

from .. import _lib

_DTYPES = (torch.bfloat16, torch.float16)


def _require(value: torch.Tensor, what: str) -> None:
    if value.dtype not in _DTYPES:
        raise ValueError(f"{what} takes float16 or bfloat16 activations on MI355X, got {value.dtype}")


def _empty(value: torch.Tensor) -> torch.Tensor:
    return torch.empty(value.shape, dtype=value.dtype, device=value.device)


def rms_norm(
    value: torch.Tensor,
    weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    *,
    weight_offset: float = 0.0,
) -> torch.Tensor:
    """RMSNorm over the last axis with FP32 reduction and affine math, one rounding.

    ``x * rsqrt(mean(x^2) + eps) * (weight + weight_offset)``; unweighted when ``weight`` is
    None (``kinomlx/kernels/fused_ops.py:412-457``, Metal arithmetic ``:141-193``).
    """
    _require(value, "rms_norm")
    out = _empty(value)
    if value.numel() == 0:
        return out
    if weight is None:
        _lib.launch_adaln_norm(value, out, None, None, eps, _lib.KX_NORM_RMS)
        return out
    if weight.dim() != 1 or weight.shape[0] != value.shape[-1]:
        raise ValueError(f"rms_norm weight must have shape ({value.shape[-1]},)")
    _lib.launch_rmsnorm_rope(value, out, weight, eps, weight_offset, norm_width=value.shape[-1])
    return out


def layer_norm(value: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Non-affine LayerNorm, FP32 statistics (``mx.fast.layer_norm(x, None, None, eps)`` as
    called at ``kinomlx/models/flux2/transformer.py:57``)."""
    _require(value, "layer_norm")
    out = _empty(value)
    if value.numel():
        _lib.launch_adaln_norm(value, out, None, None, eps, _lib.KX_NORM_LAYER)
    return out


def gelu_approx(value: torch.Tensor) -> torch.Tensor:
    """tanh GELU with FP32 opmath and the inner argument clamped to +-10
    (``kinomlx/kernels/fused_ops.py:27-35,327-350``)."""
    _require(value, "gelu_approx")
    src = value.contiguous()
    out = _empty(value)
    if value.numel():
        _lib.launch_unary("kx_gelu_tanh", src, out)
    return out


def silu(value: torch.Tensor) -> torch.Tensor:
    """SiLU with FP32 opmath (``kinomlx/kernels/fused_ops.py:40-45,353-372``)."""
    _require(value, "silu")
    src = value.contiguous()
    out = _empty(value)
    if value.numel():
        _lib.launch_unary("kx_silu", src, out)
    return out


def swiglu(value: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * content`` over the two halves of the last axis, one pass
    (``kinomlx/models/flux2/transformer.py:63-65``)."""
    _require(value, "swiglu")
    if value.shape[-1] % 2:
        raise ValueError("swiglu needs an even last axis")
    out = torch.empty((*value.shape[:-1], value.shape[-1] // 2), dtype=value.dtype, device=value.device)
    if out.numel():
        _lib.launch_swiglu(value, out)
    return out


__all__ = ["gelu_approx", "layer_norm", "rms_norm", "silu", "swiglu"]
