"""Deterministic Euler diffusion steps on MI355X.

Mirror of ``kinomlx/samplers/steps.py`` (``euler_velocity_step`` ``:8-32``, ``euler_step``
``:35-72``): the same argument checks, the scalar coefficient formed on the host in double
precision and narrowed to FP32, one HIP pass over the latent.
"""

from __future__ import annotations

import math

import torch

from .. import _lib


def euler_velocity_step(sample: torch.Tensor, velocity: torch.Tensor, sigma: float, sigma_next: float) -> torch.Tensor:
    """``sample + dtype(float32(sigma_next - sigma) * velocity)``: the scaled velocity is
    narrowed to the velocity dtype before the add (``steps.py:8-32``)."""
    if not math.isfinite(sigma) or not math.isfinite(sigma_next):
        raise ValueError("Euler velocity sigmas must be finite")
    if tuple(sample.shape) != tuple(velocity.shape):
        raise ValueError(f"velocity shape {tuple(velocity.shape)} does not match sample {tuple(sample.shape)}")
    if sample.dtype != velocity.dtype:
        raise ValueError(f"velocity dtype {velocity.dtype} does not match sample dtype {sample.dtype}")
    out = torch.empty_like(sample, memory_format=torch.contiguous_format)
    if sample.numel():
        _lib.launch_euler_velocity_step(sample.contiguous(), velocity.contiguous(), out, sigma_next - sigma)
    return out


def euler_step(sample: torch.Tensor, denoised: torch.Tensor, sigma: float, sigma_next: float) -> torch.Tensor:
    """``denoised + (sigma_next / sigma) * (sample - denoised)`` in FP32, cast to the sample
    dtype (``steps.py:35-72``)."""
    if not math.isfinite(sigma) or sigma <= 0.0:
        raise ValueError(f"current sigma must be positive and finite, got {sigma!r}")
    if tuple(sample.shape) != tuple(denoised.shape):
        raise ValueError(f"denoised shape {tuple(denoised.shape)} does not match sample {tuple(sample.shape)}")
    ratio = sigma_next / sigma
    out = torch.empty_like(sample, memory_format=torch.contiguous_format)
    if sample.numel():
        _lib.launch_euler_step(sample.contiguous(), denoised.contiguous(), out, ratio)
    return out


__all__ = ["euler_step", "euler_velocity_step"]
