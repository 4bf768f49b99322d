"""Latent state of an LTX-2 stream and the conditioning composite on MI355X.

Mirror of ``LatentState`` (``kinomlx/models/ltx2/types.py:97-125``) and ``post_process_latent``
(``kinomlx/models/ltx2/state.py:70-83``); the composite is one HIP pass.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib


@dataclass(frozen=True)
class LatentState:
    """``latent (B, T, C)``, ``denoise_mask (B, T[, 1])`` (1 = denoise fully, 0 = keep),
    ``positions``, ``clean_latent`` and ``uniform_mask`` (true iff every mask entry is 1; a
    host flag, never derived from the mask on the device)."""

    latent: torch.Tensor
    denoise_mask: torch.Tensor
    positions: torch.Tensor
    clean_latent: torch.Tensor
    uniform_mask: bool = True


def post_process_latent(denoised: torch.Tensor, state: LatentState) -> torch.Tensor:
    """``denoised * mask + clean * (1 - mask)`` in FP32, one rounding to the denoised dtype;
    the prediction itself when the mask is uniform (``state.py:70-83``)."""
    if state.uniform_mask:
        return denoised
    mask = state.denoise_mask
    if mask.dim() == 3 and mask.shape[-1] == 1:
        mask = mask[..., 0]
    if denoised.dim() != 3 or mask.shape != denoised.shape[:2] or state.clean_latent.shape != denoised.shape:
        raise ValueError("the conditioning composite takes (B, T, C) latents and a (B, T) mask")
    batch, tokens, channels = (int(s) for s in denoised.shape)
    out = torch.empty_like(denoised, memory_format=torch.contiguous_format)
    _lib.launch_mask_composite(denoised.contiguous(), state.clean_latent.contiguous(), mask.float().contiguous(),
                               out, rows=batch * tokens, dim=channels)
    return out


__all__ = ["LatentState", "post_process_latent"]
