"""Model inputs and the velocity -> denoised (X0) conversion on MI355X.

Mirror of ``kinomlx/models/ltx2/transformer/wrappers.py`` (``Modality``, ``_to_denoised``,
``X0Model``). The conversion is one HIP pass over the latent and the velocity.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib


@dataclass(frozen=True)
class Modality:
    """One patchified stream supplied to the model (``wrappers.py:15-35``): ``latent (B, T, C)``,
    ``context (B, Tc, D)``, ``timesteps (B,)`` or ``(B, T)``, ``sigma`` scalar or ``(B,)``,
    ``positions (B, axes, T, 2)``."""

    latent: torch.Tensor
    context: torch.Tensor
    timesteps: torch.Tensor
    sigma: torch.Tensor
    positions: torch.Tensor
    enabled: bool = True
    context_mask: torch.Tensor | None = None
    attention_mask: torch.Tensor | None = None
    keyframes_mask: torch.Tensor | None = None
    positional_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None
    cross_positional_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None
    sparse_attention: object | None = None


def _to_denoised(modality: Modality, velocity: torch.Tensor | None) -> torch.Tensor | None:
    """``latent - timesteps * velocity`` in FP32, one rounding to the latent dtype
    (``wrappers.py:48-66``); ``(B,)`` timesteps broadcast over tokens and channels, ``(B, T)``
    over channels."""
    if velocity is None:
        return None
    latent = modality.latent
    timestep = modality.timesteps
    if timestep.dim() not in (1, 2):
        raise ValueError("modality timesteps must have shape (B,) or (B, T)")
    if latent.dim() != 3 or velocity.shape != latent.shape:
        raise ValueError("the X0 conversion takes (B, T, C) latents and velocities of one shape")
    batch, tokens, channels = (int(s) for s in latent.shape)
    if timestep.shape[0] != batch or (timestep.dim() == 2 and timestep.shape[1] != tokens):
        raise ValueError("modality timesteps do not match the latent")
    ts = timestep.float().contiguous()
    out = torch.empty_like(latent)
    _lib.launch_to_denoised(latent.contiguous(), velocity.contiguous(), ts, out, rows=batch * tokens,
                            dim=channels, ts_div=tokens if timestep.dim() == 1 else 1)
    return out


class X0Model:
    """Convert a velocity model's outputs to per-token denoised predictions (``wrappers.py:69-90``)."""

    def __init__(self, velocity_model) -> None:
        self.velocity_model = velocity_model

    @property
    def num_blocks(self) -> int:
        return self.velocity_model.num_blocks

    def __call__(self, video: Modality | None, audio: Modality | None = None):
        video_velocity, audio_velocity = self.velocity_model(video, audio)
        return (
            _to_denoised(video, video_velocity) if video is not None else None,
            _to_denoised(audio, audio_velocity) if audio is not None else None,
        )


__all__ = ["Modality", "X0Model"]
