"""One LTX-2 denoising step on MI355X: the X0 transformer call, the Euler updates and the finite
checks, for the video stream alone or with the audio stream.

Mirror of the deterministic-Euler path of ``kinomlx/models/ltx2/denoise.py``
(``LTX2DenoiseError`` ``:11-12``, ``_advance_sample`` ``:60-85``, ``_advance_state``
``:100-120``, ``modality_from_state`` ``:123-156``, ``denoise_step`` ``:159-258``). The finite check is one reduction kernel over the new latent; its one-int flag is the
step's only device-to-host read, as ``mx.stack([...]).tolist()`` is the reference's.
"""

from __future__ import annotations

from dataclasses import replace
from typing import Literal

import torch

from .. import _lib
from ..samplers.steps import euler_step
from .state import LatentState, post_process_latent
from .wrappers import Modality

DenoiseStepKind = Literal["deterministic-euler", "ancestral-rf"]


class LTX2DenoiseError(RuntimeError):
    """A completed denoise step produced nonfinite active latents."""


def all_finite(*values: torch.Tensor) -> list[bool]:
    """``mx.all(mx.isfinite(value))`` per tensor through the finite-check kernel, with one host
    read for all of them (the reference stacks the flags and reads them once, ``:244-258``)."""
    flags = torch.empty(len(values), dtype=torch.int32, device=values[0].device)
    for index, value in enumerate(values):
        _lib.launch_all_finite(value.contiguous(), flags[index:index + 1])
    return [bool(v) for v in flags.tolist()]


def modality_from_state(state: LatentState, context: torch.Tensor, sigma: float, *, enabled: bool = True,
                        context_mask: torch.Tensor | None = None, keyframes_mask: torch.Tensor | None = None,
                        sparse_attention: object | None = None) -> Modality:
    """Scalar-timestep fast path: ``(B,)`` timesteps of ``sigma`` for a uniform mask, else
    ``mask * sigma`` per token (``denoise.py:123-156``)."""
    sigma_tensor = torch.full((state.latent.shape[0],), sigma, dtype=torch.float32, device=state.latent.device)
    if state.uniform_mask:
        timesteps = sigma_tensor
    else:
        mask = state.denoise_mask
        if mask.dim() == 3 and mask.shape[-1] == 1:
            mask = mask[..., 0]
        timesteps = mask.float() * sigma
    return Modality(latent=state.latent, context=context, timesteps=timesteps, sigma=sigma_tensor,
                    positions=state.positions, enabled=enabled, context_mask=context_mask,
                    keyframes_mask=keyframes_mask, sparse_attention=sparse_attention)


def _advance_sample(sample: torch.Tensor, denoised: torch.Tensor, *, sigma: float, sigma_next: float,
                    step_kind: DenoiseStepKind, noise: torch.Tensor | None) -> torch.Tensor:
    if step_kind == "deterministic-euler":
        if noise is not None:
            raise ValueError("deterministic Euler must not receive transition noise")
        return euler_step(sample, denoised, sigma, sigma_next)
    if step_kind == "ancestral-rf":
        raise ValueError("the ancestral RF step is not built for MI355X")
    raise ValueError(f"unknown denoise step kind {step_kind!r}")


def denoise_step(video_state: LatentState, audio_state: LatentState | None = None, *, sigma: float,
                 sigma_next: float, transformer, video_context: torch.Tensor,
                 audio_context: torch.Tensor | None = None, video_context_mask: torch.Tensor | None = None,
                 audio_context_mask: torch.Tensor | None = None, video_keyframes_mask: torch.Tensor | None = None,
                 video_enabled: bool = True, audio_enabled: bool = True,
                 step_kind: DenoiseStepKind = "deterministic-euler", video_noise: torch.Tensor | None = None,
                 audio_noise: torch.Tensor | None = None,
                 video_sparse_attention: object | None = None) -> tuple[LatentState, LatentState | None]:
    """Run one X0 transformer call and the Euler update of each enabled stream, then check the
    new latents are finite (``denoise.py:159-258``). ``transformer`` is an ``X0Model``."""
    video_modality = modality_from_state(video_state, video_context, sigma, enabled=video_enabled,
                                         context_mask=video_context_mask, keyframes_mask=video_keyframes_mask,
                                         sparse_attention=video_sparse_attention)
    audio_modality = None
    if audio_state is not None:
        if audio_context is None:
            raise ValueError("audio context is required for an audio latent state")
        audio_modality = modality_from_state(audio_state, audio_context, sigma, enabled=audio_enabled,
                                             context_mask=audio_context_mask)
    video_denoised, audio_denoised = transformer(video_modality, audio_modality)
    active = []
    if video_enabled:
        if video_denoised is None:
            raise RuntimeError("transformer returned no video prediction")
        latent = _advance_sample(video_state.latent, post_process_latent(video_denoised, video_state), sigma=sigma,
                                 sigma_next=sigma_next, step_kind=step_kind, noise=video_noise)
        video_state = replace(video_state, latent=latent)
        active.append(("video", video_state.latent))
    if audio_state is not None and audio_enabled:
        if audio_denoised is None:
            raise RuntimeError("transformer returned no audio prediction")
        latent = _advance_sample(audio_state.latent, post_process_latent(audio_denoised, audio_state), sigma=sigma,
                                 sigma_next=sigma_next, step_kind=step_kind, noise=audio_noise)
        audio_state = replace(audio_state, latent=latent)
        active.append(("audio", audio_state.latent))
    if active:
        for (modality, value), valid in zip(active, all_finite(*(v for _, v in active))):
            if not valid:
                raise LTX2DenoiseError(f"LTX-2 denoising produced a nonfinite {modality} latent in {value.dtype}.")
    return video_state, audio_state


__all__ = [
    "DenoiseStepKind",
    "LTX2DenoiseError",
    "all_finite",
    "denoise_step",
    "modality_from_state",
]
