"""LTX-2 timestep embeddings and the AdaLN modulation producers on MI355X.

Mirror of ``kinomlx/models/ltx2/transformer/timestep.py`` (``get_timestep_embedding``,
``TimestepEmbedding``, ``CombinedTimestepEmbeddings``, ``AdaLayerNormSingle``). The sinusoidal
features come from one HIP kernel that writes the hidden dtype directly (the reference's FP32
features followed by ``.astype``: the same single rounding); the MLP's first SiLU runs in the
GEMM epilogue; the second SiLU (the embedding itself is also an output) is the SiLU kernel.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from ..kernels.fused_ops import silu
from .attention import Linear


def get_timestep_embedding(timesteps: torch.Tensor, embedding_dim: int = 256, *, max_period: int = 10000,
                           out_dtype: torch.dtype = torch.float32, time_scale: float = 1.0) -> torch.Tensor:
    """Cosine-then-sine timestep features ``(N, embedding_dim)`` (``timestep.py:13-28``).

    ``out_dtype`` (fp32 or bf16) is the dtype the features are stored in, after the FP32
    arithmetic; ``time_scale`` multiplies the timesteps first, in FP32 (the preprocessor's
    ``value * timestep_scale``, ``preprocessing.py:66-75``).
    """
    if timesteps.dim() != 1:
        raise ValueError("timesteps must be a one-dimensional array")
    t = timesteps if timesteps.dtype == torch.float32 else timesteps.float()
    out = torch.empty((t.shape[0], embedding_dim), dtype=out_dtype, device=t.device)
    _lib.launch_timestep_embedding(t.contiguous(), out, -math.log(max_period), time_scale)
    return out


class TimestepEmbedding:
    """``linear_2(silu(linear_1(features)))`` over the sinusoidal features, with SiLU in the
    first GEMM's epilogue (``timestep.py:31-49``).
    ``linear_1`` and ``linear_2`` (``Linear`` with biases) are assigned after construction."""

    def __init__(self, embedding_dim: int) -> None:
        self.embedding_dim = embedding_dim
        self.linear_1: Linear | None = None
        self.linear_2: Linear | None = None

    def __call__(self, timestep: torch.Tensor, hidden_dtype: torch.dtype, *, time_scale: float = 1.0) -> torch.Tensor:
        if hidden_dtype != torch.bfloat16:
            raise ValueError(f"the MI355X timestep MLP runs in bfloat16, got {hidden_dtype}")
        value = get_timestep_embedding(timestep, out_dtype=hidden_dtype, time_scale=time_scale)
        # silu(linear_1(x)): the SiLU is applied to the FP32 accumulator before the one rounding
        value = self.linear_1(value, activation="silu")
        value = self.linear_2(value)
        if value.shape[-1] != self.embedding_dim:
            raise ValueError(
                f"timestep embedding produced width {value.shape[-1]}, expected {self.embedding_dim}"
            )
        return value


class CombinedTimestepEmbeddings:
    """Holds the timestep MLP under the attribute path the checkpoint keys use
    (``emb.timestep_embedder``; ``timestep.py:52-60``)."""

    def __init__(self, embedding_dim: int) -> None:
        self.timestep_embedder = TimestepEmbedding(embedding_dim)

    def __call__(self, timestep: torch.Tensor, hidden_dtype: torch.dtype, *, time_scale: float = 1.0) -> torch.Tensor:
        return self.timestep_embedder(timestep, hidden_dtype, time_scale=time_scale)


class AdaLayerNormSingle:
    """Timestep MLP plus one modulation projection (``timestep.py:63-85``): returns
    ``(linear(silu(embedded)), embedded)``, widths ``num_embeddings * D`` and ``D``. ``linear``
    (with bias) is assigned after construction."""

    def __init__(self, embedding_dim: int, num_embeddings: int) -> None:
        self.embedding_dim = embedding_dim
        self.num_embeddings = num_embeddings
        self.emb = CombinedTimestepEmbeddings(embedding_dim)
        self.linear: Linear | None = None

    def __call__(self, timestep: torch.Tensor, hidden_dtype: torch.dtype, *,
                 time_scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
        embedded = self.emb(timestep, hidden_dtype, time_scale=time_scale)
        modulation = self.linear(silu(embedded))
        return modulation, embedded


__all__ = [
    "AdaLayerNormSingle",
    "CombinedTimestepEmbeddings",
    "TimestepEmbedding",
    "get_timestep_embedding",
]
