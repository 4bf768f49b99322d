"""Split rotary embeddings for LTX-2 tokens on MI355X.

Mirror of ``kinomlx/models/ltx2/transformer/rope.py``: ``LTXRopeType``,
``apply_split_rotary_emb``, ``apply_rotary_emb``, ``precompute_freqs_cis``. Tables are built on
the positions' device in FP32 token-major storage and returned as head-major
``(B, H, T, dim / (2H))`` views, the layout the split-RoPE kernel reads without a copy.
"""

from __future__ import annotations

import math
from enum import Enum
from functools import lru_cache

import torch

from ..kernels import split_rope


class LTXRopeType(Enum):
    """Position-embedding layouts supported by the LTX-2 graphs."""

    SPLIT = "split"


def apply_split_rotary_emb(value: torch.Tensor, cos_freqs: torch.Tensor, sin_freqs: torch.Tensor) -> torch.Tensor:
    """Split-half RoPE preserving the activation dtype (``rope.py:18-61``).

    Flattened-head ``(B, T, H * Dh)`` activations take the kernel directly; head-major
    ``(B, H, T, Dh)`` activations are laid out token-major around the same kernel.
    """
    if cos_freqs.shape != sin_freqs.shape:
        raise ValueError("RoPE cosine and sine tensors must have matching shapes")
    if split_rope.applies(value, cos_freqs, sin_freqs):
        return split_rope.rotate(value, cos_freqs, sin_freqs)
    if value.dim() == 4 and cos_freqs.dim() == 4:
        batch, heads, tokens, head_dim = value.shape
        if head_dim % 2:
            raise ValueError("split RoPE requires an even head dimension")
        flat = value.transpose(1, 2).reshape(batch, tokens, heads * head_dim)
        rotated = split_rope.rotate(flat, cos_freqs, sin_freqs)
        return rotated.reshape(batch, tokens, heads, head_dim).transpose(1, 2)
    raise ValueError("the RoPE kernel does not apply to these activations and tables")


def apply_rotary_emb(value: torch.Tensor, freqs_cis: tuple[torch.Tensor, torch.Tensor],
                     rope_type: LTXRopeType = LTXRopeType.SPLIT) -> torch.Tensor:
    """Apply a checkpoint-selected RoPE layout (``rope.py:64-72``)."""
    if rope_type is not LTXRopeType.SPLIT:
        raise ValueError(f"unsupported RoPE type: {rope_type}")
    return apply_split_rotary_emb(value, *freqs_cis)


@lru_cache(maxsize=8)
def _frequency_grid(theta: float, position_dims: int, inner_dim: int, double_precision: bool) -> tuple[float, ...]:
    """``theta ** (j / (n - 1)) * pi / 2`` in host double precision (``rope.py:75-92``)."""
    count = inner_dim // (2 * position_dims)
    if count <= 0:
        raise ValueError("RoPE dimension is too small for its position axes")
    exponents = (0.0,) if count == 1 else tuple(i / (count - 1) for i in range(count))
    del double_precision
    return tuple(math.pow(theta, e) * math.pi / 2 for e in exponents)


def _fractional_positions(positions: torch.Tensor, max_pos: tuple[int, ...], *,
                          use_middle_indices_grid: bool) -> torch.Tensor:
    """``(B, axes, T[, 2])`` positions -> ``(B, T, axes)`` FP32 fractions (``rope.py:95-112``)."""
    if positions.shape[1] != len(max_pos):
        raise ValueError("position axes must match max_pos")
    if use_middle_indices_grid:
        if positions.dim() != 4 or positions.shape[-1] != 2:
            raise ValueError("middle-position RoPE expects (B, axes, T, 2) bounds")
        positions = (positions[..., 0].float() + positions[..., 1].float()) / 2.0
    elif positions.dim() == 4:
        positions = positions[..., 0]
    elif positions.dim() != 3:
        raise ValueError("RoPE positions must have three or four dimensions")
    scale = torch.tensor(max_pos, dtype=torch.float32, device=positions.device)[None, :, None]
    return (positions.float() / scale).transpose(1, 2)


def precompute_freqs_cis(
    indices_grid: torch.Tensor,
    *,
    dim: int,
    out_dtype: torch.dtype = torch.float32,
    theta: float = 10000.0,
    max_pos: tuple[int, ...] | list[int] = (20, 2048, 2048),
    use_middle_indices_grid: bool = False,
    num_attention_heads: int = 32,
    rope_type: LTXRopeType = LTXRopeType.SPLIT,
    use_double_precision: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Split-RoPE cosine/sine tables for one token grid (``rope.py:115-176``)."""
    if rope_type is not LTXRopeType.SPLIT:
        raise ValueError(f"unsupported RoPE type: {rope_type}")
    if dim % num_attention_heads:
        raise ValueError("RoPE dimension must divide evenly across attention heads")
    resolved = tuple(max_pos)
    fractional = _fractional_positions(indices_grid, resolved, use_middle_indices_grid=use_middle_indices_grid)
    grid = torch.tensor(
        _frequency_grid(theta, indices_grid.shape[1], dim, use_double_precision),
        dtype=torch.float32, device=indices_grid.device,
    )
    scaled = fractional * 2.0 - 1.0
    frequencies = scaled[..., None] * grid[None, None, None, :]  # (B, T, axes, n)
    batch, tokens = frequencies.shape[0], frequencies.shape[1]
    frequencies = frequencies.transpose(2, 3).reshape(batch, tokens, -1)
    padding = dim // 2 - frequencies.shape[-1]
    if padding < 0:
        raise ValueError("RoPE frequency grid exceeds half the model dimension")
    cos = torch.cos(frequencies)
    sin = torch.sin(frequencies)
    if padding:
        cos = torch.cat([torch.ones((batch, tokens, padding), dtype=cos.dtype, device=cos.device), cos], dim=-1)
        sin = torch.cat([torch.zeros((batch, tokens, padding), dtype=sin.dtype, device=sin.device), sin], dim=-1)
    cos = cos.reshape(batch, tokens, num_attention_heads, -1).to(out_dtype).contiguous()
    sin = sin.reshape(batch, tokens, num_attention_heads, -1).to(out_dtype).contiguous()
    return cos.transpose(1, 2), sin.transpose(1, 2)


__all__ = ["LTXRopeType", "apply_rotary_emb", "apply_split_rotary_emb", "precompute_freqs_cis"]
