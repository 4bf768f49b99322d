"""Split rotary embeddings for LTX-2 tokens on MI355X.

Mirror of ``kinomlx/models/ltx2/transformer/rope.py``: ``LTXRopeType``,
``apply_split_rotary_emb``, ``apply_rotary_emb``, ``precompute_freqs_cis``. Tables are built on
the GPU by one HIP kernel in FP32 token-major storage and returned as head-major
``(B, H, T, dim / (2H))`` views, the layout the split-RoPE kernel reads without a copy.
"""

from __future__ import annotations

import math
from enum import Enum
from functools import lru_cache

import torch

from .. import _lib
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


def _position_tensor(positions: torch.Tensor, max_pos: tuple[int, ...], *,
                     use_middle_indices_grid: bool) -> tuple[torch.Tensor, bool]:
    """fp32 contiguous positions for the table kernel and whether it averages the two bounds
    (the argument checks of ``_fractional_positions``, ``rope.py:95-112``)."""
    if positions.shape[1] != len(max_pos):
        raise ValueError("position axes must match max_pos")
    if use_middle_indices_grid:
        if positions.dim() != 4 or positions.shape[-1] != 2:
            raise ValueError("middle-position RoPE expects (B, axes, T, 2) bounds")
    elif positions.dim() not in (3, 4):
        raise ValueError("RoPE positions must have three or four dimensions")
    return positions.float().contiguous(), use_middle_indices_grid


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
    """Split-RoPE cosine/sine tables for one token grid (``rope.py:115-176``), built by one HIP
    kernel: ``(B, H, T, dim / 2H)`` head-major views of token-major ``(B, T, dim / 2)`` fp32
    storage (the layout the norm + RoPE kernels read)."""
    if rope_type is not LTXRopeType.SPLIT:
        raise ValueError(f"unsupported RoPE type: {rope_type}")
    if dim % num_attention_heads:
        raise ValueError("RoPE dimension must divide evenly across attention heads")
    resolved = tuple(max_pos)
    positions, middle = _position_tensor(indices_grid, resolved, use_middle_indices_grid=use_middle_indices_grid)
    grid_values = _frequency_grid(theta, indices_grid.shape[1], dim, use_double_precision)
    half = dim // 2
    if half < len(grid_values) * len(resolved):
        raise ValueError("RoPE frequency grid exceeds half the model dimension")
    device = positions.device
    grid = torch.tensor(grid_values, dtype=torch.float32, device=device)
    scale = torch.tensor(resolved, dtype=torch.float32, device=device)
    batch, tokens = int(positions.shape[0]), int(positions.shape[2])
    cos = torch.empty((batch, tokens, half), dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    _lib.launch_ltx_rope_tables(positions, scale, grid, cos, sin, middle=middle)
    if out_dtype != torch.float32:
        cos, sin = cos.to(out_dtype), sin.to(out_dtype)
    cos = cos.view(batch, tokens, num_attention_heads, -1)
    sin = sin.view(batch, tokens, num_attention_heads, -1)
    return cos.transpose(1, 2), sin.transpose(1, 2)


__all__ = ["LTXRopeType", "apply_rotary_emb", "apply_split_rotary_emb", "precompute_freqs_cis"]
