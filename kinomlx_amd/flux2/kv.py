"""FLUX.2 attention entry point on MI355X (mirror of ``kinomlx/models/flux2/kv.py:48-54``).

``attend`` takes ``(batch, tokens, heads, head_dim)`` queries, keys and values, as the FLUX.2
blocks produce them, and returns the same layout. The flattened-head form of that layout is
exactly what the flash-attention kernel reads, so the reference's transposes to and from
``(batch, heads, tokens, head_dim)`` disappear: no copy is made on either side.
"""

from __future__ import annotations

import torch

from ..ltx2 import dense_attention as _dense


def _flat(value: torch.Tensor, name: str) -> torch.Tensor:
    if value.dim() != 4:
        raise ValueError(f"attend takes (batch, tokens, heads, head_dim) {name}, got {tuple(value.shape)}")
    if value.stride(-1) != 1 or value.stride(-2) != value.shape[-1]:
        raise ValueError(f"attend {name} must have contiguous heads")
    return value.flatten(2)


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """Non-causal ``softmax(q k^T / sqrt(head_dim)) v`` per head; scale ``head_dim ** -0.5``."""
    heads, head_dim = int(query.shape[-2]), int(query.shape[-1])
    if key.shape[-2:] != query.shape[-2:] or value.shape != key.shape:
        raise ValueError("attend: keys and values must match the queries' heads and head width")
    out = _dense.batched_attention(_flat(query, "query"), _flat(key, "key"), _flat(value, "value"), heads=heads,
                                   scale=head_dim ** -0.5)
    return out.view(*query.shape)


__all__ = ["attend"]
