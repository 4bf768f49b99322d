"""Split-half rotary position embedding in one pass on MI355X.

Mirror of ``kinomlx/kernels/split_rope.py`` (``set_enabled``, ``enabled``, ``available``,
``applies``, ``rotate``). Flattened-head activations ``(batch, tokens, heads * dim)`` are rotated
by FP32 head-major tables ``(1 or batch, heads, tokens, dim / 2)``. Each product is rounded in
FP32 before the difference or sum and one cast, so the result has the bits of the reference's
graph arithmetic (``split_rope.py:35-56``).

The kernel reads the tables token-major, ``(batch, tokens, heads, dim / 2)``: the layout
``precompute_freqs_cis`` builds them in, so its head-major views reach the kernel without a
copy; any other table layout is copied token-major first.
"""

from __future__ import annotations

import torch

from .. import _lib

_DTYPES = (torch.bfloat16, torch.float16)
_enabled = True


def set_enabled(enabled: bool) -> None:
    """Rotate through the kernel wherever it applies (the default). With the kernel switched
    off, ``applies`` is False; there is no other MI355X rotation path."""
    global _enabled
    _enabled = bool(enabled)


def enabled() -> bool:
    """Whether the RoPE kernel is switched on."""
    return _enabled


def available(dtype: torch.dtype) -> bool:
    """Whether the kernel is built, a GPU is visible, and this activation dtype is supported."""
    return dtype in _DTYPES and _lib.available()


def applies(value: torch.Tensor, cos_freqs: torch.Tensor, sin_freqs: torch.Tensor) -> bool:
    """Whether ``rotate`` handles these flattened-head activations and FP32 head-major tables
    (contract of ``kinomlx/kernels/split_rope.py:144-156``)."""
    if not _enabled or value.dim() != 3 or cos_freqs.dim() != 4:
        return False
    if cos_freqs.shape != sin_freqs.shape:
        return False
    if cos_freqs.dtype != torch.float32 or sin_freqs.dtype != torch.float32:
        return False
    table_batch, heads, tokens, half = (int(s) for s in cos_freqs.shape)
    batch = int(value.shape[0])
    if table_batch not in (1, batch) or tuple(value.shape) != (batch, tokens, heads * 2 * half):
        return False
    if not (value.is_cuda and cos_freqs.is_cuda and sin_freqs.is_cuda):
        return False
    return available(value.dtype)


def token_major(table: torch.Tensor) -> torch.Tensor:
    """``(B, H, T, half)`` head-major table -> contiguous ``(B, T, H, half)`` storage (a view
    when the table already is a transpose of token-major data)."""
    tm = table.transpose(1, 2)
    return tm if tm.is_contiguous() else tm.contiguous()


def rotate(value: torch.Tensor, cos_freqs: torch.Tensor, sin_freqs: torch.Tensor) -> torch.Tensor:
    """Rotate each head's halves of ``value`` by the tables, keeping the reference's bits."""
    if not applies(value, cos_freqs, sin_freqs):
        raise ValueError("the RoPE kernel does not apply to these activations and tables")
    table_batch, heads, tokens, half = (int(s) for s in cos_freqs.shape)
    batch = int(value.shape[0])
    out = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    if out.numel() == 0:
        return out
    _lib.launch_rope_split(
        value, out, token_major(cos_freqs), token_major(sin_freqs), batch=batch, tokens=tokens,
        heads=heads, half=half, table_batched=table_batch == batch and batch > 1,
    )
    return out


__all__ = ["applies", "available", "enabled", "rotate", "set_enabled", "token_major"]
