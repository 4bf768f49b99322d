"""Dense (non-causal) flash attention for unmasked attention calls, on gfx950 MFMA.

Mirror of ``kinomlx/models/ltx2/kernels/dense_attention.py`` (``HEAD_DIMS``, ``applies``,
``dense_attention``). Queries are token-major ``(query_tokens, heads * dim)`` and keys/values
``(key_tokens, heads * dim)`` — the layout of the projections, so neither side needs a head
transpose and self- and cross-attention are the same call. q, k and v are float16 or bfloat16,
multiplied on MFMA in that type (P rounded to it too); scores and accumulation are FP32, and the
output has the queries' shape and dtype (``dense_attention.py:47,112-116``).

Differences from the M1 kernel, by design: bf16 inputs stay bf16 (no FP16 saturation step:
MI355X multiplies bf16 natively, so values beyond the FP16 range stay finite without a clip), and
64-wide heads take the kernel at any token count (the reference's 512-token floor was an M1 speed
heuristic against MLX's SDPA).
"""

from __future__ import annotations

import torch

from .. import _lib

HEAD_DIMS = (64, 128)
_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)


def applies(query: torch.Tensor, key: torch.Tensor, *, heads: int) -> bool:
    """Whether flattened-head ``(batch, tokens, heads * dim)`` queries and keys take the kernel
    (contract of ``dense_attention.py:87-104``)."""
    return (
        query.dim() == 3
        and key.dim() == 3
        and query.dtype in _SUPPORTED_DTYPES
        and key.dtype == query.dtype
        and query.shape[0] == key.shape[0]
        and query.shape[-1] == key.shape[-1]
        and heads > 0
        and query.shape[-1] in tuple(heads * d for d in HEAD_DIMS)
        and query.shape[1] > 0
        and key.shape[1] > 0
        and query.is_cuda
        and _lib.available()
    )


def score_bias(mask: torch.Tensor, *, batch: int, heads: int, tq: int, tk: int,
               dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, tuple]:
    """An SDPA mask as the kernel's additive bias (in ``dtype``, the queries' type) and its
    (batch, head, query) strides.

    Shapes follow ``_prepare_attention_mask`` (``attention.py:136-141``): ``(Tq, Tk)`` is shared
    by every batch and head, ``(B, Tq, Tk)`` by every head, ``(B | 1, H | 1, Tq | 1, Tk)`` as
    given. A boolean mask keeps its True keys (False -> -inf); other dtypes are cast to ``dtype``
    and added to the scaled scores. Broadcast axes get stride 0; rows are padded to a multiple of 4
    keys when the layout needs it."""
    if mask.dim() == 2:
        mask = mask[None, None]
    elif mask.dim() == 3:
        mask = mask[:, None]
    if mask.dim() != 4 or mask.shape[-1] != tk:
        raise ValueError(f"attention mask must end in the key axis ({tk}), got {tuple(mask.shape)}")
    for axis, full in zip(range(3), (batch, heads, tq)):
        if mask.shape[axis] not in (1, full):
            raise ValueError(f"attention mask {tuple(mask.shape)} does not broadcast to ({batch}, {heads}, {tq}, {tk})")
    if mask.dtype == torch.bool:
        mask = torch.where(mask, 0.0, float("-inf"))
    mask = mask.to(dtype)
    strides = [mask.stride(a) if mask.shape[a] != 1 else 0 for a in range(3)]
    if mask.stride(-1) != 1 or any(st % 4 for st in strides) or mask.data_ptr() % 8:
        padded = torch.zeros((*mask.shape[:3], (tk + 3) // 4 * 4), dtype=dtype, device=mask.device)
        padded[..., :tk] = mask
        mask = padded
        strides = [mask.stride(a) if mask.shape[a] != 1 else 0 for a in range(3)]
    return mask, tuple(strides)


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, heads: int, batch: int,
               tq: int, tk: int, dim: int, gate: torch.Tensor | None, scale: float | None,
               out: torch.Tensor | None = None, kv_heads: int | None = None,
               mask: torch.Tensor | None = None) -> torch.Tensor:
    if out is None:
        out = torch.empty((batch, tq, heads * dim), dtype=q.dtype, device=q.device)
    elif (out.dtype != q.dtype or tuple(out.shape) != (batch, tq, heads * dim) or out.stride(-1) != 1
          or (batch > 1 and out.stride(0) != tq * out.stride(1))):
        raise ValueError(f"attention out must be {q.dtype} ({batch}, {tq}, {heads * dim}) with contiguous rows")
    if gate is not None:
        if gate.dtype != q.dtype or tuple(gate.shape[-1:]) != (heads,):
            raise ValueError(f"attention gate must be {q.dtype} (..., {heads})")
        gate = gate.reshape(batch * tq, heads)
    bias = strides = None
    if mask is not None:
        bias, strides = score_bias(mask, batch=batch, heads=heads, tq=tq, tk=tk, dtype=q.dtype)
    _lib.launch_attention(
        q, k, v, out, batch=batch, tq=tq, tk=tk, heads=heads, head_dim=dim,
        scale=dim ** -0.5 if scale is None else scale, gate=gate, kv_heads=kv_heads, bias=bias, bias_strides=strides,
    )
    return out


def _check(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, width: int) -> int:
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(
            f"dense attention needs float16 or bfloat16 q, k and v, got {q.dtype}, {k.dtype}, {v.dtype}"
        )
    dim = width // heads if heads > 0 and width % heads == 0 else 0
    return dim


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, heads: int,
                    gate: torch.Tensor | None = None) -> torch.Tensor:
    """Dense attention of ``(query_tokens, heads * dim)`` queries over ``(key_tokens, ...)``
    (``dense_attention.py:106-153``). ``dim`` is 64 or 128. ``gate`` (optional, the queries' dtype,
    ``(query_tokens, heads)``) multiplies each head's output before the one rounding."""
    width = q.shape[1] if q.dim() == 2 else 0
    dim = _check(q, k, v, heads, width)
    if (
        dim not in HEAD_DIMS
        or k.dim() != 2
        or k.shape[1] != width
        or v.shape != k.shape
        or q.shape[0] == 0
        or k.shape[0] == 0
    ):
        raise ValueError(
            f"dense attention needs (query_tokens, {heads} * 64 or 128) queries and matching "
            f"(key_tokens, width) keys and values, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}"
        )
    out = _attention(q, k, v, heads=heads, batch=1, tq=q.shape[0], tk=k.shape[0], dim=dim,
                     gate=gate, scale=None)
    return out[0]


def batched_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, heads: int,
                      gate: torch.Tensor | None = None, scale: float | None = None,
                      out: torch.Tensor | None = None, kv_heads: int | None = None,
                      mask: torch.Tensor | None = None) -> torch.Tensor:
    """``(batch, tokens, heads * dim)`` form of ``dense_attention``; q/k/v (and ``out``, when
    given) may be strided row views, e.g. column slices of a fused QKV projection or of the
    buffer the next projection reads. With ``kv_heads`` (grouped-query attention) k and v hold
    ``kv_heads * dim`` columns and query head ``h`` reads key/value head
    ``h // (heads // kv_heads)``. ``mask`` is the SDPA mask (``score_bias``)."""
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape or q.shape[0] != k.shape[0]:
        raise ValueError("batched attention needs (batch, tokens, heads * dim) q, k and v")
    width = q.shape[-1]
    dim = _check(q, k, v, heads, width)
    groups = heads if kv_heads is None else kv_heads
    if groups <= 0 or heads % groups:
        raise ValueError(f"{heads} query heads do not group over {groups} key/value heads")
    if dim not in HEAD_DIMS or k.shape[-1] != groups * dim:
        raise ValueError(f"attention head width must be 64 or 128, got {width} / {heads}")
    batch, tq, tk = q.shape[0], q.shape[1], k.shape[1]
    if tk == 0:
        raise ValueError("attention needs at least one key")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.stride(-1) != 1 or (batch > 1 and t.stride(0) != t.shape[1] * t.stride(1)):
            raise ValueError(f"attention {name} must have contiguous rows, evenly strided over the batch")
    return _attention(q, k, v, heads=heads, batch=batch, tq=tq, tk=tk, dim=dim, gate=gate, scale=scale, out=out,
                      kv_heads=kv_heads, mask=mask)


__all__ = ["HEAD_DIMS", "applies", "batched_attention", "dense_attention", "score_bias"]
