"""LTX-2 attention on MI355X: gated multi-head attention with full-width Q/K RMSNorm and split
RoPE.

Mirror of ``kinomlx/models/ltx2/transformer/attention.py`` (``Attention``, ``RMSNorm``,
``rms_norm``, ``scaled_dot_product_attention``, ``dense_kernel_attention``). The call sequence of
``Attention.__call__`` (``:291-371``) is kept; the MI355X schedule fuses it into:

* one MFMA GEMM for Q, K and V when the projections are fused (``fuse_projections``: one
  ``(3 * inner, in)`` weight whose row blocks back ``to_q``/``to_k``/``to_v``), writing one
  ``(T, 3 * inner)`` buffer whose column slices feed the next kernels without copies;
* the gate logits GEMM with ``2 * sigmoid`` in its epilogue;
* one pass over Q and K together for the weighted RMSNorms and the split RoPE (FP32 throughout;
  the fp32 RoPE tables, as large as Q and K together, are read once);
* the flash-attention kernel with the per-head gate applied before its one rounding;
* the output GEMM, optionally with the block's gated residual in its epilogue.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..kernels import fused_ops, mpp_linear, split_rope
from ..kernels.quantized import PretransposedQuantizedLinear, QuantizedLinear
from . import dense_attention as _dense
from .rope import LTXRopeType


class Linear:
    """``nn.Linear`` counterpart: ``(out, in)`` bf16 weight and optional bias;
    ``layer(x) = addmm(bias, x, W^T)`` through the MFMA kernel, with the kernel's epilogues."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        self.weight = weight
        self.bias = bias

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[1])

    def __call__(self, value: torch.Tensor, *, activation: str | None = None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        return mpp_linear.fused_linear(value, self.weight, self.bias, activation=activation,
                                       residual=residual, gate=gate, out=out, out_dtype=out_dtype)


def rms_norm(value: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """Central RMSNorm precision policy (``attention.py:112-118``)."""
    return fused_ops.rms_norm(value, weight, eps)


class RMSNorm:
    """RMS normalization with a checkpoint-backed scale vector (``attention.py:121-133``)."""

    def __init__(self, dims: int, *, eps: float = 1e-6, weight: torch.Tensor | None = None) -> None:
        self.dims = dims
        self.eps = eps
        self.weight = weight

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        if value.shape[-1] != self.dims:
            raise ValueError(f"RMSNorm expects width {self.dims}, got {value.shape[-1]}")
        return rms_norm(value, self.weight, self.eps)


def _fused_norm_rope_ok(dim: int, head_dim: int) -> bool:
    return dim % 512 == 0 and dim // 512 in (1, 2, 4, 8) and head_dim >= 16 and 512 % head_dim == 0


def norm_rope(value: torch.Tensor, norm: RMSNorm, pe: tuple[torch.Tensor, torch.Tensor] | None,
              heads: int) -> torch.Tensor:
    """Weighted RMSNorm over the full width, then split RoPE on the normalized value; one pass
    when the shape allows (``attention.py:353-359`` then ``rope.py:18-61``)."""
    batch, tokens, dim = value.shape
    head_dim = dim // heads
    out = torch.empty((batch, tokens, dim), dtype=value.dtype, device=value.device)
    if out.numel() == 0:
        return out
    if pe is None:
        _lib.launch_rmsnorm_rope(value, out, norm.weight, norm.eps, 0.0, norm_width=dim)
        return out
    cos, sin = pe
    if not (cos.dim() == 4 and cos.shape[1] == heads and cos.shape[2] == tokens and cos.shape[3] * 2 == head_dim
            and cos.shape[0] in (1, batch) and cos.dtype == torch.float32 and cos.shape == sin.shape):
        raise ValueError("RoPE tables must be fp32 (1 or batch, heads, tokens, head_dim / 2)")
    if _fused_norm_rope_ok(dim, head_dim):
        cos_tm, sin_tm = split_rope.token_major(cos), split_rope.token_major(sin)
        _lib.launch_rmsnorm_rope(
            value, out, norm.weight, norm.eps, 0.0, norm_width=dim, rope_kind=_lib.KX_ROPE_SPLIT,
            cos=cos_tm, sin=sin_tm, table_ld=heads * head_dim // 2, table_hs=head_dim // 2,
            tokens=tokens, table_batched=cos.shape[0] > 1, head_dim=head_dim,
        )
        return out
    _lib.launch_rmsnorm_rope(value, out, norm.weight, norm.eps, 0.0, norm_width=dim)
    return split_rope.rotate(out, cos, sin)


def norm_rope_qk(q_raw: torch.Tensor, k_raw: torch.Tensor, q_norm: RMSNorm, k_norm: RMSNorm,
                 pe: tuple[torch.Tensor, torch.Tensor], heads: int):
    """``(norm_rope(q), norm_rope(k))`` for Q and K of the same tokens and tables in one pass
    (the tables are read once); None when the fused kernel does not take the shape."""
    batch, tokens, dim = q_raw.shape
    head_dim = dim // heads
    cos, sin = pe
    if (head_dim != 128 or q_norm.weight is None or k_norm.weight is None or q_norm.eps != k_norm.eps
            or q_norm.weight.dtype != k_norm.weight.dtype or not (cos.dim() == 4 and cos.shape[1] == heads
            and cos.shape[2] == tokens and cos.shape[3] * 2 == head_dim and cos.shape[0] in (1, batch)
            and cos.dtype == torch.float32 and cos.shape == sin.shape)):
        return None
    q = torch.empty((batch, tokens, dim), dtype=q_raw.dtype, device=q_raw.device)
    k = torch.empty_like(q)
    if q.numel() == 0:
        return q, k
    cos_tm, sin_tm = split_rope.token_major(cos), split_rope.token_major(sin)
    if not _lib.launch_qk_rmsnorm_rope(q_raw, k_raw, q, k, q_norm.weight, k_norm.weight, q_norm.eps, cos=cos_tm,
                                       sin=sin_tm, table_ld=heads * head_dim // 2, table_hs=head_dim // 2,
                                       tokens=tokens, table_batched=cos.shape[0] > 1):
        return None
    return q, k


def dense_kernel_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, heads: int,
                           gate: torch.Tensor | None = None) -> torch.Tensor:
    """The flash-attention kernel on flattened-head ``(batch, tokens, heads * dim)`` inputs;
    keys and values may have their own token count (``attention.py:192-206``)."""
    return _dense.batched_attention(query, key, value, heads=heads, gate=gate)


def scaled_dot_product_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, heads: int,
                                 dim_head: int, mask: torch.Tensor | None = None,
                                 compile_attention: bool = True) -> torch.Tensor:
    """Attention on flattened-head inputs (``attention.py:224-246``); ``mask`` is the SDPA mask
    (``_prepare_attention_mask``, ``:136-141``), added to the scores inside the kernel."""
    del compile_attention
    if query.shape[-1] != heads * dim_head:
        raise ValueError("query width must be heads * dim_head")
    return _dense.batched_attention(query, key, value, heads=heads, mask=mask)


def _cat_layers(layers):
    """One fused layer whose output row blocks are ``layers`` in order, and views back into it.
    Dense layers (and pretransposed mxfp8 layers, which run on their exact bf16 dequantization)
    fuse into one dense layer; quantized layers of one mode and format into one quantized layer
    (their packed rows, scales and biases are per output row)."""
    if all(isinstance(layer, (Linear, PretransposedQuantizedLinear)) for layer in layers):
        def dense(layer):
            return layer.weight if isinstance(layer, Linear) else layer._dense

        if any(dense(layer) is None for layer in layers):
            return None
        weight = torch.cat([dense(layer) for layer in layers], dim=0).contiguous()
        has_bias = [layer.bias is not None for layer in layers]
        bias = None
        if any(has_bias):
            bias = torch.cat([
                layer.bias.to(weight.dtype) if layer.bias is not None else
                torch.zeros(layer.out_features, dtype=weight.dtype, device=weight.device)
                for layer in layers
            ]).contiguous()
        fused = Linear(weight, bias)
        start = 0
        for layer in layers:
            stop = start + layer.out_features
            if isinstance(layer, Linear):
                layer.weight = weight[start:stop]
            else:
                layer._dense = weight[start:stop]
            if layer.bias is not None:
                layer.bias = bias[start:stop]
            start = stop
        return fused
    if all(isinstance(layer, QuantizedLinear) for layer in layers):
        first = layers[0]
        if any((layer.mode, layer.bits, layer.group_size) != (first.mode, first.bits, first.group_size)
               for layer in layers):
            return None
        words = torch.cat([layer.weight for layer in layers], dim=0).contiguous()
        scales = torch.cat([layer.scales for layer in layers], dim=0).contiguous()
        biases = None if first.biases is None else torch.cat([layer.biases for layer in layers], dim=0).contiguous()
        bias = None
        if any(layer.bias is not None for layer in layers):
            bias = torch.cat([
                layer.bias.to(torch.bfloat16) if layer.bias is not None else
                torch.zeros(layer.out_features, dtype=torch.bfloat16, device=words.device)
                for layer in layers
            ]).contiguous()
        return QuantizedLinear(words, scales, biases, bias, group_size=first.group_size, bits=first.bits,
                               mode=first.mode)
    return None


def _dense_weight(layer):
    """The bf16 ``(out, in)`` weight a layer multiplies by (a quantized layer's exact
    dequantization), or None for a layer of another kind."""
    if isinstance(layer, Linear):
        return layer.weight
    if isinstance(layer, PretransposedQuantizedLinear):
        return layer._dense
    if isinstance(layer, QuantizedLinear) and layer.weight.is_cuda:
        return layer._dense if layer._dense is not None else layer.dequantized()
    return None


def qknorm_rope_projection(layer, value: torch.Tensor, out: torch.Tensor, *, q_width: int, k_width: int,
                           norm_q: torch.Tensor, norm_k: torch.Tensor, eps: float, weight_offset: float,
                           cos: torch.Tensor, sin: torch.Tensor) -> bool:
    """``out = layer(value)`` with the query columns ``[0, q_width)`` and key columns
    ``[q_width, q_width + k_width)`` normalized per 128-wide head (``(x * rsqrt(mean(x^2) + eps))
    * (w + weight_offset)`` of the bf16 projection) and rotated in adjacent pairs, all in the GEMM's
    epilogue (``kx_gemm_qknorm_rope_bf16``). ``value`` ``(R, in)`` and ``out`` ``(R, out)`` are the
    rows of ``R / T`` sequences of ``T`` tokens; ``cos``/``sin`` are their fp32 tables, ``(T, 128)``
    or ``(1 | R / T, T, 128)``, with unit-stride rows. Returns False (nothing written) when the layer
    or the shapes do not take this path; the caller then runs the separate passes."""
    weight = _dense_weight(layer)
    if (weight is None or weight.dtype != torch.bfloat16 or value.dtype != torch.bfloat16 or value.dim() != 2
            or out.dim() != 2 or cos.dim() not in (2, 3) or cos.shape != sin.shape or cos.stride() != sin.stride()):
        return False
    rows, k = int(value.shape[0]), int(value.shape[1])
    n = int(weight.shape[0])
    tokens = int(cos.shape[-2])
    batches = 1 if cos.dim() == 2 else int(cos.shape[0])
    if (rows == 0 or tokens == 0 or rows % tokens or batches not in (1, rows // tokens) or cos.shape[-1] != 128
            or q_width % 128 or k_width % 128 or q_width + k_width > n or k % 64 or int(weight.shape[1]) != k
            or norm_q.shape != (128,) or norm_k.shape != (128,) or norm_q.dtype != norm_k.dtype
            or cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.stride(-1) != 1
            or cos.stride(-2) % 4 or (batches > 1 and cos.stride(0) % 4) or cos.data_ptr() % 16
            or sin.data_ptr() % 16 or tuple(out.shape) != (rows, n) or out.dtype != torch.bfloat16
            or out.stride(-1) != 1 or out.stride(0) % 4 or out.data_ptr() % 8):
        return False
    a = value if value.stride(-1) == 1 and value.stride(0) % 8 == 0 and value.data_ptr() % 16 == 0 else value.contiguous()
    bias = getattr(layer, "bias", None)
    bias = None if bias is None else bias.to(torch.bfloat16).contiguous()
    _lib.launch_gemm_qknorm_rope(a, weight, out, bias=bias, q_end=q_width, k_end=q_width + k_width,
                                 norm_q=norm_q.contiguous(), norm_k=norm_k.contiguous(), eps=eps,
                                 weight_offset=weight_offset, cos=cos, sin=sin, table_ld=int(cos.stride(-2)),
                                 table_hs=0, table_rows=tokens, table_bs=int(cos.stride(0)) if batches > 1 else 0)
    return True


class Attention:
    """Multi-head attention with Q/K RMSNorm, split RoPE and per-head gates
    (``attention.py:249-371``). Weights are assigned after construction, as the reference's
    loader does: ``to_q``/``to_k``/``to_v``/``to_out``/``to_gate_logits`` hold ``Linear`` or
    ``QuantizedLinear`` layers and ``q_norm.weight``/``k_norm.weight`` the norm scales."""

    def __init__(
        self,
        query_dim: int,
        *,
        heads: int = 8,
        dim_head: int = 64,
        context_dim: int | None = None,
        rope_type: LTXRopeType = LTXRopeType.SPLIT,
        norm_eps: float = 1e-6,
        apply_gated_attention: bool = False,
        compile_attention: bool = True,
        dense_kernel: bool = True,
    ) -> None:
        if heads <= 0 or dim_head <= 0:
            raise ValueError("attention heads and head dimension must be positive")
        self.heads = heads
        self.dim_head = dim_head
        self.query_dim = query_dim
        self.context_dim = query_dim if context_dim is None else context_dim
        self.rope_type = rope_type
        self.compile_attention = compile_attention
        self.dense_kernel = dense_kernel
        self.apply_gated_attention = apply_gated_attention
        inner = heads * dim_head
        self.q_norm = RMSNorm(inner, eps=norm_eps)
        self.k_norm = RMSNorm(inner, eps=norm_eps)
        self.to_q = self.to_k = self.to_v = self.to_out = None
        self.to_gate_logits = None
        self._qkv = None
        self._kv = None

    def fuse_projections(self, *, self_attention: bool = True) -> None:
        """Concatenate Q/K/V (self-attention) or K/V (cross-attention on a context) into one
        weight; the per-projection layers become views into it (no extra memory for dense
        weights)."""
        if self_attention:
            self._qkv = _cat_layers([self.to_q, self.to_k, self.to_v])
        else:
            self._kv = _cat_layers([self.to_k, self.to_v])

    def project(self, value: torch.Tensor, *, context: torch.Tensor | None = None,
                pe=None, k_pe=None):
        """Gate, normalized/rotated Q and K, and V, as the kernel reads them."""
        if value.shape[-1] != self.query_dim:
            raise ValueError(f"attention query expects width {self.query_dim}, got {value.shape[-1]}")
        gate = None
        if self.to_gate_logits is not None:
            gate = self.to_gate_logits(value, activation="sigmoid2")
        source = value if context is None else context
        if source.shape[-1] != self.context_dim:
            raise ValueError(f"attention context expects width {self.context_dim}, got {source.shape[-1]}")
        inner = self.heads * self.dim_head
        if context is None and self._qkv is not None:
            qkv = self._qkv(value)
            q_raw, k_raw, v = qkv[..., :inner], qkv[..., inner:2 * inner], qkv[..., 2 * inner:]
        else:
            q_raw = self.to_q(value)
            if self._kv is not None:
                kv = self._kv(source)
                k_raw, v = kv[..., :inner], kv[..., inner:]
            else:
                k_raw, v = self.to_k(source), self.to_v(source)
        if pe is not None and k_pe is None and k_raw.shape == q_raw.shape:
            qk = norm_rope_qk(q_raw, k_raw, self.q_norm, self.k_norm, pe, self.heads)
            if qk is not None:
                return gate, qk[0], qk[1], v
        q = norm_rope(q_raw, self.q_norm, pe, self.heads)
        k = norm_rope(k_raw, self.k_norm, pe if k_pe is None else k_pe, self.heads) if pe is not None else \
            norm_rope(k_raw, self.k_norm, None, self.heads)
        return gate, q, k, v

    def attend(self, value: torch.Tensor, *, context: torch.Tensor | None = None,
               mask: torch.Tensor | None = None, pe=None, k_pe=None) -> torch.Tensor:
        """Everything before the output projection (gated attention output ``(B, T, inner)``)."""
        gate, q, k, v = self.project(value, context=context, pe=pe, k_pe=k_pe)
        return _dense.batched_attention(q, k, v, heads=self.heads, gate=gate, mask=mask)

    def __call__(self, value: torch.Tensor, *, context: torch.Tensor | None = None,
                 mask: torch.Tensor | None = None, pe=None, k_pe=None, sparse=None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """``to_out(attention)``; with ``residual``/``gate`` the block's gated residual
        ``residual + gate * to_out(attention)`` is formed in the output GEMM's epilogue, written
        as ``out_dtype`` (default the input dtype; fp32 carries the residual stream unrounded)."""
        if sparse is not None:
            raise ValueError("sparse (Sol-Attn) attention is not built for MI355X")
        attended = self.attend(value, context=context, mask=mask, pe=pe, k_pe=k_pe)
        return self.to_out(attended, residual=residual, gate=gate, out_dtype=out_dtype)


__all__ = [
    "Attention",
    "Linear",
    "RMSNorm",
    "dense_kernel_attention",
    "norm_rope",
    "norm_rope_qk",
    "qknorm_rope_projection",
    "rms_norm",
    "scaled_dot_product_attention",
]
