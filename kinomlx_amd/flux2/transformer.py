"""FLUX.2 transformer blocks on MI355X.

Mirror of ``kinomlx/models/flux2/transformer.py``: ``rotary_positions``, ``rotate``,
``joint_attention``, ``normalized``, ``swiglu``, ``QKNorm``, ``FeedForward``,
``DoubleAttention``, ``DoubleBlock``, ``SingleAttention``, ``SingleBlock`` and ``Modulation``,
with the same names, call signatures and math, on torch tensors. Weights are assigned after
construction, as the reference's loader does; every projection holds a ``Linear`` or a
``QuantizedLinear`` (``(out, in)`` weights, no biases in FLUX.2).

Kernel schedule of one double-stream block (text ``Tt`` + image ``Ti`` tokens, joint order
[text, image] as the reference concatenates them, ``transformer.py:111-121``):

  LayerNorm-modulate(image), LayerNorm-modulate(text)
  -> image QKV GEMM and text QKV GEMM writing the rows of one joint ``(T, 3D)`` buffer
  -> per-head QKNorm + adjacent-pair RoPE, one pass per stream and per Q/K, writing the joint
     Q and K buffers (the ``concatenate`` calls become row offsets, and the reference's
     separate norm and rotate passes become one FP32 pass)
  -> flash attention over the joint sequence (V read in place from the QKV buffer)
  -> to_out / to_add_out GEMMs with ``x + gate * .`` in their epilogues (FP32 residual stream)
  -> LayerNorm-modulate -> linear_in GEMM -> SwiGLU -> linear_out GEMM (+ x + gate * .)

A single-stream block runs its fused ``to_qkv_mlp_proj`` GEMM once, normalizes and rotates Q
and K from column slices of it, writes the attention output and ``swiglu(mlp)`` side by side
into the one buffer ``to_out`` reads (the reference's ``concatenate``), and forms the gated
residual in the ``to_out`` epilogue.

Between a block's two residual adds the stream is carried in FP32 and rounded to bf16 once,
by the last epilogue; the reference rounds after each add. bf16 is the only activation dtype
(no FP16 route, so no ``clip(+-65504)``). The reference-KV path (``reference_kv``) is not
built: it raises.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..kernels import fused_ops
from ..ltx2 import dense_attention as _dense
from ..ltx2.attention import Linear, _cat_layers, qknorm_rope_projection
from ..ltx2.transformer import layer_norm_modulate
from .kv import attend

__all__ = [
    "DoubleAttention",
    "DoubleBlock",
    "FeedForward",
    "Linear",
    "Modulation",
    "QKNorm",
    "SingleAttention",
    "SingleBlock",
    "attend",
    "joint_attention",
    "normalized",
    "rotary_positions",
    "rotate",
    "swiglu",
]

HEADS = 32
HEAD_DIM = 128


def rotary_positions(ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """FP32 ``(B, T, 1, 128)`` cosine/sine tables of four independent position axes, each
    frequency repeated for its adjacent channel pair (``transformer.py:17-22``):
    ``frequency[i] = 2000 ** (-2i / 32)``, ``i < 16``; angles ``ids[..., a] * frequency``."""
    if ids.dim() != 3 or ids.shape[-1] != 4:
        raise ValueError("FLUX.2 ids must have shape (batch, tokens, 4)")
    frequency = torch.tensor(2000.0, dtype=torch.float32, device=ids.device) ** (
        -torch.arange(0, 32, 2, dtype=torch.float32, device=ids.device) / 32)
    angles = (ids.float()[..., None] * frequency).reshape(*ids.shape[:-1], 64)
    angles = torch.repeat_interleave(angles, 2, dim=-1)
    return torch.cos(angles)[:, :, None].contiguous(), torch.sin(angles)[:, :, None].contiguous()


def _tables(positions: tuple[torch.Tensor, torch.Tensor], batch: int, tokens: int, head_dim: int):
    """Validated ``(cos, sin)`` of shape ``(1 or B, T, 1, Dh)`` with contiguous rows."""
    cos, sin = positions
    if (cos.dtype != torch.float32 or sin.shape != cos.shape or cos.dim() != 4 or cos.shape[0] not in (1, batch)
            or cos.shape[1] != tokens or cos.shape[2] != 1 or cos.shape[3] != head_dim):
        raise ValueError(f"rotary tables must be fp32 (1 or {batch}, {tokens}, 1, {head_dim})")
    if not (cos.is_contiguous() and sin.is_contiguous()):
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def rotate(value: torch.Tensor, positions: tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
    """Adjacent-pair RoPE ``(x0, x1) -> (x0 c - x1 s, x1 c + x0 s)`` in FP32, one rounding
    (``transformer.py:25-29``); ``value`` is ``(B, T, H, Dh)`` bf16, the tables ``(1|B, T, 1, Dh)``.
    Bit-exact with the reference's op order: each product rounded, then the sum."""
    if value.dtype != torch.bfloat16 or value.dim() != 4:
        raise ValueError("rotate takes bfloat16 (batch, tokens, heads, head_dim) values on MI355X")
    batch, tokens, heads, head_dim = (int(s) for s in value.shape)
    if head_dim % 2:
        raise ValueError("rotate needs an even head width")
    cos, sin = _tables(positions, batch, tokens, head_dim)
    src = value if value.is_contiguous() else value.contiguous()
    out = torch.empty_like(src)
    if out.numel():
        _lib.launch_rope_pair(src.view(batch * tokens, heads * head_dim), out.view(batch * tokens, heads * head_dim),
                              cos, sin, heads=heads, head_dim=head_dim, table_ld=head_dim, table_hs=0,
                              tokens=tokens, table_batched=cos.shape[0] > 1)
    return out


def joint_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    positions: tuple[torch.Tensor, torch.Tensor], *, text_tokens: int = 0,
                    reference_kv=None, layer: int = 0) -> torch.Tensor:
    """Rotate Q and K, attend, flatten heads (``transformer.py:35-53``)."""
    del text_tokens, layer
    if reference_kv is not None:
        raise ValueError("reference-KV attention is not built for MI355X")
    result = attend(rotate(query, positions), rotate(key, positions), value)
    return result.reshape(*query.shape[:2], -1)


def normalized(value: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``layer_norm(x, eps=1e-6) * (1 + scale) + shift`` in one FP32 pass
    (``transformer.py:56-57``)."""
    return layer_norm_modulate(value, shift, scale, 1e-6)


def swiglu(value: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * content`` of the two halves of the last axis (``transformer.py:63-65``)."""
    return fused_ops.swiglu(value)


class QKNorm:
    """Per-head weighted RMSNorm, FP32 reduction and scale, eps 1e-6 (``transformer.py:68-75``)."""

    def __init__(self) -> None:
        self.weight: torch.Tensor | None = None

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        return fused_ops.rms_norm(value, self.weight, 1e-6)


class FeedForward:
    """``linear_out(swiglu(linear_in(x)))`` (``transformer.py:78-85``)."""

    def __init__(self) -> None:
        self.linear_in = None
        self.linear_out = None

    def __call__(self, value: torch.Tensor, *, residual: torch.Tensor | None = None,
                 gate: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """With ``residual``/``gate`` the block's ``residual + gate * ff(x)`` is formed in the
        ``linear_out`` epilogue, written as ``out_dtype`` (default the input dtype)."""
        return self.linear_out(fused_ops.swiglu(self.linear_in(value)), residual=residual, gate=gate,
                               out_dtype=out_dtype)


def _norm_rope_into(raw: torch.Tensor, out: torch.Tensor, norm: QKNorm, cos: torch.Tensor, sin: torch.Tensor,
                    row0: int, heads: int) -> None:
    """``out = pair_rope(per_head_rms_norm(raw))`` for ``raw``/``out`` of shape ``(B, Ts, D)``
    (strided row views) whose tokens start at joint position ``row0``; one launch per batch
    entry (a batch of row views at a joint offset is not one evenly strided row set)."""
    batch, tokens, width = raw.shape
    head_dim = width // heads
    if norm.weight is None or norm.weight.shape != (head_dim,):
        raise ValueError(f"QKNorm weight must have shape ({head_dim},)")
    for b in range(batch):
        tb = b if cos.shape[0] > 1 else 0
        ct, st = cos[tb, row0:row0 + tokens, 0], sin[tb, row0:row0 + tokens, 0]
        _lib.launch_rmsnorm_rope(raw[b], out[b], norm.weight, 1e-6, 0.0, norm_width=head_dim,
                                 rope_kind=_lib.KX_ROPE_PAIR, cos=ct, sin=st, table_ld=head_dim, table_hs=0,
                                 tokens=tokens, head_dim=head_dim)


def _linear_rows_into(layer, value: torch.Tensor, out: torch.Tensor) -> None:
    """``out[b] = layer(value[b])`` for every batch entry; ``out`` is a row view of a larger
    buffer (a batch of such views is not one evenly strided row set when ``B > 1``)."""
    if value.shape[0] == 1:
        layer(value, out=out)
        return
    for b in range(value.shape[0]):
        layer(value[b], out=out[b])


class DoubleAttention:
    """Joint text+image attention with separate per-stream projections and QK norms
    (``transformer.py:88-133``)."""

    def __init__(self, *, heads: int = HEADS, head_dim: int = HEAD_DIM) -> None:
        self.heads = heads
        self.head_dim = head_dim
        self.to_q = self.to_k = self.to_v = None
        self.add_q_proj = self.add_k_proj = self.add_v_proj = None
        self.to_out = [None]
        self.to_add_out = None
        self.norm_q, self.norm_k = QKNorm(), QKNorm()
        self.norm_added_q, self.norm_added_k = QKNorm(), QKNorm()
        self._qkv = self._added_qkv = None

    def fuse_projections(self) -> None:
        """One ``(3D, D)`` weight per stream for Q/K/V; the per-projection layers become views
        into it."""
        self._qkv = _cat_layers([self.to_q, self.to_k, self.to_v])
        self._added_qkv = _cat_layers([self.add_q_proj, self.add_k_proj, self.add_v_proj])

    def _project(self, fused, layers, value: torch.Tensor, out: torch.Tensor) -> None:
        width = self.heads * self.head_dim
        if fused is not None:
            _linear_rows_into(fused, value, out)
            return
        for i, layer in enumerate(layers):
            _linear_rows_into(layer, value, out[..., i * width:(i + 1) * width])

    def attend(self, image: torch.Tensor, text: torch.Tensor,
               positions: tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
        """The joint attention output ``(B, Tt + Ti, H * Dh)``, text rows first."""
        if image.dim() != 3 or text.dim() != 3 or image.shape[0] != text.shape[0]:
            raise ValueError("DoubleAttention takes (batch, tokens, width) image and text")
        width = self.heads * self.head_dim
        batch, t_text, t_image = image.shape[0], text.shape[1], image.shape[1]
        tokens = t_text + t_image
        cos, sin = _tables(positions, batch, tokens, self.head_dim)
        qkv = torch.empty((batch, tokens, 3 * width), dtype=torch.bfloat16, device=image.device)
        self._stream_qkv(self._added_qkv, (self.add_q_proj, self.add_k_proj, self.add_v_proj), text,
                         qkv[:, :t_text], self.norm_added_q, self.norm_added_k, cos, sin, 0)
        self._stream_qkv(self._qkv, (self.to_q, self.to_k, self.to_v), image, qkv[:, t_text:], self.norm_q,
                         self.norm_k, cos, sin, t_text)
        return _dense.batched_attention(qkv[..., :width], qkv[..., width:2 * width], qkv[..., 2 * width:],
                                        heads=self.heads, scale=self.head_dim ** -0.5)

    def _stream_qkv(self, fused, layers, value: torch.Tensor, rows: torch.Tensor, norm_q: QKNorm, norm_k: QKNorm,
                    cos: torch.Tensor, sin: torch.Tensor, row0: int) -> None:
        """``rows`` ``(B, Ts, 3D)`` = one stream's Q/K/V projection with Q and K normalized per
        head and rotated at joint positions ``row0 + t``. With the fused weight the norm and rotation
        run in the projection's epilogue, one launch per batch entry; otherwise the projection, then
        the norm + RoPE pass (into scratch rows, copied back over the raw Q/K columns)."""
        width = self.heads * self.head_dim
        count = rows.shape[1]
        if count == 0:
            return
        for b in range(rows.shape[0]):
            tb = b if cos.shape[0] > 1 else 0
            if (fused is not None and norm_q.weight is not None and norm_k.weight is not None
                    and qknorm_rope_projection(fused, value[b], rows[b], q_width=width, k_width=width,
                                               norm_q=norm_q.weight, norm_k=norm_k.weight, eps=1e-6,
                                               weight_offset=0.0, cos=cos[tb, row0:row0 + count, 0],
                                               sin=sin[tb, row0:row0 + count, 0])):
                continue
            entry = rows[b:b + 1]
            self._project(fused, layers, value[b:b + 1], entry)
            normed = torch.empty((1, count, 2 * width), dtype=torch.bfloat16, device=rows.device)
            _norm_rope_into(entry[..., :width], normed[..., :width], norm_q, cos[tb:tb + 1], sin[tb:tb + 1], row0,
                            self.heads)
            _norm_rope_into(entry[..., width:2 * width], normed[..., width:], norm_k, cos[tb:tb + 1],
                            sin[tb:tb + 1], row0, self.heads)
            entry[..., :2 * width].copy_(normed)

    def __call__(self, image: torch.Tensor, text: torch.Tensor, positions: tuple[torch.Tensor, torch.Tensor],
                 reference_kv=None, layer: int = 0, *, image_residual: torch.Tensor | None = None,
                 image_gate: torch.Tensor | None = None, text_residual: torch.Tensor | None = None,
                 text_gate: torch.Tensor | None = None, out_dtype: torch.dtype | None = None):
        """``(to_out(image rows), to_add_out(text rows))``; with the residual/gate pairs the
        block's gated residuals are formed in those GEMMs' epilogues."""
        del layer
        if reference_kv is not None:
            raise ValueError("reference-KV attention is not built for MI355X")
        result = self.attend(image, text, positions)
        t_text = text.shape[1]
        image_out = self.to_out[0](result[:, t_text:], residual=image_residual, gate=image_gate,
                                   out_dtype=out_dtype)
        text_out = self.to_add_out(result[:, :t_text], residual=text_residual, gate=text_gate, out_dtype=out_dtype)
        return image_out, text_out


def _split_mod(modulation: torch.Tensor, count: int) -> tuple[torch.Tensor, ...]:
    """``(B, count * D)`` or ``(B, 1|T, count * D)`` modulation -> ``count`` FP32 views
    ``(B, 1|T, D)`` (``mx.split(..., count, axis=-1)``)."""
    mod = modulation[:, None] if modulation.dim() == 2 else modulation
    mod = mod.float()
    if mod.stride(-1) != 1 or mod.data_ptr() % 16:
        mod = mod.contiguous()
    return tuple(torch.chunk(mod, count, dim=-1))


class DoubleBlock:
    """Double-stream block (``transformer.py:136-167``): gated joint attention, then a gated
    feed-forward per stream. ``ff``/``ff_context`` hold FLUX ``FeedForward`` layers (or any
    feed-forward taking ``residual``/``gate``/``out_dtype``, such as LTX's GELU MLP)."""

    def __init__(self, *, heads: int = HEADS, head_dim: int = HEAD_DIM) -> None:
        self.attn = DoubleAttention(heads=heads, head_dim=head_dim)
        self.ff, self.ff_context = FeedForward(), FeedForward()

    def fuse_projections(self) -> None:
        self.attn.fuse_projections()

    def __call__(self, image: torch.Tensor, text: torch.Tensor, image_mod: torch.Tensor, text_mod: torch.Tensor,
                 positions: tuple[torch.Tensor, torch.Tensor], reference_kv=None, layer: int = 0, *,
                 out_dtype: torch.dtype | None = None):
        """``(image, text)`` after the block, in ``out_dtype`` (default: the input dtype). The
        streams may be bfloat16 (the reference's hidden dtype) or an FP32 residual stream carried
        across blocks, which skips the rounding of the hidden state between blocks."""
        if image.dtype != text.dtype or image.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("DoubleBlock takes bfloat16 (or fp32 residual stream) image and text on MI355X")
        out_dtype = image.dtype if out_dtype is None else out_dtype
        shift, scale, gate, ff_shift, ff_scale, ff_gate = _split_mod(image_mod, 6)
        ts, tc, tg, fs, fc, fg = _split_mod(text_mod, 6)
        # image1/text1: the residual streams in FP32 between the two adds
        image1, text1 = self.attn(
            normalized(image, shift, scale), normalized(text, ts, tc), positions, reference_kv, layer,
            image_residual=image, image_gate=gate, text_residual=text, text_gate=tg, out_dtype=torch.float32,
        )
        image2 = self.ff(normalized(image1, ff_shift, ff_scale), residual=image1, gate=ff_gate, out_dtype=out_dtype)
        text2 = self.ff_context(normalized(text1, fs, fc), residual=text1, gate=fg, out_dtype=out_dtype)
        return image2, text2


class SingleAttention:
    """Single-stream attention and MLP sharing one fused projection (``transformer.py:170-198``):
    ``to_qkv_mlp_proj`` splits into [D, D, D, 2F]; ``to_out(concat[attention, swiglu(mlp)])``."""

    def __init__(self, *, heads: int = HEADS, head_dim: int = HEAD_DIM) -> None:
        self.heads = heads
        self.head_dim = head_dim
        self.to_qkv_mlp_proj = None
        self.to_out = None
        self.norm_q, self.norm_k = QKNorm(), QKNorm()

    def __call__(self, value: torch.Tensor, positions: tuple[torch.Tensor, torch.Tensor], reference_kv=None,
                 layer: int = 0, text_tokens: int = 0, *, residual: torch.Tensor | None = None,
                 gate: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        del layer, text_tokens
        if reference_kv is not None:
            raise ValueError("reference-KV attention is not built for MI355X")
        if value.dim() != 3:
            raise ValueError("SingleAttention takes (batch, tokens, width) values")
        width = self.heads * self.head_dim
        batch, tokens = value.shape[0], value.shape[1]
        total = int(self.to_qkv_mlp_proj.out_features)
        mlp_width = total - 3 * width
        if mlp_width <= 0 or mlp_width % 2:
            raise ValueError(f"to_qkv_mlp_proj width {total} does not split into [{width} x 3, 2F]")
        cos, sin = _tables(positions, batch, tokens, self.head_dim)
        fused = torch.empty((batch, tokens, total), dtype=torch.bfloat16, device=value.device)
        if (self.norm_q.weight is not None and self.norm_k.weight is not None and value.is_contiguous()
                and qknorm_rope_projection(self.to_qkv_mlp_proj, value.view(batch * tokens, -1),
                                           fused.view(batch * tokens, total), q_width=width, k_width=width,
                                           norm_q=self.norm_q.weight, norm_k=self.norm_k.weight, eps=1e-6,
                                           weight_offset=0.0, cos=cos[:, :, 0], sin=sin[:, :, 0])):
            q, k = fused[..., :width], fused[..., width:2 * width]
        else:  # the projection, then the norm + RoPE pass
            self.to_qkv_mlp_proj(value, out=fused)
            q = torch.empty((batch, tokens, width), dtype=torch.bfloat16, device=value.device)
            k = torch.empty_like(q)
            _norm_rope_into(fused[..., :width], q, self.norm_q, cos, sin, 0, self.heads)
            _norm_rope_into(fused[..., width:2 * width], k, self.norm_k, cos, sin, 0, self.heads)
        joined = torch.empty((batch, tokens, width + mlp_width // 2), dtype=torch.bfloat16, device=value.device)
        _dense.batched_attention(q, k, fused[..., 2 * width:3 * width], heads=self.heads,
                                     scale=self.head_dim ** -0.5, out=joined[..., :width])
        _lib.launch_swiglu(fused[..., 3 * width:], joined[..., width:])
        return self.to_out(joined, residual=residual, gate=gate, out_dtype=out_dtype)


class SingleBlock:
    """``x + gate * attn(normalized(x))`` (``transformer.py:201-220``), the gated residual
    formed in the ``to_out`` epilogue."""

    def __init__(self, *, heads: int = HEADS, head_dim: int = HEAD_DIM) -> None:
        self.attn = SingleAttention(heads=heads, head_dim=head_dim)

    def __call__(self, value: torch.Tensor, modulation: torch.Tensor, positions: tuple[torch.Tensor, torch.Tensor],
                 reference_kv=None, layer: int = 0, text_tokens: int = 0, *,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """The block's output in ``out_dtype`` (default: the input dtype); ``value`` may be
        bfloat16 or an FP32 residual stream carried across blocks."""
        if value.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("SingleBlock takes bfloat16 (or fp32 residual stream) values on MI355X")
        shift, scale, gate = _split_mod(modulation, 3)
        return self.attn(normalized(value, shift, scale), positions, reference_kv, layer, text_tokens,
                         residual=value, gate=gate, out_dtype=value.dtype if out_dtype is None else out_dtype)


class Modulation:
    """``linear(silu(x))`` (``transformer.py:223-229``)."""

    def __init__(self) -> None:
        self.linear = None

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        return self.linear(fused_ops.silu(value))
