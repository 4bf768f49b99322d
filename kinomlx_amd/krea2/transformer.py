"""Krea 2 transformer block surface on MI355X.

Mirror of ``kinomlx/models/krea2/transformer/model.py``: ``Krea2RMSNorm``,
``Krea2RotaryEmbedding``, ``apply_rotary_embedding``, ``Krea2Attention``, ``Krea2SwiGLU``,
``split_six_way_modulation`` and ``Krea2TransformerBlock``, same names and math on torch tensors.
Weights are assigned after construction (``Linear``/``QuantizedLinear`` projections, FP32 or bf16
norm weights), as the reference's loader does.

MI355X schedule of one block:

  zero-centred RMSNorm + (1 + scale) / shift in one FP32 pass (the norm weight is folded into
  the modulation scale: ``n (w + 1)(1 + s) + shift = n (1 + s') + shift``)
  -> one GEMM for Q/K/V (``fuse_projections``) and the gate GEMM with ``sigmoid`` in its epilogue
  -> per-head zero-centred RMSNorm + adjacent-pair RoPE in one pass per Q and K, token-major
     (the reference's head-major transposes are never materialised)
  -> grouped-query flash attention (K/V heads are read in place, not repeated per query head)
  -> ``attended * sigmoid(gate)`` -> ``to_out`` with ``x + pregate * .`` in its epilogue
  -> the same modulated norm -> one GEMM for gate/up -> SwiGLU -> ``down`` with
     ``x + postgate * .`` in its epilogue.

The residual stream is carried in FP32 between the two adds and rounded once. Attention masks
and the reference-attention capture path are not built and raise ``ValueError``; the text-fusion
blocks are outside this path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib
from ..kernels import fused_ops
from ..ltx2 import dense_attention as _dense
from ..ltx2.attention import Linear, _cat_layers, qknorm_rope_projection
from ..ltx2.transformer import adaln

__all__ = [
    "Krea2Attention",
    "Krea2BlockConfig",
    "Krea2RMSNorm",
    "Krea2RotaryEmbedding",
    "Krea2SwiGLU",
    "Krea2TransformerBlock",
    "Linear",
    "apply_rotary_embedding",
    "split_six_way_modulation",
]


class Krea2RMSNorm:
    """Zero-centred RMSNorm ``x * rsqrt(mean(x^2) + eps) * (weight + 1)``, FP32 reduction and
    affine math, one rounding (``model.py:29-46``)."""

    def __init__(self, dims: int, eps: float) -> None:
        self.dims = dims
        self.eps = eps
        self.weight: torch.Tensor | None = None

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        if value.shape[-1] != self.dims:
            raise ValueError(f"Krea RMSNorm expects width {self.dims}, got {value.shape[-1]}")
        return fused_ops.rms_norm(value, self.weight, self.eps, weight_offset=1.0)


class Krea2RotaryEmbedding:
    """Per-axis real RoPE tables with adjacent-pair frequency repetition (``model.py:49-66``):
    ``1 / theta ** (arange(0, d, 2) / d)`` per axis, axes concatenated in declared order; FP32
    ``(B, T, sum(axes_dims))`` cosine and sine."""

    def __init__(self, *, theta: float, axes_dims: tuple[int, ...]) -> None:
        self.theta = theta
        self.axes_dims = tuple(axes_dims)

    def __call__(self, position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        if position_ids.dim() != 3 or position_ids.shape[-1] != len(self.axes_dims):
            raise ValueError("Krea position_ids must have shape [batch, sequence, position_axes]")
        positions = position_ids.float()
        parts = []
        for axis, dims in enumerate(self.axes_dims):
            exponent = torch.arange(0, dims, 2, dtype=torch.float32, device=positions.device) / dims
            frequencies = 1.0 / (torch.tensor(self.theta, dtype=torch.float32, device=positions.device) ** exponent)
            angles = positions[..., axis, None] * frequencies
            parts.append(torch.repeat_interleave(angles, 2, dim=-1))
        combined = torch.cat(parts, dim=-1)
        return torch.cos(combined).contiguous(), torch.sin(combined).contiguous()


def _check_tables(cos: torch.Tensor, sin: torch.Tensor, batch: int, tokens: int, head_dim: int):
    if (cos.dtype != torch.float32 or sin.shape != cos.shape or cos.dim() != 3 or cos.shape[0] not in (1, batch)
            or cos.shape[1] != tokens or cos.shape[2] != head_dim):
        raise ValueError(f"Krea rotary tables must be fp32 (1 or {batch}, {tokens}, {head_dim})")
    return cos.contiguous(), sin.contiguous()


def apply_rotary_embedding(queries: torch.Tensor, keys: torch.Tensor, cos: torch.Tensor,
                           sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Adjacent-pair real RoPE on head-major ``(B, H, T, Dh)`` queries and keys with
    ``(B, T, Dh)`` tables, FP32 products each rounded then summed, one cast back
    (``model.py:69-92``); bit-exact with that op order."""
    if queries.shape[-1] != cos.shape[-1] or keys.shape[-1] != cos.shape[-1]:
        raise ValueError("Krea rotary width must match query and key head dimensions")

    def apply(value: torch.Tensor) -> torch.Tensor:
        if value.dtype != torch.bfloat16 or value.dim() != 4:
            raise ValueError("Krea rotary embedding takes bfloat16 (batch, heads, tokens, head_dim) on MI355X")
        batch, heads, tokens, head_dim = (int(s) for s in value.shape)
        c, s = _check_tables(cos, sin, batch, tokens, head_dim)
        src = value.contiguous()
        out = torch.empty_like(src)
        for b in range(batch if out.numel() else 0):
            tb = b if c.shape[0] > 1 else 0
            _lib.launch_rope_pair(src[b].view(heads * tokens, head_dim), out[b].view(heads * tokens, head_dim),
                                  c[tb], s[tb], heads=1, head_dim=head_dim, table_ld=head_dim, table_hs=0,
                                  tokens=tokens, table_batched=False)
        return out

    return apply(queries), apply(keys)


def _fused_norm_rope_ok(width: int, head_dim: int, *tensors: torch.Tensor) -> bool:
    """The one-pass norm + pair RoPE kernel's shape and alignment contract."""
    return (width % 512 == 0 and width // 512 in (1, 2, 4, 8) and 512 % head_dim == 0 and head_dim % 8 == 0
            and head_dim // 8 in (8, 16, 32)
            and all(t.data_ptr() % 16 == 0 and t.stride(-2) % 8 == 0 for t in tensors))


def _norm_rope_rows(raw: torch.Tensor, norm: Krea2RMSNorm, tables, heads: int) -> torch.Tensor:
    """Token-major ``(B, T, heads * Dh)`` rows -> per-head zero-centred RMSNorm, then pair RoPE
    with ``(1|B, T, Dh)`` tables; one pass when the kernel's contract holds, else the norm pass
    and the standalone rotation pass."""
    batch, tokens, width = raw.shape
    head_dim = width // heads
    out = torch.empty((batch, tokens, width), dtype=torch.bfloat16, device=raw.device)
    if out.numel() == 0:
        return out
    if norm.weight is None or norm.weight.shape != (head_dim,):
        raise ValueError(f"Krea RMSNorm weight must have shape ({head_dim},)")
    cos = sin = None
    if tables is not None:
        cos, sin = _check_tables(*tables, batch, tokens, head_dim)
    for b in range(batch):
        x, y = raw[b], out[b]
        if cos is None:
            _lib.launch_rmsnorm_rope(x, y, norm.weight, norm.eps, 1.0, norm_width=head_dim)
            continue
        tb = b if cos.shape[0] > 1 else 0
        if _fused_norm_rope_ok(width, head_dim, x, y):
            _lib.launch_rmsnorm_rope(x, y, norm.weight, norm.eps, 1.0, norm_width=head_dim,
                                     rope_kind=_lib.KX_ROPE_PAIR, cos=cos[tb], sin=sin[tb], table_ld=head_dim,
                                     table_hs=0, tokens=tokens, head_dim=head_dim)
        else:
            _lib.launch_rmsnorm_rope(x, y, norm.weight, norm.eps, 1.0, norm_width=head_dim)
            _lib.launch_rope_pair(y, y, cos[tb], sin[tb], heads=heads, head_dim=head_dim, table_ld=head_dim,
                                  table_hs=0, tokens=tokens, table_batched=False)
    return out


class Krea2Attention:
    """Grouped-query attention with zero-centred Q/K norms and a sigmoid output gate
    (``model.py:95-196``). ``to_q``/``to_k``/``to_v``/``to_gate``/``to_out`` hold the projections."""

    def __init__(self, *, hidden_size: int, num_heads: int, num_kv_heads: int, eps: float) -> None:
        if hidden_size % num_heads:
            raise ValueError("Krea attention hidden size must be divisible by query heads")
        if num_heads % num_kv_heads:
            raise ValueError("Krea attention query heads must be divisible by KV heads")
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = hidden_size // num_heads
        self.scale = self.head_dim ** -0.5
        self.to_q = self.to_k = self.to_v = self.to_gate = self.to_out = None
        self.norm_q = Krea2RMSNorm(self.head_dim, eps)
        self.norm_k = Krea2RMSNorm(self.head_dim, eps)
        self._qkv = None

    def fuse_projections(self) -> None:
        """One weight for Q/K/V; the per-projection layers become views into it."""
        self._qkv = _cat_layers([self.to_q, self.to_k, self.to_v])

    def __call__(self, hidden_states: torch.Tensor, *, attention_mask: torch.Tensor | None = None,
                 rotary: tuple[torch.Tensor, torch.Tensor] | None = None, reference_attention=None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """``to_out(attention * sigmoid(to_gate(x)))``; with ``residual``/``gate`` the block's
        ``residual + gate * .`` is formed in the ``to_out`` epilogue, written as ``out_dtype``."""
        if hidden_states.dim() != 3 or hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"Krea attention expects [batch, sequence, {self.hidden_size}] hidden states")
        batch, length = int(hidden_states.shape[0]), int(hidden_states.shape[1])
        key_mask = None
        if attention_mask is not None:
            # a boolean (batch, length) key mask; masked queries are zeroed (model.py:164-196)
            if attention_mask.dtype != torch.bool:
                raise ValueError("Krea attention mask must use a boolean dtype")
            if tuple(attention_mask.shape) != (batch, length):
                raise ValueError("Krea attention mask must match batch and sequence dimensions")
            key_mask = attention_mask[:, None, None, :]
        if reference_attention is not None:
            raise ValueError("reference attention capture is not built for MI355X")
        q_width = self.num_heads * self.head_dim
        kv_width = self.num_kv_heads * self.head_dim
        q = k = None
        if self._qkv is not None:
            qkv = torch.empty((batch, length, q_width + 2 * kv_width), dtype=torch.bfloat16,
                              device=hidden_states.device)
            if (rotary is not None and self.norm_q.weight is not None and self.norm_k.weight is not None
                    and self.norm_q.eps == self.norm_k.eps and hidden_states.is_contiguous()):
                cos, sin = _check_tables(*rotary, batch, length, self.head_dim)
                if qknorm_rope_projection(self._qkv, hidden_states.view(batch * length, -1),
                                          qkv.view(batch * length, -1), q_width=q_width, k_width=kv_width,
                                          norm_q=self.norm_q.weight, norm_k=self.norm_k.weight, eps=self.norm_q.eps,
                                          weight_offset=1.0, cos=cos, sin=sin):
                    # zero-centred norms and the rotation ran in the projection's epilogue
                    q, k = qkv[..., :q_width], qkv[..., q_width:q_width + kv_width]
            if q is None:
                self._qkv(hidden_states, out=qkv)
            q_raw, k_raw = qkv[..., :q_width], qkv[..., q_width:q_width + kv_width]
            v = qkv[..., q_width + kv_width:]
        else:
            q_raw, k_raw, v = self.to_q(hidden_states), self.to_k(hidden_states), self.to_v(hidden_states)
        sigmoid_gate = self.to_gate(hidden_states, activation="sigmoid", out_dtype=torch.float32)
        if q is None:
            q = _norm_rope_rows(q_raw, self.norm_q, rotary, self.num_heads)
            k = _norm_rope_rows(k_raw, self.norm_k, rotary, self.num_kv_heads)
        attended = _dense.batched_attention(q, k, v, heads=self.num_heads, kv_heads=self.num_kv_heads,
                                            scale=self.scale, mask=key_mask)
        if attention_mask is not None:
            # the query selection rides on the gate: a zero gate row zeroes the attended row
            sigmoid_gate = sigmoid_gate.masked_fill(~attention_mask[..., None], 0.0)
        gated = torch.empty_like(attended)
        _lib.launch_gated_residual(None, attended.view(-1, q_width), gated.view(-1, q_width),
                                   sigmoid_gate.view(-1, q_width))
        return self.to_out(gated, residual=residual, gate=gate, out_dtype=out_dtype)


class Krea2SwiGLU:
    """``down(silu(gate(x)) * up(x))`` with FP32-opmath SiLU (``model.py:199-214``)."""

    def __init__(self, hidden_size: int, *, pretranspose_down: bool = False) -> None:
        del pretranspose_down  # weights stay (out, in) on MI355X
        self.hidden_size = hidden_size
        self.gate = self.up = self.down = None
        self._gate_up = None

    def fuse_projections(self) -> None:
        """One weight whose output rows are [gate; up]: one GEMM feeds the SwiGLU pass."""
        self._gate_up = _cat_layers([self.gate, self.up])

    def __call__(self, hidden_states: torch.Tensor, *, residual: torch.Tensor | None = None,
                 residual_gate: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"Krea SwiGLU expects width {self.hidden_size}, got {hidden_states.shape[-1]}")
        if self._gate_up is not None:
            both = self._gate_up(hidden_states)
        else:  # the two products side by side in one buffer, as the fused weight writes them
            inner = self.gate.out_features
            both = torch.empty((*hidden_states.shape[:-1], 2 * inner), dtype=torch.bfloat16,
                               device=hidden_states.device)
            self.gate(hidden_states, out=both[..., :inner])
            self.up(hidden_states, out=both[..., inner:])
        hidden = fused_ops.swiglu(both)
        return self.down(hidden, residual=residual, gate=residual_gate, out_dtype=out_dtype)


def split_six_way_modulation(projected: torch.Tensor, scale_shift_table: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """Add one block's ``(6, hidden)`` table and return the official chunk order
    (``model.py:288-307``): prescale, preshift, pregate, postscale, postshift, postgate."""
    if scale_shift_table.dim() != 2 or scale_shift_table.shape[0] != 6:
        raise ValueError("Krea block modulation table must have shape [6, hidden]")
    hidden_size = scale_shift_table.shape[1]
    if projected.shape[-1] != 6 * hidden_size:
        raise ValueError("Krea projected modulation width must be six times hidden size")
    modulation = projected.reshape(*projected.shape[:-1], 6, hidden_size) + scale_shift_table
    return tuple(modulation[..., i, :] for i in range(6))


@dataclass(frozen=True)
class Krea2BlockConfig:
    """The fields of ``Krea2TransformerConfig`` one block reads (``metadata.py:87-110``)."""

    attention_head_dim: int
    num_attention_heads: int
    num_key_value_heads: int
    norm_eps: float = 1e-6

    @property
    def hidden_dim(self) -> int:
        return self.attention_head_dim * self.num_attention_heads


class Krea2TransformerBlock:
    """One time-modulated single-stream block (``model.py:310-348``)."""

    def __init__(self, config, *, pretranspose_down: bool = False) -> None:
        hidden_size = config.hidden_dim
        self.scale_shift_table: torch.Tensor | None = None
        self.norm1 = Krea2RMSNorm(hidden_size, config.norm_eps)
        self.norm2 = Krea2RMSNorm(hidden_size, config.norm_eps)
        self.attn = Krea2Attention(hidden_size=hidden_size, num_heads=config.num_attention_heads,
                                   num_kv_heads=config.num_key_value_heads, eps=config.norm_eps)
        self.ff = Krea2SwiGLU(hidden_size, pretranspose_down=pretranspose_down)

    def fuse_projections(self) -> None:
        self.attn.fuse_projections()
        self.ff.fuse_projections()

    def _modulated(self, value: torch.Tensor, norm: Krea2RMSNorm, scale: torch.Tensor,
                   shift: torch.Tensor) -> torch.Tensor:
        """``(1 + scale) * norm(x) + shift`` in one FP32 pass: the zero-centred weight is folded
        into the scale, ``(1 + scale)(1 + w) = 1 + scale'``."""
        if norm.weight is None:
            raise ValueError("Krea RMSNorm weight is not loaded")
        scale_eff = (1.0 + scale.float()) * (1.0 + norm.weight.float()) - 1.0
        return adaln(value, scale_eff, shift.float().expand_as(scale_eff), norm.eps)

    def __call__(self, hidden_states: torch.Tensor, *, time_modulation: torch.Tensor,
                 rotary: tuple[torch.Tensor, torch.Tensor], attention_mask: torch.Tensor | None,
                 reference_attention=None) -> torch.Tensor:
        if hidden_states.dtype != torch.bfloat16:
            raise ValueError("Krea2TransformerBlock takes bfloat16 hidden states on MI355X")
        prescale, preshift, pregate, postscale, postshift, postgate = split_six_way_modulation(
            time_modulation, self.scale_shift_table)
        attention_input = self._modulated(hidden_states, self.norm1, prescale, preshift)
        h1 = self.attn(attention_input, attention_mask=attention_mask, rotary=rotary,
                       reference_attention=reference_attention, residual=hidden_states, gate=pregate,
                       out_dtype=torch.float32)
        feed_forward_input = self._modulated(h1, self.norm2, postscale, postshift)
        return self.ff(feed_forward_input, residual=h1, residual_gate=postgate, out_dtype=hidden_states.dtype)
