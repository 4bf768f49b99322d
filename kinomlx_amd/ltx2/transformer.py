"""The LTX-2 DiT block on MI355X.

Mirror of ``kinomlx/models/ltx2/transformer/transformer.py``: the modulation helpers
(``adaln``, ``gated_residual``, ``modulate``, ``gate``; the reference's private ``_adaln`` ...
and their ``mx.compile``d forms, ``:16-45``), ``TransformerConfig``, ``TransformerArgs`` and
``BasicAVTransformerBlock`` with its video and audio streams (``:225-421``), text
cross-attention (``:201-223``) and audio <-> video cross-attention (``:310-371``).

Kernel schedule of one block (B=1, T video tokens, Tc text tokens):
  AdaLN(x) -> [QKV GEMM, gate GEMM (2*sigmoid)] -> Q/K norm+RoPE -> flash attention (gated)
  -> out GEMM (+ x + g0 * .) ; AdaLN(x), modulate(ctx) -> [Q GEMM, gate GEMM, KV GEMM] -> Q/K norm
  -> attention -> out GEMM (+ x + g8 * .) ; AdaLN(x) -> up GEMM (GELU) -> down GEMM (+ x + g5 * .)
Every residual add rides in a GEMM epilogue; every reduction and epilogue is FP32. Between the
block's three branches the residual stream is carried in FP32 (written by the out-projection
epilogues, read by the next AdaLN and epilogue) and rounded to the block's 16-bit type (bf16 or
fp16, the dtype of its weights) once, by the last epilogue; every other intermediate is of that
type. The reference rounds the stream after each branch
(``transformer.py:26-30`` casts to ``value.dtype``); carrying it costs 2 x T x D x 2 extra bytes
per branch and removes two of the block's output roundings. The audio stream follows the same
schedule at its own width, then the A/V cross-attention of each stream reads the other's
(AdaLN-modulated) value. Masks become an additive score bias inside the attention kernel;
sparse (Sol-Attn) attention is not built.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from .. import _lib
from ..streams import side_stream
from .attention import Attention, rms_norm
from .feed_forward import FeedForward
from .rope import LTXRopeType


def _mod32(value: torch.Tensor) -> torch.Tensor:
    v = value.float()
    return v if (v.stride(-1) == 1 and v.data_ptr() % 16 == 0) else v.contiguous()


def _mod_pair(shift: torch.Tensor, scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 ``shift`` and ``scale`` in one row layout (the kernels index both rows with one
    divisor and stride): when they broadcast differently, both are expanded to their common
    shape first."""
    shift32, scale32 = _mod32(shift), _mod32(scale)
    if shift32.shape != scale32.shape or shift32.stride() != scale32.stride():
        shape = torch.broadcast_shapes(shift32.shape, scale32.shape)
        shift32 = shift32.expand(shape).contiguous()
        scale32 = scale32.expand(shape).contiguous()
    return shift32, scale32


_HALF = (torch.bfloat16, torch.float16)



def _norm_out_dtype(value: torch.Tensor, out_dtype: torch.dtype | None, what: str) -> torch.dtype:
    if value.dtype not in (*_HALF, torch.float32):
        raise ValueError(f"{what} takes float16 or bfloat16 (or an fp32 residual stream) on MI355X, got {value.dtype}")
    dtype = out_dtype or (value.dtype if value.dtype in _HALF else torch.bfloat16)
    if dtype not in _HALF:
        raise ValueError(f"{what} writes float16 or bfloat16, not {dtype}")
    if value.dtype in _HALF and value.dtype != dtype:
        raise ValueError(f"{what}: a {value.dtype} input normalizes to {value.dtype}, not {dtype}")
    return dtype


def adaln(value: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float,
          out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``rms_norm(x) * (1 + scale) + shift`` in one FP32 pass (``transformer.py:16-23``).
    ``scale``/``shift`` broadcast as ``(D,)``, ``(B, 1, D)`` or ``(B, T, D)``. ``value`` is bf16
    or fp16, or an FP32 residual stream; the result is the 16-bit type the next GEMM reads:
    ``value``'s own (as the reference returns ``value.dtype``), or ``out_dtype`` for a stream
    (default bf16)."""
    out = torch.empty(value.shape, dtype=_norm_out_dtype(value, out_dtype, "adaln"), device=value.device)
    if value.numel():
        shift32, scale32 = _mod_pair(shift, scale)
        _lib.launch_adaln_norm(value, out, shift32, scale32, eps, _lib.KX_NORM_RMS)
    return out


def layer_norm_modulate(value: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                        eps: float = 1e-6, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``layer_norm(x) * (1 + scale) + shift`` in one FP32 pass (FLUX.2 ``normalized``,
    ``kinomlx/models/flux2/transformer.py:56-57``). ``value`` is bf16 or fp16, or an FP32
    residual stream; the result's type is chosen as ``adaln``'s."""
    out = torch.empty(value.shape, dtype=_norm_out_dtype(value, out_dtype, "layer_norm_modulate"),
                      device=value.device)
    if value.numel():
        shift32, scale32 = _mod_pair(shift, scale)
        _lib.launch_adaln_norm(value, out, shift32, scale32, eps, _lib.KX_NORM_LAYER)
    return out


def gated_residual(value: torch.Tensor, residual: torch.Tensor, gate_value: torch.Tensor) -> torch.Tensor:
    """``x + r * gate`` (``transformer.py:26-30``)."""
    out = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    if value.numel():
        _lib.launch_gated_residual(value, residual, out, _mod32(gate_value))
    return out


def modulate(value: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor) -> torch.Tensor:
    """``x * (1 + scale) + shift`` (``transformer.py:33-34``)."""
    out = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    if value.numel():
        shift32, scale32 = _mod_pair(shift, scale)
        _lib.launch_modulate(value, out, shift32, scale32)
    return out


def gate(value: torch.Tensor, gate_value: torch.Tensor) -> torch.Tensor:
    """``x * gate`` (``transformer.py:37-38``)."""
    out = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    if value.numel():
        _lib.launch_gated_residual(None, value, out, _mod32(gate_value))
    return out


def compute_dtype(attention: Attention) -> torch.dtype:
    """The 16-bit type an attention's projections multiply in: its output projection's weight
    dtype when that is float16 or bfloat16 (the transformer dtype), else bf16 (quantized layers
    dequantize to bf16)."""
    weight = getattr(attention.to_out, "weight", None)
    dtype = getattr(weight, "dtype", None)
    return dtype if dtype in _HALF else torch.bfloat16


# The reference's private names and their compiled forms map to the same fused kernels.
_adaln = _compiled_adaln = adaln
_gated_residual = _compiled_gated_residual = gated_residual
_modulate = _compiled_modulate = modulate
_gate = _compiled_gate = gate


@dataclass(frozen=True)
class TransformerConfig:
    """Shape and feature selection for one transformer stream (``transformer.py:52-63``)."""

    dim: int
    heads: int
    head_dim: int
    context_dim: int
    ff_bias: bool = True
    apply_gated_attention: bool = True
    compile_attention: bool = True
    dense_attention_kernel: bool = True


@dataclass(frozen=True)
class TransformerArgs:
    """Prepared inputs carried through every block (``transformer.py:66-82``)."""

    x: torch.Tensor
    context: torch.Tensor
    timesteps: torch.Tensor
    positional_embeddings: tuple[torch.Tensor, torch.Tensor]
    context_mask: torch.Tensor | None = None
    self_attention_mask: torch.Tensor | None = None
    embedded_timestep: torch.Tensor | None = None
    prompt_timestep: torch.Tensor | None = None
    cross_positional_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None
    cross_scale_shift_timestep: torch.Tensor | None = None
    cross_gate_timestep: torch.Tensor | None = None
    enabled: bool = True
    sparse_attention: object | None = None


class BasicAVTransformerBlock:
    """One LTX-2 block (``transformer.py:85-421``): the video stream, and with ``audio_config``
    the audio stream and the audio <-> video cross-attention. Weights are assigned after
    construction: ``attn1``/``attn2`` (``Attention``), ``ff`` (``FeedForward``),
    ``scale_shift_table`` ``(9, D)``, ``prompt_scale_shift_table`` ``(2, D)``; for audio the same
    with an ``audio_`` prefix, plus ``audio_to_video_attn``, ``video_to_audio_attn`` and the
    ``(5, D)`` tables ``scale_shift_table_a2v_ca_video`` / ``scale_shift_table_a2v_ca_audio``.

    Each stream's residual is carried in FP32 between its branches (attention, text
    cross-attention, A/V cross-attention, feed-forward) and rounded once at the end; the
    branches' gated residuals are formed in the output GEMMs' epilogues."""

    def __init__(self, idx: int, *, video_config: TransformerConfig, audio_config: TransformerConfig | None = None,
                 rope_type: LTXRopeType = LTXRopeType.SPLIT, norm_eps: float = 1e-6) -> None:
        self.idx = idx
        self.norm_eps = norm_eps
        self.video_config = video_config
        self.audio_config = audio_config
        # with both streams present, run the audio stream's launches on a second HIP stream beside
        # the video stream's (the same kernels on the same values; False keeps one stream)
        self.audio_side_stream = True
        v_backend = {"compile_attention": video_config.compile_attention,
                     "dense_kernel": video_config.dense_attention_kernel}
        self.attn1 = Attention(video_config.dim, heads=video_config.heads, dim_head=video_config.head_dim,
                               norm_eps=norm_eps, rope_type=rope_type,
                               apply_gated_attention=video_config.apply_gated_attention, **v_backend)
        self.attn2 = Attention(video_config.dim, context_dim=video_config.context_dim, heads=video_config.heads,
                               dim_head=video_config.head_dim, norm_eps=norm_eps, rope_type=rope_type,
                               apply_gated_attention=video_config.apply_gated_attention, **v_backend)
        self.ff = FeedForward(video_config.dim, bias=video_config.ff_bias)
        self.scale_shift_table: torch.Tensor | None = None
        self.prompt_scale_shift_table: torch.Tensor | None = None
        if audio_config is None:
            return
        a = audio_config
        a_backend = {"compile_attention": a.compile_attention, "dense_kernel": a.dense_attention_kernel}
        self.audio_attn1 = Attention(a.dim, heads=a.heads, dim_head=a.head_dim, norm_eps=norm_eps, rope_type=rope_type,
                                     apply_gated_attention=a.apply_gated_attention, **a_backend)
        self.audio_attn2 = Attention(a.dim, context_dim=a.context_dim, heads=a.heads, dim_head=a.head_dim,
                                     norm_eps=norm_eps, rope_type=rope_type,
                                     apply_gated_attention=a.apply_gated_attention, **a_backend)
        self.audio_ff = FeedForward(a.dim, bias=a.ff_bias)
        self.audio_scale_shift_table: torch.Tensor | None = None
        self.audio_prompt_scale_shift_table: torch.Tensor | None = None
        self.audio_to_video_attn = Attention(video_config.dim, context_dim=a.dim, heads=a.heads, dim_head=a.head_dim,
                                             norm_eps=norm_eps, rope_type=rope_type,
                                             apply_gated_attention=video_config.apply_gated_attention, **v_backend)
        self.video_to_audio_attn = Attention(a.dim, context_dim=video_config.dim, heads=a.heads, dim_head=a.head_dim,
                                             norm_eps=norm_eps, rope_type=rope_type,
                                             apply_gated_attention=a.apply_gated_attention, **a_backend)
        self.scale_shift_table_a2v_ca_audio: torch.Tensor | None = None
        self.scale_shift_table_a2v_ca_video: torch.Tensor | None = None

    def fuse_projections(self) -> None:
        """Fuse Q/K/V of the self-attentions and K/V of the text cross-attentions."""
        self.attn1.fuse_projections(self_attention=True)
        self.attn2.fuse_projections(self_attention=False)
        if self.audio_config is not None:
            self.audio_attn1.fuse_projections(self_attention=True)
            self.audio_attn2.fuse_projections(self_attention=False)
            self.audio_to_video_attn.fuse_projections(self_attention=False)
            self.video_to_audio_attn.fuse_projections(self_attention=False)

    @staticmethod
    def _ada_values(table: torch.Tensor, timestep: torch.Tensor, start: int, stop: int) -> tuple[torch.Tensor, ...]:
        """``table[start:stop] + timestep[:, :, start:stop]`` split per row (``:179-186``)."""
        values = _lib.table_add(table[start:stop], timestep[:, :, start:stop, :])
        return tuple(values[:, :, i, :] for i in range(stop - start))

    @staticmethod
    def _av_ada_values(table: torch.Tensor, scale_shift: torch.Tensor, gate_timestep: torch.Tensor):
        """``(scale_a2v, shift_a2v, scale_v2a, shift_v2a, gate)`` from a ``(5, D)`` table
        (``transformer.py:188-199``)."""
        ss = _lib.table_add(table[:4], scale_shift)
        g = _lib.table_add(table[4:5], gate_timestep)
        return (*(ss[:, :, i, :] for i in range(4)), g[:, :, 0, :])

    def _text_cross_attention(self, value: torch.Tensor, args: TransformerArgs, ada: torch.Tensor,
                              attention: Attention | None = None, prompt_table: torch.Tensor | None = None) -> torch.Tensor:
        """``x + gate(attn2(adaln(x), modulate(context)))`` with the residual in the output
        GEMM (``transformer.py:201-223`` and ``:266-276``)."""
        attention = self.attn2 if attention is None else attention
        prompt_table = self.prompt_scale_shift_table if prompt_table is None else prompt_table
        prompt = _lib.table_add(prompt_table, args.prompt_timestep)
        query = adaln(value, ada[:, :, 7], ada[:, :, 6], self.norm_eps, compute_dtype(attention))
        context = modulate(args.context, prompt[:, :, 1], prompt[:, :, 0])
        return attention(query, context=context, mask=args.context_mask, residual=value, gate=ada[:, :, 8],
                         out_dtype=torch.float32)

    def _first_branches(self, args: TransformerArgs, table, attn1: Attention, attn2: Attention, prompt_table):
        """Self-attention then text cross-attention, FP32 residual out."""
        if args.sparse_attention is not None:
            raise ValueError("sparse (Sol-Attn) attention is not built for MI355X")
        x = args.x
        ada = _lib.table_add(table, args.timesteps)
        normalized = adaln(x, ada[:, :, 1], ada[:, :, 0], self.norm_eps, compute_dtype(attn1))
        x1 = attn1(normalized, pe=args.positional_embeddings, mask=args.self_attention_mask, residual=x,
                   gate=ada[:, :, 2], out_dtype=torch.float32)
        return self._text_cross_attention(x1, args, ada, attn2, prompt_table), ada

    def __call__(self, video: TransformerArgs | None, audio: TransformerArgs | None = None):
        video_present = video is not None and video.x.numel() > 0
        audio_present = audio is not None and audio.x.numel() > 0
        if audio_present and self.audio_config is None:
            raise ValueError("this block has no audio stream (constructed without audio_config)")
        run_video = video_present and video.enabled
        run_audio = audio_present and audio.enabled
        run_a2v = run_video and audio_present
        run_v2a = run_audio and video_present
        if not (run_video or run_audio):
            return video, audio

        video_value = video.x if video_present else None
        audio_value = audio.x if audio_present else None
        # With both streams running, the audio stream's work (a few hundred tokens: small launches
        # that leave most CUs idle) goes to a second HIP stream beside the video stream's. The
        # streams join before the A/V attention (each reads the other's value) and at the end of
        # the block; every tensor one stream hands the other stays referenced until that final
        # join, so the caching allocator cannot reuse its memory while the other stream reads it.
        main = side = None
        if run_video and run_audio and self.audio_side_stream and video.x.is_cuda:
            main = torch.cuda.current_stream(video.x.device)
            side = side_stream(video.x.device)
            side.wait_stream(main)
        if run_audio:
            with torch.cuda.stream(side):
                audio_value, audio_ada = self._first_branches(audio, self.audio_scale_shift_table, self.audio_attn1,
                                                              self.audio_attn2, self.audio_prompt_scale_shift_table)
        if run_video:
            video_value, video_ada = self._first_branches(video, self.scale_shift_table, self.attn1, self.attn2,
                                                          self.prompt_scale_shift_table)
        if run_a2v or run_v2a:
            for args in (video, audio):
                if (args.cross_scale_shift_timestep is None or args.cross_gate_timestep is None
                        or args.cross_positional_embeddings is None):
                    raise ValueError("A/V attention requires cross-modal preprocessing")
            a_scale_a2v, a_shift_a2v, a_scale_v2a, a_shift_v2a, gate_v2a = self._av_ada_values(
                self.scale_shift_table_a2v_ca_audio, audio.cross_scale_shift_timestep, audio.cross_gate_timestep)
            v_scale_a2v, v_shift_a2v, v_scale_v2a, v_shift_v2a, gate_a2v = self._av_ada_values(
                self.scale_shift_table_a2v_ca_video, video.cross_scale_shift_timestep, video.cross_gate_timestep)
            video_base, audio_base = video_value, audio_value
            if side is not None:
                main.wait_stream(side)
                side.wait_stream(main)
            # rms_norm(x) * (1 + scale) + shift is one AdaLN pass per (stream, direction)
            if run_a2v:
                cdt = compute_dtype(self.audio_to_video_attn)
                query = adaln(video_base, v_scale_a2v, v_shift_a2v, self.norm_eps, cdt)
                context = adaln(audio_base, a_scale_a2v, a_shift_a2v, self.norm_eps, cdt)
                video_value = self.audio_to_video_attn(
                    query, context=context, pe=video.cross_positional_embeddings,
                    k_pe=audio.cross_positional_embeddings, residual=video_base, gate=gate_a2v,
                    out_dtype=torch.float32)
            if run_v2a:
                with torch.cuda.stream(side):
                    cdt = compute_dtype(self.video_to_audio_attn)
                    query = adaln(audio_base, a_scale_v2a, a_shift_v2a, self.norm_eps, cdt)
                    context = adaln(video_base, v_scale_v2a, v_shift_v2a, self.norm_eps, cdt)
                    audio_value = self.video_to_audio_attn(
                        query, context=context, pe=audio.cross_positional_embeddings,
                        k_pe=video.cross_positional_embeddings, residual=audio_base, gate=gate_v2a,
                        out_dtype=torch.float32)
        if run_audio:
            with torch.cuda.stream(side):
                normalized = adaln(audio_value, audio_ada[:, :, 4], audio_ada[:, :, 3], self.norm_eps,
                                   compute_dtype(self.audio_attn1))
                audio = replace(audio, x=self.audio_ff(normalized, residual=audio_value, gate=audio_ada[:, :, 5],
                                                       out_dtype=audio.x.dtype))
        if run_video:
            normalized = adaln(video_value, video_ada[:, :, 4], video_ada[:, :, 3], self.norm_eps,
                               compute_dtype(self.attn1))
            video = replace(video, x=self.ff(normalized, residual=video_value, gate=video_ada[:, :, 5],
                                             out_dtype=video.x.dtype))
        if side is not None:
            main.wait_stream(side)
        return video, audio


__all__ = [
    "BasicAVTransformerBlock",
    "TransformerArgs",
    "compute_dtype",
    "TransformerConfig",
    "adaln",
    "gate",
    "gated_residual",
    "layer_norm_modulate",
    "modulate",
    "rms_norm",
]
