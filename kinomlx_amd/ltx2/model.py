"""The LTX-2 transformer forward on MI355X: preprocessing, the block stack and the output heads,
for the video stream alone or jointly with the audio stream.

Mirror of ``kinomlx/models/ltx2/transformer/model.py`` (``LTXAVModel``: ``__init__``
``:137-323``, ``_cast_modality`` ``:364-384``, ``_process_blocks`` ``:407-467``, ``_output``
``:577-593``, ``__call__`` ``:595-635``) and of ``ModalityPreprocessor``
(``preprocessing.py:26-214``):

* ``patchify_proj`` and ``proj_out`` are MFMA GEMMs with their biases in the epilogue;
* the AdaLN modulation rows come from ``AdaLayerNormSingle`` (timestep kernel + GEMMs), the
  timestep scale folded into the timestep kernel;
* the RoPE tables from the table kernel (``precompute_freqs_cis``);
* the blocks run eagerly, one after another, on the current stream (no compile groups: every
  block is already a fixed sequence of HIP launches);
* the output head is one LayerNorm-modulate pass and the projection GEMM.

Weights are assigned after construction, as the reference's checkpoint loader does.
"""

from __future__ import annotations

from dataclasses import replace

import torch

from .. import _lib
from .attention import Linear
from .rope import precompute_freqs_cis
from .timestep import AdaLayerNormSingle
from .transformer import BasicAVTransformerBlock, TransformerArgs, TransformerConfig, layer_norm_modulate
from .wrappers import Modality


# bf16 limits used by the reference's masks (``preprocessing.py:14-23``)
_MINIMUM = -3.3895313892515355e38
_TINY = 1.1754943508222875e-38


class ModalityPreprocessor:
    """Prepare one stream and its A/V cross-attention inputs (``preprocessing.py:26-214``):
    ``patchify_proj``, the AdaLN rows, the prompt rows, the RoPE tables, and with a cross
    modality the temporal cross tables, the cross scale/shift rows and the cross gate rows."""

    def __init__(self, *, model: "LTXAVModel", prefix: str, inner_dim: int, heads: int, max_pos: tuple[int, ...],
                 cross_dim: int, cross_max_pos: int) -> None:
        self.model = model
        self.prefix = prefix
        self.inner_dim = inner_dim
        self.heads = heads
        self.max_pos = tuple(max_pos)
        self.cross_dim = cross_dim
        self.cross_max_pos = cross_max_pos

    def _part(self, name: str):
        return getattr(self.model, f"{self.prefix}{name}")

    def _timestep(self, value: torch.Tensor, adaln: AdaLayerNormSingle, batch: int, scale: float):
        """``adaln((value * scale).reshape(-1))`` reshaped to ``(B, -1, n, D)`` and ``(B, -1, D)``
        (``preprocessing.py:66-83``)."""
        modulation, embedded = adaln(value.reshape(-1), self.model.compute_dtype, time_scale=scale)
        modulation = modulation.reshape(batch, -1, adaln.num_embeddings, adaln.embedding_dim)
        return modulation, embedded.reshape(batch, -1, adaln.embedding_dim)

    @staticmethod
    def _sigma(value: torch.Tensor, batch: int) -> torch.Tensor:
        """Scalar or ``(B,)`` sigma as ``(B,)`` (``preprocessing.py:126-132``)."""
        if value.dim() == 0:
            return value[None].expand(batch)
        if value.dim() != 1 or value.shape[0] != batch:
            raise ValueError("modality sigma must be scalar or have shape (batch,)")
        return value

    def _context_mask(self, mask: torch.Tensor | None) -> torch.Tensor | None:
        """Text mask -> additive bias in the compute dtype (``preprocessing.py:85-96``): float masks
        as given ((B, Tc) -> (B, 1, 1, Tc), (B, T, Tc) -> (B, 1, T, Tc)); others 0 where set and the
        dtype minimum where not."""
        if mask is None:
            return None
        dtype = self.model.compute_dtype
        if mask.dtype in (torch.float16, torch.bfloat16, torch.float32):
            if mask.dim() == 2:
                mask = mask[:, None, None, :]
            elif mask.dim() == 3:
                mask = mask[:, None, :, :]
            return mask.to(dtype)
        return ((mask.to(dtype) - 1.0) * -_MINIMUM).reshape(mask.shape[0], 1, -1, mask.shape[-1])

    @staticmethod
    def _self_attention_mask(mask: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor | None:
        """Soft self-attention mask in [0, 1] -> log bias (``preprocessing.py:98-105``): log(max(m,
        tiny)) where m > 0, the dtype minimum elsewhere, as (B, 1, T, T)."""
        if mask is None:
            return None
        value = mask.float()
        log_bias = torch.log(torch.clamp(value, min=_TINY))
        return torch.where(value > 0, log_bias, torch.full_like(value, _MINIMUM))[:, None, ...].to(dtype)

    def _rope(self, positions: torch.Tensor, *, dim: int, max_pos: tuple[int, ...]):
        m = self.model
        return precompute_freqs_cis(positions, dim=dim, out_dtype=torch.float32, theta=m.theta, max_pos=max_pos,
                                    use_middle_indices_grid=True, num_attention_heads=self.heads,
                                    use_double_precision=m.double_precision_rope)

    def prepare(self, modality: Modality, cross_modality: Modality | None) -> TransformerArgs:
        """``preprocessing.py:134-214``."""
        m = self.model
        if modality.keyframes_mask is not None:
            raise ValueError("keyframe position embeddings are not built for MI355X")
        hidden = self._part("patchify_proj")(modality.latent)
        batch = hidden.shape[0]
        timestep, embedded = self._timestep(modality.timesteps, self._part("adaln_single"), batch, m.timestep_scale)
        sigma = self._sigma(modality.sigma, batch)
        prompt_timestep = None
        prompt_adaln = self._part("prompt_adaln_single")
        if prompt_adaln is not None:
            prompt_timestep, _ = self._timestep(sigma, prompt_adaln, batch, m.timestep_scale)
        args = TransformerArgs(
            x=hidden,
            context=modality.context.reshape(batch, -1, self.inner_dim),
            context_mask=self._context_mask(modality.context_mask),
            self_attention_mask=self._self_attention_mask(modality.attention_mask, m.compute_dtype),
            timesteps=timestep,
            positional_embeddings=modality.positional_embeddings
            or self._rope(modality.positions, dim=self.inner_dim, max_pos=self.max_pos),
            embedded_timestep=embedded,
            prompt_timestep=prompt_timestep,
            enabled=modality.enabled,
            sparse_attention=modality.sparse_attention,
        )
        if cross_modality is None:
            return args
        cross_pe = modality.cross_positional_embeddings or self._rope(
            modality.positions[:, 0:1, ...], dim=self.cross_dim, max_pos=(self.cross_max_pos,))
        stream = "video" if self.prefix == "" else "audio"
        direction = "a2v" if stream == "video" else "v2a"
        scale_shift, _ = self._timestep(modality.timesteps, getattr(m, f"av_ca_{stream}_scale_shift_adaln_single"),
                                        batch, m.timestep_scale)
        cross_sigma = self._sigma(cross_modality.sigma, batch)
        gate, _ = self._timestep(cross_sigma, getattr(m, f"av_ca_{direction}_gate_adaln_single"), batch,
                                 m.av_gate_scale)
        return replace(args, cross_positional_embeddings=cross_pe, cross_scale_shift_timestep=scale_shift,
                       cross_gate_timestep=gate)


class LTXAVModel:
    """The LTX-2 transformer: the video stream, and with ``audio_heads`` set the audio stream and
    the A/V cross-attention of every block. Audio heads must equal video heads (the A/V
    attention runs ``audio_heads`` heads on both sides)."""

    def __init__(
        self,
        *,
        num_layers: int = 48,
        video_heads: int = 32,
        video_head_dim: int = 128,
        audio_heads: int | None = None,
        audio_head_dim: int = 64,
        video_in_channels: int = 128,
        video_out_channels: int = 128,
        audio_in_channels: int = 128,
        audio_out_channels: int = 128,
        video_context_dim: int = 4096,
        audio_context_dim: int | None = None,
        video_max_pos: tuple[int, int, int] = (20, 2048, 2048),
        audio_max_pos: tuple[int] = (20,),
        positional_embedding_theta: float = 10000.0,
        timestep_scale_multiplier: float = 1000.0,
        av_ca_timestep_scale_multiplier: float = 1000.0,
        norm_eps: float = 1e-6,
        ff_bias: bool = True,
        audio_ff_bias: bool = True,
        use_prompt_adaln_single: bool = True,
        compute_dtype: torch.dtype = torch.bfloat16,
        double_precision_rope: bool = True,
        apply_gated_attention: bool = True,
    ) -> None:
        if num_layers <= 0:
            raise ValueError("transformer must contain at least one block")
        if compute_dtype != torch.bfloat16:
            raise ValueError(f"the MI355X transformer computes in bfloat16, got {compute_dtype}")
        if audio_heads is not None and audio_heads != video_heads:
            raise ValueError("LTX-2 A/V cross-attention requires equal head counts")
        self.compute_dtype = compute_dtype
        self.norm_eps = norm_eps
        self.video_inner_dim = video_heads * video_head_dim
        self.inner_dim = self.video_inner_dim
        if video_context_dim != self.video_inner_dim:
            raise ValueError("LTX-2 video context must match the video hidden dimension")
        self.heads = video_heads
        self.in_channels = video_in_channels
        self.out_channels = video_out_channels
        self.max_pos = tuple(video_max_pos)
        self.theta = positional_embedding_theta
        self.timestep_scale = timestep_scale_multiplier
        self.av_gate_scale = av_ca_timestep_scale_multiplier
        self.double_precision_rope = double_precision_rope
        self.has_audio = audio_heads is not None

        self.patchify_proj: Linear | None = None
        self.adaln_single = AdaLayerNormSingle(self.video_inner_dim, 9)
        self.prompt_adaln_single = (
            AdaLayerNormSingle(self.video_inner_dim, 2) if use_prompt_adaln_single else None
        )
        self.scale_shift_table: torch.Tensor | None = None
        self.proj_out: Linear | None = None
        video_config = TransformerConfig(dim=self.video_inner_dim, heads=video_heads, head_dim=video_head_dim,
                                         context_dim=video_context_dim, ff_bias=ff_bias,
                                         apply_gated_attention=apply_gated_attention)
        audio_config = None
        if self.has_audio:
            self.audio_inner_dim = audio_heads * audio_head_dim
            if (audio_context_dim or self.audio_inner_dim) != self.audio_inner_dim:
                raise ValueError("LTX-2 audio context must match the audio hidden dimension")
            audio_config = TransformerConfig(dim=self.audio_inner_dim, heads=audio_heads, head_dim=audio_head_dim,
                                             context_dim=self.audio_inner_dim, ff_bias=audio_ff_bias,
                                             apply_gated_attention=apply_gated_attention)
            self.audio_in_channels = audio_in_channels
            self.audio_out_channels = audio_out_channels
            self.audio_patchify_proj: Linear | None = None
            self.audio_adaln_single = AdaLayerNormSingle(self.audio_inner_dim, 9)
            self.audio_prompt_adaln_single = (
                AdaLayerNormSingle(self.audio_inner_dim, 2) if use_prompt_adaln_single else None
            )
            self.audio_scale_shift_table: torch.Tensor | None = None
            self.audio_proj_out: Linear | None = None
            self.av_ca_video_scale_shift_adaln_single = AdaLayerNormSingle(self.video_inner_dim, 4)
            self.av_ca_a2v_gate_adaln_single = AdaLayerNormSingle(self.video_inner_dim, 1)
            self.av_ca_audio_scale_shift_adaln_single = AdaLayerNormSingle(self.audio_inner_dim, 4)
            self.av_ca_v2a_gate_adaln_single = AdaLayerNormSingle(self.audio_inner_dim, 1)
            cross_max_pos = max(video_max_pos[0], audio_max_pos[0])
            self._audio_preprocessor = ModalityPreprocessor(
                model=self, prefix="audio_", inner_dim=self.audio_inner_dim, heads=audio_heads,
                max_pos=tuple(audio_max_pos), cross_dim=self.audio_inner_dim, cross_max_pos=cross_max_pos)
        else:
            cross_max_pos = video_max_pos[0]
        self._video_preprocessor = ModalityPreprocessor(
            model=self, prefix="", inner_dim=self.video_inner_dim, heads=video_heads, max_pos=self.max_pos,
            cross_dim=getattr(self, "audio_inner_dim", self.video_inner_dim), cross_max_pos=cross_max_pos)
        self.transformer_blocks = [
            BasicAVTransformerBlock(index, video_config=video_config, audio_config=audio_config, norm_eps=norm_eps)
            for index in range(num_layers)
        ]

    @property
    def num_blocks(self) -> int:
        return len(self.transformer_blocks)

    def _prepare(self, modality: Modality) -> TransformerArgs:
        """The video stream prepared without a cross modality."""
        return self._video_preprocessor.prepare(modality, None)

    def _cast_modality(self, modality: Modality) -> Modality:
        """Latent and context in the compute dtype, tables in FP32 (``model.py:364-384``)."""
        positional = modality.positional_embeddings
        if positional is not None:
            positional = (positional[0].float(), positional[1].float())
        cross = modality.cross_positional_embeddings
        if cross is not None:
            cross = (cross[0].float(), cross[1].float())
        return replace(modality, latent=modality.latent.to(self.compute_dtype),
                       context=modality.context.to(self.compute_dtype), positional_embeddings=positional,
                       cross_positional_embeddings=cross)

    # ---- blocks and output ---------------------------------------------------------------------

    def _process_blocks(self, video: TransformerArgs | None, audio: TransformerArgs | None = None):
        """Every block in order (``model.py:407-467``, the eager branch)."""
        for block in self.transformer_blocks:
            video, audio = block(video, audio)
        return video, audio

    def _output(self, value: torch.Tensor, embedded_timestep: torch.Tensor | None, table: torch.Tensor,
                projection: Linear) -> torch.Tensor:
        """``proj_out(layer_norm(x) * (1 + scale) + shift)`` with ``(shift, scale)`` =
        ``(table + embedded_timestep)`` rounded to the value dtype (``model.py:577-593``)."""
        if embedded_timestep is None:
            raise ValueError("transformer output requires an embedded timestep")
        rows = table.shape[0]
        modulation = _lib.table_add(table, embedded_timestep[:, :, None, :].expand(-1, -1, rows, -1),
                                    round_to=value.dtype)
        shift, scale = modulation[:, :, 0], modulation[:, :, 1]
        normalized = layer_norm_modulate(value, shift, scale, self.norm_eps)
        return projection(normalized)

    @staticmethod
    def _present(modality: Modality | None) -> bool:
        return modality is not None and modality.latent.numel() > 0

    def __call__(self, video: Modality | None, audio: Modality | None = None):
        """``(video velocity, audio velocity)`` (``model.py:595-635``)."""
        if video is None and audio is None:
            raise ValueError("at least one modality is required")
        if audio is not None and not self.has_audio:
            raise ValueError("this transformer has no audio stream (constructed without audio_heads)")
        video = self._cast_modality(video) if video is not None else None
        audio = self._cast_modality(audio) if audio is not None else None
        video_cross = audio if self._present(audio) else None
        audio_cross = video if self._present(video) else None
        video_args = self._video_preprocessor.prepare(video, video_cross) if self._present(video) else None
        audio_args = self._audio_preprocessor.prepare(audio, audio_cross) if self._present(audio) else None
        video_args, audio_args = self._process_blocks(video_args, audio_args)
        video_out = (self._output(video_args.x, video_args.embedded_timestep, self.scale_shift_table, self.proj_out)
                     if video_args is not None else None)
        audio_out = (self._output(audio_args.x, audio_args.embedded_timestep, self.audio_scale_shift_table,
                                  self.audio_proj_out) if audio_args is not None else None)
        return video_out, audio_out


__all__ = ["LTXAVModel", "ModalityPreprocessor"]
