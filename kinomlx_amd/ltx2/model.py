"""The LTX-2 video transformer forward on MI355X: preprocessing, the block stack and the output
head.

Mirror of the video path of ``kinomlx/models/ltx2/transformer/model.py`` (``LTXAVModel``:
``__init__`` ``:137-240``, ``_cast_modality`` ``:364-384``, ``_process_blocks`` ``:407-467``,
``_output`` ``:577-593``, ``__call__`` ``:595-635``) and of ``ModalityPreprocessor.prepare``
(``preprocessing.py:134-214``) for one stream without A/V cross-attention:

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

from .attention import Linear
from .rope import precompute_freqs_cis
from .timestep import AdaLayerNormSingle
from .transformer import BasicAVTransformerBlock, TransformerArgs, TransformerConfig, layer_norm_modulate
from .wrappers import Modality


class LTXAVModel:
    """Video stream of the LTX-2 transformer. ``audio`` arguments must be ``None``: the audio
    stream and A/V cross-attention are not built for MI355X."""

    def __init__(
        self,
        *,
        num_layers: int = 48,
        video_heads: int = 32,
        video_head_dim: int = 128,
        video_in_channels: int = 128,
        video_out_channels: int = 128,
        video_context_dim: int = 4096,
        video_max_pos: tuple[int, int, int] = (20, 2048, 2048),
        positional_embedding_theta: float = 10000.0,
        timestep_scale_multiplier: float = 1000.0,
        norm_eps: float = 1e-6,
        ff_bias: bool = True,
        use_prompt_adaln_single: bool = True,
        compute_dtype: torch.dtype = torch.bfloat16,
        double_precision_rope: bool = True,
        apply_gated_attention: bool = True,
    ) -> None:
        if num_layers <= 0:
            raise ValueError("transformer must contain at least one block")
        if compute_dtype != torch.bfloat16:
            raise ValueError(f"the MI355X transformer computes in bfloat16, got {compute_dtype}")
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
        self.double_precision_rope = double_precision_rope

        self.patchify_proj: Linear | None = None
        self.adaln_single = AdaLayerNormSingle(self.video_inner_dim, 9)
        self.prompt_adaln_single = (
            AdaLayerNormSingle(self.video_inner_dim, 2) if use_prompt_adaln_single else None
        )
        self.scale_shift_table: torch.Tensor | None = None
        self.proj_out: Linear | None = None
        config = TransformerConfig(dim=self.video_inner_dim, heads=video_heads, head_dim=video_head_dim,
                                   context_dim=video_context_dim, ff_bias=ff_bias,
                                   apply_gated_attention=apply_gated_attention)
        self.transformer_blocks = [
            BasicAVTransformerBlock(index, video_config=config, norm_eps=norm_eps) for index in range(num_layers)
        ]

    @property
    def num_blocks(self) -> int:
        return len(self.transformer_blocks)

    # ---- preprocessing (preprocessing.py:66-214) -----------------------------------------------

    def _timestep(self, value: torch.Tensor, adaln: AdaLayerNormSingle, batch: int):
        """``adaln((value * timestep_scale).reshape(-1))`` reshaped to ``(B, -1, n, D)`` and
        ``(B, -1, D)`` (``preprocessing.py:66-83``)."""
        modulation, embedded = adaln(value.reshape(-1), self.compute_dtype, time_scale=self.timestep_scale)
        modulation = modulation.reshape(batch, -1, adaln.num_embeddings, adaln.embedding_dim)
        embedded = embedded.reshape(batch, -1, adaln.embedding_dim)
        return modulation, embedded

    @staticmethod
    def _sigma(value: torch.Tensor, batch: int) -> torch.Tensor:
        """Scalar or ``(B,)`` sigma as ``(B,)`` (``preprocessing.py:126-132``)."""
        if value.dim() == 0:
            return value[None].expand(batch)
        if value.dim() != 1 or value.shape[0] != batch:
            raise ValueError("modality sigma must be scalar or have shape (batch,)")
        return value

    def _rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return precompute_freqs_cis(positions, dim=self.inner_dim, out_dtype=torch.float32, theta=self.theta,
                                    max_pos=self.max_pos, use_middle_indices_grid=True,
                                    num_attention_heads=self.heads,
                                    use_double_precision=self.double_precision_rope)

    def _prepare(self, modality: Modality) -> TransformerArgs:
        """``ModalityPreprocessor.prepare`` without a cross modality (``preprocessing.py:134-183``)."""
        if modality.keyframes_mask is not None:
            raise ValueError("keyframe position embeddings are not built for MI355X")
        if modality.context_mask is not None or modality.attention_mask is not None:
            raise ValueError("masked attention is not built for MI355X")
        hidden = self.patchify_proj(modality.latent)
        batch = hidden.shape[0]
        timestep, embedded_timestep = self._timestep(modality.timesteps, self.adaln_single, batch)
        sigma = self._sigma(modality.sigma, batch)
        prompt_timestep = None
        if self.prompt_adaln_single is not None:
            prompt_timestep, _ = self._timestep(sigma, self.prompt_adaln_single, batch)
        context = modality.context.reshape(batch, -1, self.inner_dim)
        positional = modality.positional_embeddings or self._rope(modality.positions)
        return TransformerArgs(
            x=hidden,
            context=context,
            timesteps=timestep,
            positional_embeddings=positional,
            embedded_timestep=embedded_timestep,
            prompt_timestep=prompt_timestep,
            enabled=modality.enabled,
            sparse_attention=modality.sparse_attention,
        )

    def _cast_modality(self, modality: Modality) -> Modality:
        """Latent and context in the compute dtype, tables in FP32 (``model.py:364-384``)."""
        positional = modality.positional_embeddings
        if positional is not None:
            positional = (positional[0].float(), positional[1].float())
        return replace(modality, latent=modality.latent.to(self.compute_dtype),
                       context=modality.context.to(self.compute_dtype), positional_embeddings=positional)

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
        modulation = (table[None, None].float() + embedded_timestep[:, :, None, :].float()).to(value.dtype).float()
        shift = modulation[:, :, 0].contiguous()
        scale = modulation[:, :, 1].contiguous()
        normalized = layer_norm_modulate(value, shift, scale, self.norm_eps)
        return projection(normalized)

    def __call__(self, video: Modality | None, audio: Modality | None = None):
        if audio is not None:
            raise ValueError("the audio stream and A/V attention are not built for MI355X")
        if video is None:
            raise ValueError("at least one modality is required")
        if video.latent.numel() == 0:
            return None, None
        video = self._cast_modality(video)
        args = self._prepare(video)
        args, _ = self._process_blocks(args, None)
        return self._output(args.x, args.embedded_timestep, self.scale_shift_table, self.proj_out), None


__all__ = ["LTXAVModel"]
