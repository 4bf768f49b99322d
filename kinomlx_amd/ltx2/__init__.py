"""LTX-2 on MI355X: the DiT block, the video transformer forward around it and one denoising
step (mirror of ``kinomlx/models/ltx2/transformer``, ``kinomlx/models/ltx2/kernels/
dense_attention.py``, ``kinomlx/models/ltx2/denoise.py`` and ``kinomlx/models/ltx2/state.py``)."""

from . import attention, dense_attention, denoise, feed_forward, model, rope, state, timestep, transformer, wrappers
from .attention import Attention, Linear, RMSNorm
from .feed_forward import FeedForward, GELUApprox
from .rope import LTXRopeType, apply_rotary_emb, apply_split_rotary_emb, precompute_freqs_cis
from .denoise import LTX2DenoiseError, denoise_step, modality_from_state
from .model import LTXAVModel
from .state import LatentState, post_process_latent
from .timestep import AdaLayerNormSingle, CombinedTimestepEmbeddings, TimestepEmbedding, get_timestep_embedding
from .transformer import BasicAVTransformerBlock, TransformerArgs, TransformerConfig
from .wrappers import Modality, X0Model

__all__ = [
    "AdaLayerNormSingle",
    "Attention",
    "BasicAVTransformerBlock",
    "CombinedTimestepEmbeddings",
    "FeedForward",
    "GELUApprox",
    "LTX2DenoiseError",
    "LTXAVModel",
    "LTXRopeType",
    "LatentState",
    "Linear",
    "Modality",
    "RMSNorm",
    "TimestepEmbedding",
    "TransformerArgs",
    "TransformerConfig",
    "X0Model",
    "apply_rotary_emb",
    "apply_split_rotary_emb",
    "attention",
    "denoise",
    "denoise_step",
    "dense_attention",
    "feed_forward",
    "get_timestep_embedding",
    "modality_from_state",
    "model",
    "post_process_latent",
    "precompute_freqs_cis",
    "rope",
    "state",
    "timestep",
    "transformer",
    "wrappers",
]
