"""Seeded synthetic DiT-block workloads for the five benchmark configurations.

Every tensor is drawn from its own ``torch.Generator`` seeded by (seed, name), in float32 on the
CPU, then rounded once to bf16 where the block stores it in bf16. Weights ~ N(0, 0.02); hidden
states, context and the conditioning vector ~ N(0, 1). Modulation follows the reference's AdaLN
path: a seeded N(0, 0.02) linear layer maps a 1024-d conditioning vector to the modulation rows
(LTX ``AdaLayerNormSingle`` output ``(1, 1, 9, D)`` in bf16 plus an fp32 ``scale_shift_table``,
``kinomlx/models/ltx2/transformer/transformer.py:179-186``; FLUX ``Modulation``,
``kinomlx/models/flux2/transformer.py:223-229``). There are no checkpoints: the numbers measure
kernels, not a trained model.

``params`` dicts map parameter names to CPU tensors; ``build_*`` functions turn them into the
MI355X block objects on a device.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import torch

COND_DIM = 1024


@dataclass(frozen=True)
class LTXSpec:
    """LTX-2-like video block: ``grid`` = (t, h, w) latent tokens, text via cross-attention."""

    grid: tuple[int, int, int]
    text_tokens: int
    dim: int = 4096
    heads: int = 32
    head_dim: int = 128
    ff_mult: int = 4
    bits: int | None = None  # affine-quantized linears (4 or 8) when set
    group_size: int = 64

    @property
    def tokens(self) -> int:
        return self.grid[0] * self.grid[1] * self.grid[2]


@dataclass(frozen=True)
class FluxSpec:
    """FLUX.2-like (or config-1) image block: ``grid`` = (h, w) image tokens joined with text."""

    grid: tuple[int, int]
    text_tokens: int
    dim: int
    heads: int
    head_dim: int
    ff_hidden: int
    ff: str  # "swiglu" (FLUX.2) or "gelu" (config 1, LTX FeedForward with biases)
    single: bool = False  # also run one single-stream block (config 2)

    @property
    def image_tokens(self) -> int:
        return self.grid[0] * self.grid[1]


CONFIGS = {
    1: FluxSpec(grid=(32, 32), text_tokens=128, dim=1024, heads=16, head_dim=64, ff_hidden=4096, ff="gelu"),
    2: FluxSpec(grid=(64, 64), text_tokens=512, dim=4096, heads=32, head_dim=128, ff_hidden=12288, ff="swiglu",
                single=True),
    3: LTXSpec(grid=(16, 18, 32), text_tokens=256),
    4: LTXSpec(grid=(16, 18, 32), text_tokens=256, bits=4),
    5: LTXSpec(grid=(31, 22, 40), text_tokens=256, bits=4),
}


def _generator(seed: int, name: str) -> torch.Generator:
    digest = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return torch.Generator().manual_seed(int.from_bytes(digest[:8], "little") & ((1 << 63) - 1))


def normal(seed: int, name: str, shape, std: float = 1.0, mean: float = 0.0) -> torch.Tensor:
    """float32 N(mean, std^2) of ``shape`` from the (seed, name) stream."""
    return torch.randn(tuple(shape), generator=_generator(seed, name), dtype=torch.float32) * std + mean


def bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16)


# ---- LTX-2 -------------------------------------------------------------------------------------


def ltx_positions(grid: tuple[int, int, int]) -> torch.Tensor:
    """``(1, 3, T, 2)`` integer latent-grid bounds ``[i, i + 1]`` per axis, t-major token order."""
    t, h, w = grid
    tt, hh, ww = torch.meshgrid(torch.arange(t), torch.arange(h), torch.arange(w), indexing="ij")
    start = torch.stack([tt.reshape(-1), hh.reshape(-1), ww.reshape(-1)]).float()
    return torch.stack([start, start + 1.0], dim=-1)[None]


def _ltx_attention_params(p: dict, seed: int, prefix: str, dim: int, heads: int,
                          dtype: torch.dtype = torch.bfloat16) -> None:
    for name in ("to_q", "to_k", "to_v", "to_out"):
        p[f"{prefix}.{name}.weight"] = normal(seed, f"{prefix}.{name}.weight", (dim, dim), 0.02).to(dtype)
        p[f"{prefix}.{name}.bias"] = normal(seed, f"{prefix}.{name}.bias", (dim,), 0.02).to(dtype)
    p[f"{prefix}.to_gate_logits.weight"] = normal(seed, f"{prefix}.to_gate_logits.weight", (heads, dim), 0.02).to(dtype)
    p[f"{prefix}.to_gate_logits.bias"] = normal(seed, f"{prefix}.to_gate_logits.bias", (heads,), 0.02).to(dtype)
    for name in ("q_norm", "k_norm"):
        p[f"{prefix}.{name}.weight"] = normal(seed, f"{prefix}.{name}.weight", (dim,), 0.02, 1.0).to(dtype)


def ltx_params(spec: LTXSpec, seed: int = 0, dtype: torch.dtype = torch.bfloat16) -> dict[str, torch.Tensor]:
    """Dense parameters of one LTX video block (``dtype``: bf16, or fp16 for the reference's
    default FP16 transformer) plus its per-step modulation rows (fp32 tables, ``dtype`` rows)."""
    d = spec.dim
    p: dict[str, torch.Tensor] = {}
    _ltx_attention_params(p, seed, "attn1", d, spec.heads, dtype)
    _ltx_attention_params(p, seed, "attn2", d, spec.heads, dtype)
    f = d * spec.ff_mult
    p["ff.proj_in.weight"] = normal(seed, "ff.proj_in.weight", (f, d), 0.02).to(dtype)
    p["ff.proj_in.bias"] = normal(seed, "ff.proj_in.bias", (f,), 0.02).to(dtype)
    p["ff.proj_out.weight"] = normal(seed, "ff.proj_out.weight", (d, f), 0.02).to(dtype)
    p["ff.proj_out.bias"] = normal(seed, "ff.proj_out.bias", (d,), 0.02).to(dtype)
    p["scale_shift_table"] = normal(seed, "scale_shift_table", (9, d), 0.02)
    p["prompt_scale_shift_table"] = normal(seed, "prompt_scale_shift_table", (2, d), 0.02)
    cond = normal(seed, "cond", (1, COND_DIM))
    w_mod = bf16(normal(seed, "adaln.linear.weight", (9 * d, COND_DIM), 0.02)).float()
    p["timesteps"] = (cond @ w_mod.T).reshape(1, 1, 9, d).to(dtype)
    return p


QUANTIZED_LTX_LINEARS = tuple(
    f"{a}.{n}" for a in ("attn1", "attn2") for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits")
) + ("ff.proj_in", "ff.proj_out")


def quantize_ltx_params(p: dict[str, torch.Tensor], bits: int, group_size: int = 64) -> dict[str, torch.Tensor]:
    """Replace every block linear's weight by its packed affine form (``.wq/.scales/.biases``)."""
    from .kernels.quantized import quantize

    q = dict(p)
    for name in QUANTIZED_LTX_LINEARS:
        words, scales, biases = quantize(q.pop(f"{name}.weight"), group_size, bits)
        q[f"{name}.wq"] = words
        q[f"{name}.scales"] = scales
        q[f"{name}.biases"] = biases
        q[f"{name}.group_size"] = torch.tensor(group_size)
        q[f"{name}.bits"] = torch.tensor(bits)
    return q


def ltx_inputs(spec: LTXSpec, seed: int = 0, dtype: torch.dtype = torch.bfloat16) -> dict[str, torch.Tensor]:
    """Hidden states ``(1, T, D)``, context ``(1, Tc, D)`` (bf16, or ``dtype``) and RoPE positions."""
    return {
        "x": normal(seed, "x", (1, spec.tokens, spec.dim)).to(dtype),
        "context": normal(seed, "context", (1, spec.text_tokens, spec.dim)).to(dtype),
        "positions": ltx_positions(spec.grid),
    }


def _layer(p: dict, name: str, device):
    from .kernels.quantized import QuantizedLinear
    from .ltx2.attention import Linear

    bias = p.get(f"{name}.bias")
    bias = None if bias is None else bias.to(device)
    if f"{name}.wq" in p:
        return QuantizedLinear(
            p[f"{name}.wq"].to(device), p[f"{name}.scales"].to(device), p[f"{name}.biases"].to(device), bias,
            group_size=int(p[f"{name}.group_size"]), bits=int(p[f"{name}.bits"]),
        )
    return Linear(p[f"{name}.weight"].to(device), bias)


def build_ltx_block(spec: LTXSpec, p: dict[str, torch.Tensor], device, *, fuse: bool = True):
    """The MI355X ``BasicAVTransformerBlock`` holding ``p``'s weights on ``device``."""
    from .ltx2.transformer import BasicAVTransformerBlock, TransformerConfig

    cfg = TransformerConfig(dim=spec.dim, heads=spec.heads, head_dim=spec.head_dim, context_dim=spec.dim)
    block = BasicAVTransformerBlock(0, video_config=cfg)
    for a in ("attn1", "attn2"):
        attn = getattr(block, a)
        for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits"):
            setattr(attn, n, _layer(p, f"{a}.{n}", device))
        attn.q_norm.weight = p[f"{a}.q_norm.weight"].to(device)
        attn.k_norm.weight = p[f"{a}.k_norm.weight"].to(device)
    block.ff.project_in.proj = _layer(p, "ff.proj_in", device)
    block.ff.project_out = _layer(p, "ff.proj_out", device)
    block.scale_shift_table = p["scale_shift_table"].to(device)
    block.prompt_scale_shift_table = p["prompt_scale_shift_table"].to(device)
    if fuse:
        block.fuse_projections()
    return block


@dataclass(frozen=True)
class LTXAudioSpec:
    """The audio stream of a joint LTX-2 block: ``tokens`` audio latents (25 per second of
    video), text via cross-attention, ``heads`` equal to the video stream's."""

    tokens: int
    text_tokens: int
    dim: int = 2048
    heads: int = 32
    head_dim: int = 64
    ff_mult: int = 4


def _ltx_cross_params(p: dict, seed: int, prefix: str, qdim: int, cdim: int, heads: int, head_dim: int) -> None:
    inner = heads * head_dim
    for name, shape in (("to_q", (inner, qdim)), ("to_k", (inner, cdim)), ("to_v", (inner, cdim)),
                        ("to_out", (qdim, inner))):
        p[f"{prefix}.{name}.weight"] = bf16(normal(seed, f"{prefix}.{name}.weight", shape, 0.02))
        p[f"{prefix}.{name}.bias"] = bf16(normal(seed, f"{prefix}.{name}.bias", (shape[0],), 0.02))
    p[f"{prefix}.to_gate_logits.weight"] = bf16(normal(seed, f"{prefix}.to_gate_logits.weight", (heads, qdim), 0.02))
    p[f"{prefix}.to_gate_logits.bias"] = bf16(normal(seed, f"{prefix}.to_gate_logits.bias", (heads,), 0.02))
    for name in ("q_norm", "k_norm"):
        p[f"{prefix}.{name}.weight"] = bf16(normal(seed, f"{prefix}.{name}.weight", (inner,), 0.02, 1.0))


def ltx_av_params(spec: LTXSpec, audio: LTXAudioSpec, seed: int = 0) -> dict[str, torch.Tensor]:
    """Dense bf16 parameters of one joint A/V block: the video block of ``ltx_params``, the audio
    stream under ``audio_`` names, both cross-attentions and their ``(5, D)`` tables, and the
    per-step rows (``timesteps`` (1, 1, 9, D), ``audio_timesteps``, ``cross_ss`` (1, 1, 4, D),
    ``cross_gate`` (1, 1, 1, D) and their audio forms)."""
    p = ltx_params(spec, seed)
    a = ltx_params(LTXSpec(grid=(1, 1, audio.tokens), text_tokens=audio.text_tokens, dim=audio.dim,
                           heads=audio.heads, head_dim=audio.head_dim, ff_mult=audio.ff_mult), seed + 7919)
    for name, value in a.items():
        p[f"audio_{name}"] = value
    _ltx_cross_params(p, seed, "audio_to_video_attn", spec.dim, audio.dim, audio.heads, audio.head_dim)
    _ltx_cross_params(p, seed, "video_to_audio_attn", audio.dim, spec.dim, audio.heads, audio.head_dim)
    p["scale_shift_table_a2v_ca_video"] = normal(seed, "av_table_video", (5, spec.dim), 0.02)
    p["scale_shift_table_a2v_ca_audio"] = normal(seed, "av_table_audio", (5, audio.dim), 0.02)
    for pre, d in (("", spec.dim), ("audio_", audio.dim)):
        p[f"{pre}cross_ss"] = bf16(normal(seed, f"{pre}cross_ss", (1, 1, 4, d), 0.3))
        p[f"{pre}cross_gate"] = bf16(normal(seed, f"{pre}cross_gate", (1, 1, 1, d), 0.3))
    return p


def ltx_av_inputs(spec: LTXSpec, audio: LTXAudioSpec, seed: int = 0) -> dict[str, torch.Tensor]:
    """``ltx_inputs`` plus the audio stream ``(1, Ta, Da)``, its context and its ``(1, 1, Ta, 2)``
    temporal bounds."""
    out = ltx_inputs(spec, seed)
    out["audio_x"] = bf16(normal(seed, "audio_x", (1, audio.tokens, audio.dim)))
    out["audio_context"] = bf16(normal(seed, "audio_context", (1, audio.text_tokens, audio.dim)))
    start = torch.arange(audio.tokens, dtype=torch.float32)
    out["audio_positions"] = torch.stack([start, start + 1.0], dim=-1)[None, None]
    return out


def build_ltx_av_block(spec: LTXSpec, audio: LTXAudioSpec, p: dict, device, *, fuse: bool = True):
    """The MI355X joint ``BasicAVTransformerBlock`` holding ``p``'s weights on ``device``."""
    from .ltx2.transformer import BasicAVTransformerBlock, TransformerConfig

    vcfg = TransformerConfig(dim=spec.dim, heads=spec.heads, head_dim=spec.head_dim, context_dim=spec.dim)
    acfg = TransformerConfig(dim=audio.dim, heads=audio.heads, head_dim=audio.head_dim, context_dim=audio.dim)
    block = BasicAVTransformerBlock(0, video_config=vcfg, audio_config=acfg)
    for pre in ("", "audio_"):
        for a in ("attn1", "attn2"):
            attn = getattr(block, f"{pre}{a}")
            for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits"):
                setattr(attn, n, _layer(p, f"{pre}{a}.{n}", device))
            attn.q_norm.weight = p[f"{pre}{a}.q_norm.weight"].to(device)
            attn.k_norm.weight = p[f"{pre}{a}.k_norm.weight"].to(device)
        ff = getattr(block, f"{pre}ff")
        ff.project_in.proj = _layer(p, f"{pre}ff.proj_in", device)
        ff.project_out = _layer(p, f"{pre}ff.proj_out", device)
        setattr(block, f"{pre}scale_shift_table", p[f"{pre}scale_shift_table"].to(device))
        setattr(block, f"{pre}prompt_scale_shift_table", p[f"{pre}prompt_scale_shift_table"].to(device))
    for a in ("audio_to_video_attn", "video_to_audio_attn"):
        attn = getattr(block, a)
        for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits"):
            setattr(attn, n, _layer(p, f"{a}.{n}", device))
        attn.q_norm.weight = p[f"{a}.q_norm.weight"].to(device)
        attn.k_norm.weight = p[f"{a}.k_norm.weight"].to(device)
    block.scale_shift_table_a2v_ca_video = p["scale_shift_table_a2v_ca_video"].to(device)
    block.scale_shift_table_a2v_ca_audio = p["scale_shift_table_a2v_ca_audio"].to(device)
    if fuse:
        block.fuse_projections()
    return block


def ltx_model_params(spec: LTXSpec, num_blocks: int, *, in_channels: int = 128, out_channels: int = 128,
                     seed: int = 0) -> dict:
    """Dense bf16 parameters of an LTX video transformer: ``blocks`` (one ``ltx_params`` dict per
    block, without the per-step ``timesteps``), ``patchify_proj``, ``adaln_single`` (9 rows),
    ``prompt_adaln_single`` (2 rows), the output ``scale_shift_table`` ``(2, D)`` and ``proj_out``.
    Weights N(0, 0.02), biases N(0, 0.02), tables N(0, 0.02)."""
    d = spec.dim
    p: dict = {"blocks": []}
    for index in range(num_blocks):
        block = ltx_params(spec, seed * 1000 + index)
        block.pop("timesteps")
        p["blocks"].append(block)

    def lin(name: str, n: int, k: int) -> None:
        p[f"{name}.weight"] = bf16(normal(seed, f"model.{name}.weight", (n, k), 0.02))
        p[f"{name}.bias"] = bf16(normal(seed, f"model.{name}.bias", (n,), 0.02))

    lin("patchify_proj", d, in_channels)
    for prefix, rows in (("adaln_single", 9), ("prompt_adaln_single", 2)):
        lin(f"{prefix}.emb.timestep_embedder.linear_1", d, 256)
        lin(f"{prefix}.emb.timestep_embedder.linear_2", d, d)
        lin(f"{prefix}.linear", rows * d, d)
    p["scale_shift_table"] = bf16(normal(seed, "model.scale_shift_table", (2, d), 0.02))
    lin("proj_out", out_channels, d)
    return p


def ltx_model_inputs(spec: LTXSpec, *, in_channels: int = 128, seed: int = 0) -> dict[str, torch.Tensor]:
    """Latent ``(1, T, C)`` N(0, 1) bf16, context ``(1, Tc, D)`` bf16 and RoPE positions."""
    return {
        "latent": bf16(normal(seed, "latent", (1, spec.tokens, in_channels))),
        "context": bf16(normal(seed, "context", (1, spec.text_tokens, spec.dim))),
        "positions": ltx_positions(spec.grid),
    }


def _assign_adaln(adaln, p: dict, prefix: str, device) -> None:
    embedder = adaln.emb.timestep_embedder
    embedder.linear_1 = _layer(p, f"{prefix}.emb.timestep_embedder.linear_1", device)
    embedder.linear_2 = _layer(p, f"{prefix}.emb.timestep_embedder.linear_2", device)
    adaln.linear = _layer(p, f"{prefix}.linear", device)


def build_ltx_model(spec: LTXSpec, p: dict, device, *, in_channels: int = 128, out_channels: int = 128,
                    fuse: bool = True):
    """The MI355X ``LTXAVModel`` (video stream) holding ``p``'s weights on ``device``."""
    from .ltx2.model import LTXAVModel

    model = LTXAVModel(num_layers=max(1, len(p["blocks"])), video_heads=spec.heads, video_head_dim=spec.head_dim,
                       video_in_channels=in_channels, video_out_channels=out_channels, video_context_dim=spec.dim)
    model.transformer_blocks = [build_ltx_block(spec, block, device, fuse=fuse) for block in p["blocks"]]
    model.patchify_proj = _layer(p, "patchify_proj", device)
    _assign_adaln(model.adaln_single, p, "adaln_single", device)
    _assign_adaln(model.prompt_adaln_single, p, "prompt_adaln_single", device)
    model.scale_shift_table = p["scale_shift_table"].to(device)
    model.proj_out = _layer(p, "proj_out", device)
    return model


def random_ltx_model(spec: LTXSpec, num_blocks: int, device, *, in_channels: int = 128, out_channels: int = 128,
                     seed: int = 0):
    """An ``LTXAVModel`` of ``num_blocks`` blocks with N(0, 0.02) weights drawn directly on
    ``device`` (one seeded device generator; for timing runs, where host-side generation of
    tens of GB of weights would dominate). Every block has its own weights; with ``spec.bits``
    the block linears are quantized on the device into the packed affine layout."""
    gen = torch.Generator(device=device).manual_seed(seed)

    def rnd(shape, std=0.02, mean=0.0):
        return torch.randn(tuple(shape), generator=gen, device=device, dtype=torch.float32) * std + mean

    d, f = spec.dim, spec.dim * spec.ff_mult
    blocks = []
    for _ in range(num_blocks):
        p: dict[str, torch.Tensor] = {}
        for prefix in ("attn1", "attn2"):
            for name in ("to_q", "to_k", "to_v", "to_out"):
                p[f"{prefix}.{name}.weight"] = bf16(rnd((d, d)))
                p[f"{prefix}.{name}.bias"] = bf16(rnd((d,)))
            p[f"{prefix}.to_gate_logits.weight"] = bf16(rnd((spec.heads, d)))
            p[f"{prefix}.to_gate_logits.bias"] = bf16(rnd((spec.heads,)))
            for name in ("q_norm", "k_norm"):
                p[f"{prefix}.{name}.weight"] = bf16(rnd((d,), 0.02, 1.0))
        p["ff.proj_in.weight"], p["ff.proj_in.bias"] = bf16(rnd((f, d))), bf16(rnd((f,)))
        p["ff.proj_out.weight"], p["ff.proj_out.bias"] = bf16(rnd((d, f))), bf16(rnd((d,)))
        p["scale_shift_table"] = rnd((9, d))
        p["prompt_scale_shift_table"] = rnd((2, d))
        if spec.bits:
            p = quantize_ltx_params(p, spec.bits, spec.group_size)
        blocks.append(build_ltx_block(spec, p, device))
        del p
    top: dict[str, torch.Tensor] = {}

    def lin(name: str, n: int, k: int) -> None:
        top[f"{name}.weight"], top[f"{name}.bias"] = bf16(rnd((n, k))), bf16(rnd((n,)))

    lin("patchify_proj", d, in_channels)
    for prefix, rows in (("adaln_single", 9), ("prompt_adaln_single", 2)):
        lin(f"{prefix}.emb.timestep_embedder.linear_1", d, 256)
        lin(f"{prefix}.emb.timestep_embedder.linear_2", d, d)
        lin(f"{prefix}.linear", rows * d, d)
    top["scale_shift_table"] = bf16(rnd((2, d)))
    lin("proj_out", out_channels, d)
    top["blocks"] = []
    model = build_ltx_model(spec, top, device, in_channels=in_channels, out_channels=out_channels)
    model.transformer_blocks = blocks
    return model


_AV_STEP_ROWS = ("timesteps", "audio_timesteps", "cross_ss", "cross_gate", "audio_cross_ss", "audio_cross_gate")


def _av_top_params(p: dict, spec: LTXSpec, audio: LTXAudioSpec, in_channels: int, out_channels: int, lin) -> None:
    for pre, d in (("", spec.dim), ("audio_", audio.dim)):
        lin(f"{pre}patchify_proj", d, in_channels)
        for name, rows in ((f"{pre}adaln_single", 9), (f"{pre}prompt_adaln_single", 2)):
            lin(f"{name}.emb.timestep_embedder.linear_1", d, 256)
            lin(f"{name}.emb.timestep_embedder.linear_2", d, d)
            lin(f"{name}.linear", rows * d, d)
        lin(f"{pre}proj_out", out_channels, d)
    for name, d, rows in (("av_ca_video_scale_shift_adaln_single", spec.dim, 4),
                          ("av_ca_a2v_gate_adaln_single", spec.dim, 1),
                          ("av_ca_audio_scale_shift_adaln_single", audio.dim, 4),
                          ("av_ca_v2a_gate_adaln_single", audio.dim, 1)):
        lin(f"{name}.emb.timestep_embedder.linear_1", d, 256)
        lin(f"{name}.emb.timestep_embedder.linear_2", d, d)
        lin(f"{name}.linear", rows * d, d)


def ltx_av_model_params(spec: LTXSpec, audio: LTXAudioSpec, num_blocks: int, *, in_channels: int = 128,
                        out_channels: int = 128, seed: int = 0) -> dict:
    """Dense bf16 parameters of a joint audio/video LTX transformer: ``blocks`` (``ltx_av_params``
    per block, without the per-step rows), both streams' patchify / AdaLN / prompt / output
    parts, the four A/V AdaLN producers and the two ``(2, D)`` output tables."""
    p: dict = {"blocks": []}
    for index in range(num_blocks):
        block = ltx_av_params(spec, audio, seed * 1000 + index)
        for name in _AV_STEP_ROWS:
            block.pop(name)
        p["blocks"].append(block)

    def lin(name: str, n: int, k: int) -> None:
        p[f"{name}.weight"] = bf16(normal(seed, f"model.{name}.weight", (n, k), 0.02))
        p[f"{name}.bias"] = bf16(normal(seed, f"model.{name}.bias", (n,), 0.02))

    _av_top_params(p, spec, audio, in_channels, out_channels, lin)
    p["scale_shift_table"] = bf16(normal(seed, "model.scale_shift_table", (2, spec.dim), 0.02))
    p["audio_scale_shift_table"] = bf16(normal(seed, "model.audio_scale_shift_table", (2, audio.dim), 0.02))
    return p


def ltx_av_model_inputs(spec: LTXSpec, audio: LTXAudioSpec, *, in_channels: int = 128, seed: int = 0) -> dict:
    """``ltx_model_inputs`` plus the audio latent ``(1, Ta, C)``, audio context and bounds."""
    out = ltx_model_inputs(spec, in_channels=in_channels, seed=seed)
    out["audio_latent"] = bf16(normal(seed, "audio_latent", (1, audio.tokens, in_channels)))
    out["audio_context"] = bf16(normal(seed, "audio_context", (1, audio.text_tokens, audio.dim)))
    start = torch.arange(audio.tokens, dtype=torch.float32)
    out["audio_positions"] = torch.stack([start, start + 1.0], dim=-1)[None, None]
    return out


def build_ltx_av_model(spec: LTXSpec, audio: LTXAudioSpec, p: dict, device, *, in_channels: int = 128,
                       out_channels: int = 128, fuse: bool = True):
    """The MI355X joint ``LTXAVModel`` holding ``p``'s weights on ``device``."""
    from .ltx2.model import LTXAVModel

    model = LTXAVModel(num_layers=max(1, len(p["blocks"])), video_heads=spec.heads, video_head_dim=spec.head_dim,
                       audio_heads=audio.heads, audio_head_dim=audio.head_dim, video_in_channels=in_channels,
                       video_out_channels=out_channels, audio_in_channels=in_channels,
                       audio_out_channels=out_channels, video_context_dim=spec.dim)
    model.transformer_blocks = [build_ltx_av_block(spec, audio, b, device, fuse=fuse) for b in p["blocks"]]
    for pre in ("", "audio_"):
        setattr(model, f"{pre}patchify_proj", _layer(p, f"{pre}patchify_proj", device))
        setattr(model, f"{pre}proj_out", _layer(p, f"{pre}proj_out", device))
        setattr(model, f"{pre}scale_shift_table", p[f"{pre}scale_shift_table"].to(device))
        _assign_adaln(getattr(model, f"{pre}adaln_single"), p, f"{pre}adaln_single", device)
        _assign_adaln(getattr(model, f"{pre}prompt_adaln_single"), p, f"{pre}prompt_adaln_single", device)
    for name in ("av_ca_video_scale_shift_adaln_single", "av_ca_a2v_gate_adaln_single",
                 "av_ca_audio_scale_shift_adaln_single", "av_ca_v2a_gate_adaln_single"):
        _assign_adaln(getattr(model, name), p, name, device)
    return model


def random_ltx_av_model(spec: LTXSpec, audio: LTXAudioSpec, num_blocks: int, device, *, in_channels: int = 128,
                        out_channels: int = 128, seed: int = 0):
    """A joint ``LTXAVModel`` of ``num_blocks`` blocks with every tensor drawn on ``device``
    (N(0, 0.02); norm scales N(1, 0.02)) in the shapes of ``ltx_av_model_params`` (for timing)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    template = ltx_av_params(spec, audio, seed)

    def draw(name: str, like: torch.Tensor) -> torch.Tensor:
        mean = 1.0 if name.endswith("norm.weight") else 0.0
        value = torch.randn(tuple(like.shape), generator=gen, device=device) * 0.02 + mean
        return value.to(like.dtype)

    blocks = []
    for _ in range(num_blocks):
        b = {k: draw(k, v) for k, v in template.items() if k not in _AV_STEP_ROWS}
        blocks.append(build_ltx_av_block(spec, audio, b, device))
        del b
    top: dict = {"blocks": []}

    def lin(name: str, n: int, k: int) -> None:
        top[f"{name}.weight"] = draw(name, torch.empty((n, k), dtype=torch.bfloat16))
        top[f"{name}.bias"] = draw(name, torch.empty((n,), dtype=torch.bfloat16))

    _av_top_params(top, spec, audio, in_channels, out_channels, lin)
    top["scale_shift_table"] = draw("t", torch.empty((2, spec.dim), dtype=torch.bfloat16))
    top["audio_scale_shift_table"] = draw("t", torch.empty((2, audio.dim), dtype=torch.bfloat16))
    model = build_ltx_av_model(spec, audio, top, device, in_channels=in_channels, out_channels=out_channels)
    model.transformer_blocks = blocks
    return model


# ---- FLUX.2 / config 1 ---------------------------------------------------------------------------


def flux_ids(spec: FluxSpec) -> torch.Tensor:
    """``(1, Tt + Ti, 4)`` FLUX.2 ids: text ``(0, 0, 0, l)`` then image ``(0, h, w, 0)``."""
    h, w = spec.grid
    text = torch.zeros(spec.text_tokens, 4)
    text[:, 3] = torch.arange(spec.text_tokens, dtype=torch.float32)
    hh, ww = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
    image = torch.zeros(h * w, 4)
    image[:, 1] = hh.reshape(-1).float()
    image[:, 2] = ww.reshape(-1).float()
    return torch.cat([text, image])[None]


def config1_positions(spec: FluxSpec) -> torch.Tensor:
    """``(1, Tt + Ti, 2)`` (h, w) positions: text at (0, 0), image on its grid."""
    h, w = spec.grid
    hh, ww = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
    image = torch.stack([hh.reshape(-1), ww.reshape(-1)], dim=-1).float()
    return torch.cat([torch.zeros(spec.text_tokens, 2), image])[None]


def axis_rope_tables(positions: torch.Tensor, *, theta: float, axes_dims: tuple[int, ...]):
    """Per-axis adjacent-pair tables ``(B, T, Dh)`` (Krea ``Krea2RotaryEmbedding``,
    ``kinomlx/models/krea2/transformer/model.py:49-66``), computed in float32 on the CPU."""
    parts = []
    for axis, dims in enumerate(axes_dims):
        freqs = 1.0 / (torch.tensor(theta, dtype=torch.float32) ** (torch.arange(0, dims, 2, dtype=torch.float32) / dims))
        angles = positions[..., axis, None].float() * freqs
        parts.append(torch.repeat_interleave(angles, 2, dim=-1))
    combined = torch.cat(parts, dim=-1)
    return torch.cos(combined), torch.sin(combined)


def flux_params(spec: FluxSpec, seed: int = 0) -> dict[str, torch.Tensor]:
    d, dh = spec.dim, spec.head_dim
    p: dict[str, torch.Tensor] = {}
    for name in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out", "to_add_out"):
        p[f"attn.{name}.weight"] = bf16(normal(seed, f"attn.{name}.weight", (d, d), 0.02))
    for name in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        p[f"attn.{name}.weight"] = bf16(normal(seed, f"attn.{name}.weight", (dh,), 0.02, 1.0))
    f = spec.ff_hidden
    for prefix in ("ff", "ff_context"):
        if spec.ff == "swiglu":
            p[f"{prefix}.linear_in.weight"] = bf16(normal(seed, f"{prefix}.linear_in.weight", (2 * f, d), 0.02))
            p[f"{prefix}.linear_out.weight"] = bf16(normal(seed, f"{prefix}.linear_out.weight", (d, f), 0.02))
        else:
            p[f"{prefix}.proj_in.weight"] = bf16(normal(seed, f"{prefix}.proj_in.weight", (f, d), 0.02))
            p[f"{prefix}.proj_in.bias"] = bf16(normal(seed, f"{prefix}.proj_in.bias", (f,), 0.02))
            p[f"{prefix}.proj_out.weight"] = bf16(normal(seed, f"{prefix}.proj_out.weight", (d, f), 0.02))
            p[f"{prefix}.proj_out.bias"] = bf16(normal(seed, f"{prefix}.proj_out.bias", (d,), 0.02))
    cond = normal(seed, "cond", (1, COND_DIM))
    for stream in ("image_mod", "text_mod"):
        w = bf16(normal(seed, f"{stream}.linear.weight", (6 * d, COND_DIM), 0.02)).float()
        p[stream] = bf16((cond @ w.T).reshape(6, d))
    if spec.single:
        p["single.attn.to_qkv_mlp_proj.weight"] = bf16(
            normal(seed, "single.attn.to_qkv_mlp_proj.weight", (3 * d + 2 * f, d), 0.02))
        p["single.attn.to_out.weight"] = bf16(normal(seed, "single.attn.to_out.weight", (d, d + f), 0.02))
        for name in ("norm_q", "norm_k"):
            p[f"single.attn.{name}.weight"] = bf16(normal(seed, f"single.attn.{name}.weight", (dh,), 0.02, 1.0))
        w = bf16(normal(seed, "single_mod.linear.weight", (3 * d, COND_DIM), 0.02)).float()
        p["single_mod"] = bf16((cond @ w.T).reshape(3, d))
    return p


def flux_inputs(spec: FluxSpec, seed: int = 0) -> dict[str, torch.Tensor]:
    return {
        "image": bf16(normal(seed, "image", (1, spec.image_tokens, spec.dim))),
        "text": bf16(normal(seed, "text", (1, spec.text_tokens, spec.dim))),
    }


def flux_rope(spec: FluxSpec) -> tuple[torch.Tensor, torch.Tensor]:
    """``(T, Dh)`` fp32 adjacent-pair tables for the joint [text, image] sequence."""
    if spec.ff == "swiglu":
        ids = flux_ids(spec)
        frequency = 2000.0 ** (-torch.arange(0, 32, 2, dtype=torch.float32) / 32)
        angles = (ids[..., None] * frequency).reshape(*ids.shape[:-1], 64)
        angles = torch.repeat_interleave(angles, 2, dim=-1)
        return torch.cos(angles)[0], torch.sin(angles)[0]
    half = spec.head_dim // 2
    cos, sin = axis_rope_tables(config1_positions(spec), theta=10000.0, axes_dims=(half, half))
    return cos[0], sin[0]


def build_flux_double_block(spec: FluxSpec, p: dict[str, torch.Tensor], device, *, fuse: bool = True):
    """The MI355X FLUX.2 ``DoubleBlock`` holding ``p``'s weights on ``device``. Config 1 (``ff ==
    "gelu"``) takes LTX's GELU ``FeedForward`` (biased ``proj_in``/``proj_out``) per stream."""
    from .flux2.transformer import DoubleBlock
    from .ltx2.feed_forward import FeedForward as GeluFeedForward

    block = DoubleBlock(heads=spec.heads, head_dim=spec.head_dim)
    attn = block.attn
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_add_out"):
        setattr(attn, n, _layer(p, f"attn.{n}", device))
    attn.to_out = [_layer(p, "attn.to_out", device)]
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        getattr(attn, n).weight = p[f"attn.{n}.weight"].to(device)
    for prefix in ("ff", "ff_context"):
        if spec.ff == "swiglu":
            ff = getattr(block, prefix)
            ff.linear_in = _layer(p, f"{prefix}.linear_in", device)
            ff.linear_out = _layer(p, f"{prefix}.linear_out", device)
        else:
            ff = GeluFeedForward(spec.dim, mult=spec.ff_hidden // spec.dim)
            ff.project_in.proj = _layer(p, f"{prefix}.proj_in", device)
            ff.project_out = _layer(p, f"{prefix}.proj_out", device)
            setattr(block, prefix, ff)
    if fuse:
        block.fuse_projections()
    return block


def build_flux_single_block(spec: FluxSpec, p: dict[str, torch.Tensor], device):
    """The MI355X FLUX.2 ``SingleBlock`` holding ``p``'s ``single.*`` weights on ``device``."""
    from .flux2.transformer import SingleBlock

    block = SingleBlock(heads=spec.heads, head_dim=spec.head_dim)
    block.attn.to_qkv_mlp_proj = _layer(p, "single.attn.to_qkv_mlp_proj", device)
    block.attn.to_out = _layer(p, "single.attn.to_out", device)
    block.attn.norm_q.weight = p["single.attn.norm_q.weight"].to(device)
    block.attn.norm_k.weight = p["single.attn.norm_k.weight"].to(device)
    return block


def flux_tables(spec: FluxSpec, device) -> tuple[torch.Tensor, torch.Tensor]:
    """``(1, T, 1, Dh)`` fp32 rotary tables for the joint [text, image] sequence on ``device``."""
    cos, sin = flux_rope(spec)
    return cos[None, :, None].contiguous().to(device), sin[None, :, None].contiguous().to(device)


def flop_count(spec) -> dict[str, float]:
    """Algorithmic work of one block: GEMM ``2MNK``, attention ``4 H Tq Tk Dh``."""
    if isinstance(spec, LTXSpec):
        t, tc, d, h, dh, f = spec.tokens, spec.text_tokens, spec.dim, spec.heads, spec.head_dim, spec.dim * spec.ff_mult
        gemm = 2.0 * t * d * (4 * d + h) + 2.0 * t * d * (2 * d + h) + 2.0 * tc * d * 2 * d + 2.0 * 2 * t * d * f
        attn = 4.0 * h * dh * (t * t + t * tc)
        return {"gemm": gemm, "attention": attn, "total": gemm + attn}
    ti, tt, d, h, dh, f = spec.image_tokens, spec.text_tokens, spec.dim, spec.heads, spec.head_dim, spec.ff_hidden
    ff_in = 2 * f if spec.ff == "swiglu" else f
    gemm = 2.0 * (ti + tt) * d * (4 * d) + 2.0 * (ti + tt) * d * (ff_in + f)
    t = ti + tt
    attn = 4.0 * h * dh * t * t
    if spec.single:
        gemm += 2.0 * t * d * (3 * d + 2 * f) + 2.0 * t * (d + f) * d
        attn *= 2
    return {"gemm": gemm, "attention": attn, "total": gemm + attn}


__all__ = [
    "CONFIGS",
    "FluxSpec",
    "LTXSpec",
    "build_flux_double_block",
    "build_flux_single_block",
    "LTXAudioSpec",
    "build_ltx_av_block",
    "build_ltx_av_model",
    "build_ltx_block",
    "build_ltx_model",
    "flux_tables",
    "flop_count",
    "flux_inputs",
    "flux_params",
    "flux_rope",
    "ltx_av_inputs",
    "ltx_av_model_inputs",
    "ltx_av_model_params",
    "ltx_av_params",
    "ltx_inputs",
    "ltx_model_inputs",
    "ltx_model_params",
    "ltx_params",
    "ltx_positions",
    "normal",
    "quantize_ltx_params",
    "random_ltx_av_model",
    "random_ltx_model",
]
