"""LTX-2 transformer checkpoints on MI355X: source-key conversion, loading into HBM, prepared
(``__quant__.`` / ``__layout__.``) tensors and quantize-on-load.

Mirror of ``convert_checkpoint_key`` and its tables (``kinomlx/models/ltx2/transformer/graph.py:
84-115,322-359``), of the quantize step of the weight preparation (``kinomlx/models/ltx2/
preparation.py:139-157``: ``mx.quantize(w or w.T, group_size, bits, mode)`` on the block linears
that ``quant_mode_for_key`` routes, ``kinomlx/models/ltx2/weights/tensors.py:256-283``), and of the
binding of prepared checkpoints (``kinomlx/models/ltx2/weights/loading.py:82-110``: keys under
``__quant__.`` are packed linears whose mode comes from the settings, ``quantization.py:199-274``;
keys under ``__layout__.`` are ``weight_t``, the transposed dense weight). The tensors move from the
file to HBM through ``kinomlx_amd.io.load_to_device``; on-load quantization runs the
``kx_quantize_affine_bf16`` / ``kx_quantize_mxfp8_bf16`` / ``kx_quantize_fp4_bf16`` (mxfp4 and nvfp4
feed-forward layers, ``video_ff_quantize_specs``) kernels on the resident bf16 weight.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import Path

import torch

from ..io.safetensors import inspect_safetensors, load_to_device
from ..kernels.quantized import PretransposedQuantizedLinear, QuantizedLinear, quant_defaults, quantize
from .attention import Linear
from .model import LTXAVModel

QUANT_KEY_PREFIX = "__quant__."
LAYOUT_KEY_PREFIX = "__layout__."
# TransformerQuantize (kinomlx/models/ltx2/weights/schema.py:13-21)
TRANSFORMER_QUANTIZE_MODES = ("off", "mxfp8-blocks", "mxfp8-blocks-pretranspose")
DIFFUSION_PREFIX = "model.diffusion_model."
_DIFFUSION_PREFIXES = (DIFFUSION_PREFIX, "diffusion_model.", "")
_TRANSFORMER_ROOTS = (
    "adaln_single.",
    "audio_adaln_single.",
    "audio_patchify_proj.",
    "audio_proj_out.",
    "audio_prompt_adaln_single.",
    "audio_scale_shift_table",
    "av_ca_a2v_gate_adaln_single.",
    "av_ca_audio_scale_shift_adaln_single.",
    "av_ca_v2a_gate_adaln_single.",
    "av_ca_video_scale_shift_adaln_single.",
    "keyframes_abs_pos_embedding",
    "norm_out.",
    "audio_norm_out.",
    "patchify_proj.",
    "proj_out.",
    "prompt_adaln_single.",
    "scale_shift_table",
    "transformer_blocks.",
)
_VIDEO_ONLY_SKIP_FRAGMENTS = ("av_ca", "a2v", "audio")
_REPLACEMENTS = (
    (re.compile(r"\.to_out\.0\."), ".to_out."),
    (re.compile(r"(^|\.)ff\.net\.0\.proj\."), r"\1ff.project_in.proj."),
    (re.compile(r"(^|\.)ff\.net\.2\."), r"\1ff.project_out."),
    (re.compile(r"(^|\.)audio_ff\.net\.0\.proj\."), r"\1audio_ff.project_in.proj."),
    (re.compile(r"(^|\.)audio_ff\.net\.2\."), r"\1audio_ff.project_out."),
)

# the block linears the reference quantizes (attention projections and the feed-forward)
QUANTIZED_LINEARS = tuple(
    f"{a}.{n}" for a in ("attn1", "attn2") for n in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits")
) + ("ff.project_in.proj", "ff.project_out")


@dataclass(frozen=True)
class ConvertedTransformerKey:
    """One normalized source key and its alias priority (lower wins)."""

    target_key: str
    priority: int


def _strip_source_wrapper(key: str) -> tuple[str, int] | None:
    for priority, prefix in enumerate(_DIFFUSION_PREFIXES[:-1]):
        if key.startswith(prefix):
            return key[len(prefix):], priority
    for offset, prefix in enumerate(_DIFFUSION_PREFIXES[:-1], start=3):
        position = key.find("." + prefix)
        if position >= 0:
            return key[position + 1 + len(prefix):], offset
    if key.startswith(_TRANSFORMER_ROOTS):
        return key, 2
    for root in _TRANSFORMER_ROOTS:
        position = key.find("." + root)
        if position >= 0:
            return key[position + 1:], 6
    return None


def convert_checkpoint_key(checkpoint_key: str, *, include_audio: bool = False) -> ConvertedTransformerKey | None:
    """Source key -> model key, or None for keys outside the (video) transformer
    (``graph.py:341-359``)."""
    stripped = _strip_source_wrapper(checkpoint_key)
    if stripped is None:
        return None
    logical, priority = stripped
    if "embeddings_connector." in logical:
        return None
    if not include_audio and any(fragment in logical.lower() for fragment in _VIDEO_ONLY_SKIP_FRAGMENTS):
        return None
    for pattern, replacement in _REPLACEMENTS:
        logical = pattern.sub(replacement, logical)
    return ConvertedTransformerKey(logical, priority)


def checkpoint_bindings(path: Path | str) -> dict[str, str]:
    """Model key -> source key for every transformer tensor of the file; where several source
    keys alias one model key, the lowest priority wins (ties are an error). Prepared tensors keep
    their prefix: ``__quant__.<key>`` and ``__layout__.<key>`` (``loading.py:89-100``)."""
    chosen: dict[str, tuple[int, str]] = {}
    for name in inspect_safetensors(path).tensor_names:
        if name.startswith((QUANT_KEY_PREFIX, LAYOUT_KEY_PREFIX)):
            if name in chosen:
                raise ValueError(f"{path}: duplicate prepared tensor {name!r}")
            chosen[name] = (-1, name)
            continue
        converted = convert_checkpoint_key(name)
        if converted is None:
            continue
        previous = chosen.get(converted.target_key)
        if previous is not None and previous[0] == converted.priority:
            raise ValueError(f"{path}: {previous[1]!r} and {name!r} both map to {converted.target_key!r}")
        if previous is None or converted.priority < previous[0]:
            chosen[converted.target_key] = (converted.priority, name)
    return {target: source for target, (_, source) in chosen.items()}


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


def _words(t: torch.Tensor) -> torch.Tensor:
    """Packed uint32 words as the int32 tensor the quantized kernels take (same bits)."""
    return t.view(torch.int32) if t.dtype == torch.uint32 else t


def quant_pretransposed(transformer_quantize: str) -> bool:
    """``tensors.py:279-280``."""
    return transformer_quantize == "mxfp8-blocks-pretranspose"


def quant_mode_for_base(base: str, *, transformer_quantize: str = "off",
                        video_ff_quantize_specs: tuple[tuple[str, str], ...] = ()) -> str | None:
    """The quantization mode of a block linear (``quantization.py:199-218``): mxfp8 for every
    block linear under an mxfp8 ``transformer_quantize``, else the feed-forward spec's mode."""
    if transformer_quantize not in TRANSFORMER_QUANTIZE_MODES:
        raise ValueError(f"Unsupported transformer weight quantization mode: {transformer_quantize}")
    if transformer_quantize != "off" and base in QUANTIZED_LINEARS:
        return "mxfp8"
    targets = {"ff.project_in.proj": "project_in", "ff.project_out": "project_out"}
    if base in targets:
        for target, mode in video_ff_quantize_specs:
            if target == targets[base]:
                return mode
    return None


def load_transformer(path: Path | str, device, *, heads: int = 32, head_dim: int = 128,
                     quantize_bits: int | None = None, group_size: int = 64, transformer_quantize: str = "off",
                     transformer_quantize_exclude_layers: tuple[int, ...] = (),
                     video_ff_quantize_specs: tuple[tuple[str, str], ...] = (),
                     video_ff_quantize_layers: tuple[int, ...] = (),
                     video_ff_quantize_group_size: int | None = None, video_ff_quantize_bits: int | None = None,
                     fuse: bool = True, strict: bool = True) -> LTXAVModel:
    """Build the video ``LTXAVModel`` from a safetensors checkpoint with its tensors in HBM.

    Linear weights and biases are held in bf16 and the modulation tables in fp32. A block linear
    takes, in this order: its prepared packed tensors (``__quant__.<base>.weight`` / ``.scales``
    / ``.biases``, mode from ``quant_mode_for_base`` and ``quant_defaults``; the
    ``mxfp8-blocks-pretranspose`` packing is of ``weight.T``); its prepared ``__layout__.<base>.
    weight_t``; or its dense weight, quantized on the device when the settings route it
    (``transformer_quantize`` for every block linear, ``video_ff_quantize_specs`` for the
    feed-forward targets of ``video_ff_quantize_layers`` (all when empty), layers in
    ``transformer_quantize_exclude_layers`` never), or with ``quantize_bits`` (4 or 8) into the
    group-``group_size`` affine format. With ``strict``, a transformer tensor the model has no
    place for is an error."""
    if transformer_quantize not in TRANSFORMER_QUANTIZE_MODES:
        raise ValueError(f"Unsupported transformer weight quantization mode: {transformer_quantize}")
    bindings = checkpoint_bindings(path)
    tensors = load_to_device(path, device, names=bindings.values())
    params = {target: tensors.pop(source) for target, source in bindings.items()}
    used: set[str] = set()
    pretransposed = quant_pretransposed(transformer_quantize)

    def take(key: str) -> torch.Tensor:
        if key not in params:
            raise KeyError(f"{path}: checkpoint has no tensor for {key!r}")
        used.add(key)
        return params[key]

    def routed_mode(layer: int, base: str) -> str | None:
        if layer in transformer_quantize_exclude_layers:
            return None
        if transformer_quantize != "off" and base in QUANTIZED_LINEARS:
            return "mxfp8"
        if video_ff_quantize_layers and layer not in video_ff_quantize_layers:
            return None
        return quant_mode_for_base(base, video_ff_quantize_specs=video_ff_quantize_specs)

    def linear(prefix: str, layer: int | None = None, base: str | None = None):
        bias = _bf16(take(f"{prefix}.bias")) if f"{prefix}.bias" in params else None
        quant = f"{QUANT_KEY_PREFIX}{prefix}"
        if f"{quant}.weight" in params or f"{quant}.scales" in params:
            if base is None:
                raise ValueError(f"{path}: unexpected non-block quantized weight key: {quant}.weight")
            mode = quant_mode_for_base(base, transformer_quantize=transformer_quantize,
                                       video_ff_quantize_specs=video_ff_quantize_specs)
            if mode is None:
                raise ValueError(f"Missing quantization mode for transformer target: {base}")
            missing = sorted({"weight", "scales"} - {p for p in ("weight", "scales") if f"{quant}.{p}" in params})
            if missing:
                raise ValueError(f"Incomplete quantized weight target {base}: missing {', '.join(missing)}")
            gs, bits = quant_defaults(mode, video_ff_quantize_group_size, video_ff_quantize_bits)
            words, scales = _words(take(f"{quant}.weight")), take(f"{quant}.scales")
            biases = take(f"{quant}.biases") if f"{quant}.biases" in params else None
            if pretransposed and mode == "mxfp8":
                return PretransposedQuantizedLinear(words, scales, bias, group_size=gs, bits=bits, mode=mode)
            if mode == "affine":  # the affine kernels read bf16 scales and biases
                scales = _bf16(scales)
            return QuantizedLinear(words, scales, None if biases is None else _bf16(biases), bias, group_size=gs,
                                   bits=bits, mode=mode)
        layout = f"{LAYOUT_KEY_PREFIX}{prefix}.weight_t"
        if layout in params:
            return Linear(_bf16(take(layout)).t().contiguous(), bias)
        weight = _bf16(take(f"{prefix}.weight"))
        mode = routed_mode(layer, base) if base is not None else None
        if mode is not None:
            gs, bits = quant_defaults(mode, video_ff_quantize_group_size, video_ff_quantize_bits)
            params[f"{prefix}.weight"] = None
            if pretransposed and mode == "mxfp8":
                return PretransposedQuantizedLinear.from_linear(weight, bias)
            return QuantizedLinear.from_linear(weight, bias, group_size=gs, bits=bits, mode=mode)
        if base is not None and quantize_bits:
            words, scales, biases = quantize(weight, group_size, quantize_bits)
            params[f"{prefix}.weight"] = None
            return QuantizedLinear(words, scales, biases, bias, group_size=group_size, bits=quantize_bits)
        return Linear(weight, bias)

    def block_index(key: str) -> int | None:
        for prefix in (QUANT_KEY_PREFIX, LAYOUT_KEY_PREFIX, ""):
            if key.startswith(prefix + "transformer_blocks."):
                return int(key[len(prefix):].split(".")[1])
        return None

    layers = sorted({i for i in map(block_index, params) if i is not None})
    if layers != list(range(len(layers))) or not layers:
        raise ValueError(f"{path}: transformer blocks must be numbered 0..n-1, found {layers[:8]}...")
    patchify = take("patchify_proj.weight")
    proj_out = take("proj_out.weight")
    dim = int(patchify.shape[0])
    if dim != heads * head_dim:
        raise ValueError(f"{path}: hidden size {dim} does not match {heads} heads x {head_dim}")
    # a linear's weight may be stored plain, pretransposed (``__layout__.<name>.weight_t``, which
    # the reference's preparation writes for every top-level AdaLN linear, layout.py:11-20) or
    # packed (``__quant__.<name>.weight``)
    def has_linear(prefix: str) -> bool:
        return any(key in params for key in (f"{prefix}.weight", f"{LAYOUT_KEY_PREFIX}{prefix}.weight_t",
                                             f"{QUANT_KEY_PREFIX}{prefix}.weight"))

    model = LTXAVModel(num_layers=len(layers), video_heads=heads, video_head_dim=head_dim,
                       video_in_channels=int(patchify.shape[1]), video_out_channels=int(proj_out.shape[0]),
                       video_context_dim=dim, use_prompt_adaln_single=has_linear("prompt_adaln_single.linear"))
    model.patchify_proj = linear("patchify_proj")
    model.proj_out = linear("proj_out")
    model.scale_shift_table = take("scale_shift_table")
    adalns = [("adaln_single", model.adaln_single)]
    if model.prompt_adaln_single is not None:
        adalns.append(("prompt_adaln_single", model.prompt_adaln_single))
    for prefix, adaln in adalns:
        embedder = adaln.emb.timestep_embedder
        embedder.linear_1 = linear(f"{prefix}.emb.timestep_embedder.linear_1")
        embedder.linear_2 = linear(f"{prefix}.emb.timestep_embedder.linear_2")
        adaln.linear = linear(f"{prefix}.linear")
    for index, block in zip(layers, model.transformer_blocks):
        prefix = f"transformer_blocks.{index}"
        for name in ("attn1", "attn2"):
            attn = getattr(block, name)
            for proj in ("to_q", "to_k", "to_v", "to_out", "to_gate_logits"):
                setattr(attn, proj, linear(f"{prefix}.{name}.{proj}", index, f"{name}.{proj}"))
            attn.q_norm.weight = take(f"{prefix}.{name}.q_norm.weight")
            attn.k_norm.weight = take(f"{prefix}.{name}.k_norm.weight")
        block.ff.project_in.proj = linear(f"{prefix}.ff.project_in.proj", index, "ff.project_in.proj")
        block.ff.project_out = linear(f"{prefix}.ff.project_out", index, "ff.project_out")
        block.scale_shift_table = take(f"{prefix}.scale_shift_table").float()
        block.prompt_scale_shift_table = take(f"{prefix}.prompt_scale_shift_table").float()
        if fuse:
            block.fuse_projections()
    unused = sorted(set(params) - used)
    if strict and unused:
        raise ValueError(f"{path}: transformer tensors with no place in the video model: {unused[:6]}")
    return model


__all__ = [
    "DIFFUSION_PREFIX",
    "LAYOUT_KEY_PREFIX",
    "QUANT_KEY_PREFIX",
    "TRANSFORMER_QUANTIZE_MODES",
    "quant_mode_for_base",
    "quant_pretransposed",
    "QUANTIZED_LINEARS",
    "ConvertedTransformerKey",
    "checkpoint_bindings",
    "convert_checkpoint_key",
    "load_transformer",
]
