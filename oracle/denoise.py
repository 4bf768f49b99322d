"""CPU restatement of the steps either side of the LTX-2 blocks (test infrastructure only):
timestep features and the AdaLN modulation producers, RoPE table angles, the output head, the
X0 conversion, the conditioning composite, the Euler updates and the finite check.

Each function names the reference file:line whose MLX arithmetic it restates. Arrays are numpy
float32; bfloat16 data is carried as float32 values that bf16 represents exactly, and every
``astype(bfloat16)`` of the reference is a ``to_bf16`` here.
"""

from __future__ import annotations

import math

import numpy as np

from .blocks import ltx_av_block, ltx_video_block
from .ops import F32, layer_norm, linear, silu, to_bf16

__all__ = [
    "adaln_single",
    "all_finite",
    "euler_step",
    "euler_velocity_step",
    "ltx_av_forward",
    "ltx_forward",
    "output_head",
    "post_process_latent",
    "timestep_embedding",
    "timestep_mlp",
    "to_denoised",
]


def _f32(value) -> np.ndarray:
    return np.asarray(value, dtype=F32)


def timestep_embedding(timesteps, embedding_dim: int = 256, *, max_period: int = 10000,
                       time_scale: float = 1.0) -> np.ndarray:
    """``get_timestep_embedding`` (``kinomlx/models/ltx2/transformer/timestep.py:13-28``):
    exponent ``(-ln(max_period) * j) / half`` in FP32, angles ``t * exp(exponent)``, cosines
    then sines, a zero column for odd widths. ``time_scale`` is the preprocessor's FP32
    ``value * timestep_scale`` (``preprocessing.py:66-75``)."""
    t = _f32(timesteps)
    if t.ndim != 1:
        raise ValueError("timesteps must be a one-dimensional array")
    t = (t * F32(time_scale)).astype(F32)
    half = embedding_dim // 2
    exponent = (F32(-math.log(max_period)) * np.arange(half, dtype=F32)).astype(F32) / F32(half)
    angles = (t[:, None] * np.exp(exponent.astype(F32))[None, :]).astype(F32)
    out = np.concatenate([np.cos(angles), np.sin(angles)], axis=-1).astype(F32)
    if embedding_dim % 2:
        out = np.pad(out, [(0, 0), (0, 1)])
    return out


def _lin(params: dict, name: str, value, store) -> np.ndarray:
    return store(linear(value, params[f"{name}.weight"], params.get(f"{name}.bias")))


def timestep_mlp(params: dict, prefix: str, timesteps, *, time_scale: float = 1.0,
                 bf16_graph: bool = False) -> np.ndarray:
    """``TimestepEmbedding.__call__`` (``timestep.py:40-49``): features cast to the hidden
    dtype (bf16), ``linear_2(silu(linear_1(x)))``. ``bf16_graph`` also rounds the first
    linear's output before the SiLU, as the reference's graph stores it."""
    store = to_bf16 if bf16_graph else (lambda v: v)
    value = to_bf16(timestep_embedding(timesteps, time_scale=time_scale))
    hidden = store(silu(store(_lin(params, f"{prefix}.linear_1", value, lambda v: v))))
    return store(_lin(params, f"{prefix}.linear_2", hidden, lambda v: v))


def adaln_single(params: dict, prefix: str, timesteps, *, time_scale: float = 1.0,
                 bf16_graph: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """``AdaLayerNormSingle.__call__`` (``timestep.py:74-85``): ``(linear(silu(embedded)),
    embedded)`` with the MLP under ``{prefix}.emb.timestep_embedder``."""
    store = to_bf16 if bf16_graph else (lambda v: v)
    embedded = timestep_mlp(params, f"{prefix}.emb.timestep_embedder", timesteps, time_scale=time_scale,
                            bf16_graph=bf16_graph)
    modulation = store(_lin(params, f"{prefix}.linear", store(silu(embedded)), lambda v: v))
    return modulation, embedded


def output_head(params: dict, value, embedded_timestep, *, eps: float = 1e-6,
                bf16_graph: bool = False) -> np.ndarray:
    """``LTXAVModel._output`` (``kinomlx/models/ltx2/transformer/model.py:577-593``):
    ``(table + embedded)`` cast to bf16 as ``(shift, scale)``, then
    ``proj_out(layer_norm(x) * (1 + scale) + shift)``. ``value (B, T, D)``, embedded
    ``(B, 1 | T, D)``."""
    store = to_bf16 if bf16_graph else (lambda v: v)
    table = _f32(params["scale_shift_table"])
    modulation = to_bf16(table[None, None] + _f32(embedded_timestep)[:, :, None, :])
    shift, scale = modulation[:, :, 0], modulation[:, :, 1]
    x = _f32(value)
    if bf16_graph:
        normalized = store(store(store(layer_norm(x, eps)) * store(F32(1.0) + scale)) + shift)
    else:
        normalized = (layer_norm(x, eps) * (F32(1.0) + scale) + shift).astype(F32)
    return store(linear(normalized, params["proj_out.weight"], params.get("proj_out.bias")))


def ltx_forward(params: dict, latent, context, timesteps, sigma, pe, *, heads: int, num_blocks: int,
                timestep_scale: float = 1000.0, eps: float = 1e-6, bf16_graph: bool = False) -> np.ndarray:
    """Video path of ``LTXAVModel.__call__`` (``model.py:595-635``) for batch 1: ``patchify_proj``,
    the AdaLN rows from ``adaln_single`` (timesteps ``(1,)``) and ``prompt_adaln_single``
    (sigma), ``num_blocks`` blocks whose parameters are ``params["blocks"][i]``
    (``ltx_video_block``), then ``output_head``. ``pe`` is the ``(cos, sin)`` head-major pair.
    Returns the ``(T, C)`` velocity."""
    store = to_bf16 if bf16_graph else (lambda v: v)
    hidden = store(linear(latent, params["patchify_proj.weight"], params["patchify_proj.bias"]))
    modulation, embedded = adaln_single(params, "adaln_single", timesteps, time_scale=timestep_scale,
                                        bf16_graph=bf16_graph)
    prompt, _ = adaln_single(params, "prompt_adaln_single", sigma, time_scale=timestep_scale,
                             bf16_graph=bf16_graph)
    d = hidden.shape[-1]
    modulation = to_bf16(modulation).reshape(9, d)
    prompt = to_bf16(prompt).reshape(2, d)
    x = to_bf16(hidden)
    for block in params["blocks"][:num_blocks]:
        p = dict(block)
        p["ada"] = _f32(block["scale_shift_table"]) + modulation
        p["prompt"] = _f32(block["prompt_scale_shift_table"]) + prompt
        x = to_bf16(ltx_video_block(p, x, context, pe, heads=heads, eps=eps, bf16_graph=bf16_graph))
    return output_head(params, x[None], to_bf16(embedded).reshape(1, 1, d), eps=eps, bf16_graph=bf16_graph)[0]


def ltx_av_forward(params: dict, latent, audio_latent, context, audio_context, timesteps, audio_timesteps, sigma,
                   audio_sigma, pes, *, heads: int, audio_heads: int, num_blocks: int, timestep_scale: float = 1000.0,
                   av_gate_scale: float = 1000.0, eps: float = 1e-6, bf16_graph: bool = False):
    """Joint audio/video ``LTXAVModel.__call__`` for batch 1 (``model.py:595-635``) with both
    streams' preprocessing (``preprocessing.py:134-214``): patchify, the AdaLN / prompt rows, the
    A/V scale-shift rows from each stream's own timesteps and the A/V gate rows from the other
    stream's sigma times ``av_gate_scale``; ``ltx_av_block`` per block; both output heads.
    ``pes`` = (video, audio, video cross, audio cross) tables. Returns the two ``(T, C)``
    velocities."""
    store = to_bf16 if bf16_graph else (lambda v: v)
    bf = to_bf16
    v = bf(store(linear(latent, params["patchify_proj.weight"], params["patchify_proj.bias"])))
    a = bf(store(linear(audio_latent, params["audio_patchify_proj.weight"], params["audio_patchify_proj.bias"])))
    dv, da = v.shape[-1], a.shape[-1]

    def rows(prefix, t, scale, n, d):
        mod, emb = adaln_single(params, prefix, t, time_scale=scale, bf16_graph=bf16_graph)
        return bf(mod).reshape(n, d), bf(emb).reshape(d)

    mod_v, emb_v = rows("adaln_single", timesteps, timestep_scale, 9, dv)
    prompt_v, _ = rows("prompt_adaln_single", sigma, timestep_scale, 2, dv)
    mod_a, emb_a = rows("audio_adaln_single", audio_timesteps, timestep_scale, 9, da)
    prompt_a, _ = rows("audio_prompt_adaln_single", audio_sigma, timestep_scale, 2, da)
    ss_v, _ = rows("av_ca_video_scale_shift_adaln_single", timesteps, timestep_scale, 4, dv)
    gate_v, _ = rows("av_ca_a2v_gate_adaln_single", audio_sigma, av_gate_scale, 1, dv)
    ss_a, _ = rows("av_ca_audio_scale_shift_adaln_single", audio_timesteps, timestep_scale, 4, da)
    gate_a, _ = rows("av_ca_v2a_gate_adaln_single", sigma, av_gate_scale, 1, da)
    for block in params["blocks"][:num_blocks]:
        p = {k: val for k, val in block.items() if "scale_shift_table" not in k}
        p["ada"] = _f32(block["scale_shift_table"]) + mod_v
        p["prompt"] = _f32(block["prompt_scale_shift_table"]) + prompt_v
        p["audio_ada"] = _f32(block["audio_scale_shift_table"]) + mod_a
        p["audio_prompt"] = _f32(block["audio_prompt_scale_shift_table"]) + prompt_a
        tv, ta = _f32(block["scale_shift_table_a2v_ca_video"]), _f32(block["scale_shift_table_a2v_ca_audio"])
        p["av_video"] = np.concatenate([tv[:4] + ss_v, tv[4:5] + gate_v])
        p["av_audio"] = np.concatenate([ta[:4] + ss_a, ta[4:5] + gate_a])
        v, a = ltx_av_block(p, v, a, context, audio_context, *pes, heads=heads, audio_heads=audio_heads, eps=eps,
                            bf16_graph=bf16_graph)
        v, a = bf(v), bf(a)
    head_v = {"scale_shift_table": params["scale_shift_table"], "proj_out.weight": params["proj_out.weight"],
              "proj_out.bias": params["proj_out.bias"]}
    head_a = {"scale_shift_table": params["audio_scale_shift_table"],
              "proj_out.weight": params["audio_proj_out.weight"], "proj_out.bias": params["audio_proj_out.bias"]}
    return (output_head(head_v, v[None], emb_v.reshape(1, 1, dv), eps=eps, bf16_graph=bf16_graph)[0],
            output_head(head_a, a[None], emb_a.reshape(1, 1, da), eps=eps, bf16_graph=bf16_graph)[0])


def to_denoised(latent, velocity, timesteps) -> np.ndarray:
    """``_to_denoised`` (``kinomlx/models/ltx2/transformer/wrappers.py:48-66``):
    ``latent - t * velocity`` in FP32 with ``(B,)`` timesteps over ``(B, 1, 1)`` and ``(B, T)``
    over ``(B, T, 1)``; FP32 result (the caller rounds to the latent dtype)."""
    t = _f32(timesteps)
    if t.ndim == 1:
        t = t[:, None, None]
    elif t.ndim == 2:
        t = t[..., None]
    else:
        raise ValueError("modality timesteps must have shape (B,) or (B, T)")
    return (_f32(latent) - (t * _f32(velocity)).astype(F32)).astype(F32)


def post_process_latent(denoised, clean, mask) -> np.ndarray:
    """Conditioning composite (``kinomlx/models/ltx2/state.py:70-83``):
    ``denoised * m + clean * (1 - m)`` in FP32, ``mask (B, T)`` over the channels; FP32 result."""
    m = _f32(mask)[..., None]
    keep = (_f32(denoised) * m).astype(F32)
    cond = (_f32(clean) * (F32(1.0) - m)).astype(F32)
    return (keep + cond).astype(F32)


def euler_velocity_step(sample, velocity, sigma: float, sigma_next: float, *, bf16: bool) -> np.ndarray:
    """``euler_velocity_step`` (``kinomlx/samplers/steps.py:8-32``): ``delta`` = FP32 of the
    host difference, the scaled velocity rounded to the sample dtype, then the add in that
    dtype (``bf16`` selects bfloat16 storage, else float32)."""
    round_to = to_bf16 if bf16 else (lambda v: _f32(v))
    delta = F32(sigma_next - sigma)
    scaled = round_to((delta * _f32(velocity)).astype(F32))
    return round_to((_f32(sample) + scaled).astype(F32))


def euler_step(sample, denoised, sigma: float, sigma_next: float) -> np.ndarray:
    """``euler_step`` (``kinomlx/samplers/steps.py:35-72``):
    ``denoised + float32(sigma_next / sigma) * (sample - denoised)`` in FP32; FP32 result (the
    caller rounds to the sample dtype)."""
    if not math.isfinite(sigma) or sigma <= 0.0:
        raise ValueError(f"current sigma must be positive and finite, got {sigma!r}")
    s, d = _f32(sample), _f32(denoised)
    step = (F32(sigma_next / sigma) * (s - d).astype(F32)).astype(F32)
    return (d + step).astype(F32)


def all_finite(value) -> bool:
    """``mx.all(mx.isfinite(value))`` (``kinomlx/models/ltx2/denoise.py:244-258``)."""
    return bool(np.all(np.isfinite(_f32(value))))
