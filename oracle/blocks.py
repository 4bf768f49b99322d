"""Block-level CPU restatements (test infrastructure only): the LTX-2 video block, the FLUX.2
double/single blocks and this build's config-1 double-stream block, all in FP32.

Parameters are dicts of float32 numpy arrays whose values bf16 represents exactly (the same
values the GPU path receives as bf16). Batch is 1 and tokens are the leading axis.
"""

from __future__ import annotations

import numpy as np

from .ops import (
    F32,
    adaln,
    attention,
    gate,
    gated_residual,
    gelu_approx,
    layer_norm,
    linear,
    modulate,
    normalized,
    pair_rope,
    quantized_linear,
    rms_norm,
    silu,
    split_rope,
    swiglu,
    to_bf16,
)

__all__ = [
    "KX_SITES",
    "config1_double_block",
    "flux_double_block",
    "flux_single_block",
    "krea_attention",
    "krea_block",
    "ltx_attention",
    "ltx_feed_forward",
    "ltx_av_block",
    "ltx_video_block",
    "rounding",
    "sigmoid",
]


def sigmoid(value) -> np.ndarray:
    x = np.asarray(value, dtype=F32)
    with np.errstate(over="ignore"):
        return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)


def _lin(params: dict, name: str, value: np.ndarray) -> np.ndarray:
    """One linear layer, dense or affine-quantized, by the parameter names present."""
    bias = params.get(f"{name}.bias")
    if f"{name}.wq" in params:
        return quantized_linear(
            value,
            params[f"{name}.wq"],
            params[f"{name}.scales"],
            params[f"{name}.biases"],
            bias,
            group_size=int(params[f"{name}.group_size"]),
            bits=int(params[f"{name}.bits"]),
        )
    return linear(value, params[f"{name}.weight"], bias)


def _keep(value: np.ndarray, site: str = "graph") -> np.ndarray:
    return value


# Rounding sites of a bf16 execution: where an array is stored in the activation dtype. The
# reference's MLX graph stores every intermediate (``bf16_graph``). This build's MI355X path
# stores only the operands its kernels read in bf16 (``KX_SITES``): the modulated norm output, each
# projection that feeds another kernel, the 2*sigmoid head gate, Q/K after their norm (and RoPE) in
# one rounding, the (gated) attention output, the modulated text context and the GELU / SwiGLU
# output; the output projections write the residual stream in FP32 through their epilogues.
KX_SITES = frozenset({"norm", "proj", "gate", "qk", "attn_gated", "ctx", "act"})


def rounding(mode) -> callable:
    """``store(value, site)`` for a rounding mode: ``None``/``False`` (FP32 evaluation),
    ``True``/``"graph"`` (the reference's bf16 graph: every site), ``"kx"`` (``KX_SITES``) or an
    explicit set of site names."""
    if not mode:
        return _keep
    if mode is True or mode == "graph":
        return lambda value, site="graph": to_bf16(value)
    sites = KX_SITES if mode == "kx" else mode
    if isinstance(sites, (set, frozenset)):
        return lambda value, site="graph": to_bf16(value) if site in sites else value
    raise ValueError(f"unknown rounding mode {mode!r}")


def ltx_attention(params: dict, prefix: str, value, *, heads: int, context=None, pe=None, k_pe=None, eps=1e-6,
                  store=_keep):
    """LTX ``Attention.__call__`` without mask or sparse routing
    (``kinomlx/models/ltx2/transformer/attention.py:291-371``): gate logits ``2*sigmoid``,
    full-width weighted RMSNorm on Q and K, split RoPE, SDPA, per-head gate, output projection.
    ``store`` is applied to every array the reference materialises (see ``ltx_video_block``).
    ``k_pe`` rotates the keys with their own tables (the A/V cross-attention, ``:342-344``)."""
    x = np.asarray(value, dtype=F32)
    source = x if context is None else np.asarray(context, dtype=F32)
    head_gate = None
    if f"{prefix}.to_gate_logits.weight" in params or f"{prefix}.to_gate_logits.wq" in params:
        logits = store(_lin(params, f"{prefix}.to_gate_logits", x), "gate_logits")
        head_gate = store(F32(2.0) * store(sigmoid(logits), "gate_sigmoid"), "gate")
    v = store(_lin(params, f"{prefix}.to_v", source), "proj")
    q = store(rms_norm(store(_lin(params, f"{prefix}.to_q", x), "proj"), params[f"{prefix}.q_norm.weight"], eps),
              "qk_norm")
    k = store(rms_norm(store(_lin(params, f"{prefix}.to_k", source), "proj"), params[f"{prefix}.k_norm.weight"],
                       eps), "qk_norm")
    if pe is not None:
        cos, sin = pe
        q = split_rope(q[None], cos, sin)[0]
        k_cos, k_sin = pe if k_pe is None else k_pe
        k = split_rope(k[None], k_cos, k_sin)[0]
    q, k = store(q, "qk"), store(k, "qk")
    out = store(attention(q, k, v, heads=heads), "attn")
    if head_gate is not None:
        tokens, width = out.shape
        out = (out.reshape(tokens, heads, width // heads) * head_gate[:, :, None]).reshape(tokens, width)
    return store(_lin(params, f"{prefix}.to_out", store(out, "attn_gated")), "out_proj")


def ltx_feed_forward(params: dict, prefix: str, value, store=_keep) -> np.ndarray:
    """``project_out(gelu_approx(project_in(x)))``
    (``kinomlx/models/ltx2/transformer/feed_forward.py:80-97``)."""
    hidden = store(gelu_approx(store(_lin(params, f"{prefix}.proj_in", value), "ff_in")), "act")
    return store(_lin(params, f"{prefix}.proj_out", hidden), "out_proj")


def ltx_video_block(params: dict, x, context, pe, *, heads: int, eps: float = 1e-6,
                    bf16_graph: bool = False, rounding_mode=None) -> np.ndarray:
    """Video branch of ``BasicAVTransformerBlock.__call__``
    (``kinomlx/models/ltx2/transformer/transformer.py:225-276,373-392``) with the text
    cross-attention of ``:201-223``.

    ``params["ada"]`` is ``scale_shift_table + timesteps`` as ``(9, D)`` (``:179-186``): rows
    0-2 attention (shift, scale, gate), 3-5 feed-forward, 6-8 text query. ``params["prompt"]``
    is the ``(2, D)`` context (shift, scale) (``:209-219``).

    ``bf16_graph=False`` (default) is the FP32 evaluation. ``bf16_graph=True`` restates the
    reference's own bf16 execution: FP32 opmath inside each op, and every array the MLX graph
    materialises in the activation dtype rounded to bf16 — each linear output, the stock
    ``rms_norm`` output before modulation and the modulated value (``transformer.py:16-23``),
    sigmoid and the doubled gate (``attention.py:319-325``), Q/K norms, RoPE, attention, the
    per-head gate product, the gated residual (``transformer.py:26-30``), ``_gate`` and the
    cross-attention sum (``:266-276``), GELU (``feed_forward.py:80-97``). It measures the error
    the reference itself carries against the FP32 evaluation. ``rounding_mode="kx"`` rounds only
    where this build's MI355X path stores bf16 (``KX_SITES``).
    """
    store = rounding(rounding_mode or bf16_graph)
    ada = np.asarray(params["ada"], dtype=F32)
    prompt = np.asarray(params["prompt"], dtype=F32)
    value = np.asarray(x, dtype=F32)

    def _adaln(v, scale, shift):
        return store((store(rms_norm(v, eps=eps), "norm_raw") * (F32(1.0) + scale) + shift).astype(F32), "norm")

    normalized_x = _adaln(value, ada[1], ada[0])
    attended = ltx_attention(params, "attn1", normalized_x, heads=heads, pe=pe, eps=eps, store=store)
    value = store(gated_residual(value, attended, ada[2]), "resid")

    query = _adaln(value, ada[7], ada[6])
    ctx = store(modulate(context, prompt[1], prompt[0]), "ctx")
    cross = ltx_attention(params, "attn2", query, heads=heads, context=ctx, eps=eps, store=store)
    value = store((value + store(gate(cross, ada[8]), "gated")).astype(F32), "resid")

    normalized_x = _adaln(value, ada[4], ada[3])
    return store(gated_residual(value, ltx_feed_forward(params, "ff", normalized_x, store), ada[5]), "resid")


def _heads_norm(value, weight, heads: int, eps: float = 1e-6) -> np.ndarray:
    tokens, width = value.shape
    return rms_norm(value.reshape(tokens, heads, width // heads), weight, eps).reshape(tokens, width)


def _heads_rope(value, cos, sin, heads: int) -> np.ndarray:
    tokens, width = value.shape
    rotated = pair_rope(value.reshape(tokens, heads, width // heads), cos[:, None, :], sin[:, None, :])
    return rotated.reshape(tokens, width)


def _joint_attention(q_parts, k_parts, v_parts, rope, heads: int, store=_keep) -> np.ndarray:
    """Concatenate [text, image] streams, rotate Q/K by adjacent pairs, attend
    (``kinomlx/models/flux2/transformer.py:35-53``; ``kv.py:48-54``)."""
    q = np.concatenate(q_parts, axis=0)
    k = np.concatenate(k_parts, axis=0)
    v = np.concatenate(v_parts, axis=0)
    cos, sin = rope
    q = store(_heads_rope(q, cos, sin, heads), "qk")
    k = store(_heads_rope(k, cos, sin, heads), "qk")
    return store(store(attention(q, k, v, heads=heads), "attn"), "attn_gated")


def _flux_normalized(store):
    """``normalized`` as the reference's graph evaluates it: ``mx.fast.layer_norm`` returns the
    activation dtype, then the compiled modulation (``flux2/transformer.py:56-60``)."""

    def run(value, shift, scale):
        n = store(layer_norm(value), "norm_raw")
        return store((n * (F32(1.0) + scale) + shift).astype(F32), "norm")

    return run


def _flux_swiglu(store):
    """``silu(gate) * content`` with ``fused_ops.silu`` returning the activation dtype
    (``flux2/transformer.py:63-65``)."""

    def run(value):
        half = value.shape[-1] // 2
        return store((store(silu(value[..., :half]), "act_silu") * value[..., half:]).astype(F32), "act")

    return run


def flux_double_block(params: dict, image, text, image_mod, text_mod, rope, *, heads: int, ff: str = "swiglu",
                      bf16_graph: bool = False, rounding_mode=None):
    """FLUX.2 ``DoubleBlock.__call__`` (``kinomlx/models/flux2/transformer.py:136-167``) with
    ``DoubleAttention`` (``:88-133``): LayerNorm modulation, per-head QKNorm, joint [text, image]
    attention with adjacent-pair RoPE, gated residuals.

    ``image_mod``/``text_mod`` are ``(6, D)``: shift, scale, gate, ff_shift, ff_scale, ff_gate.
    ``rope`` is ``(cos, sin)`` of shape ``(T_text + T_image, Dh)``. ``ff`` selects the
    feed-forward: ``"swiglu"`` (FLUX, ``:63-85``) or ``"gelu"`` (LTX ``FeedForward``, config 1).

    ``bf16_graph=True`` restates the reference's own bf16 execution: every array the MLX graph
    materialises in the activation dtype is rounded to bf16 — the layer norm and the modulated
    value, each projection, the QK norms, each rotation, the attention output, the gate
    products and the residual sums (``:155-166``), SiLU and the SwiGLU product.
    ``rounding_mode="kx"`` rounds only where this build's MI355X path stores bf16 (``KX_SITES``).
    """
    store = rounding(rounding_mode or bf16_graph)
    norm = _flux_normalized(store)
    glu = _flux_swiglu(store)
    image = np.asarray(image, dtype=F32)
    text = np.asarray(text, dtype=F32)
    im = np.asarray(image_mod, dtype=F32)
    tm = np.asarray(text_mod, dtype=F32)

    def lin(name, value, site="proj"):
        return store(_lin(params, name, value), site)

    def qk(name, norm_name, value):
        return store(_heads_norm(lin(name, value), params[norm_name], heads), "qk_norm")

    img_n = norm(image, im[0], im[1])
    txt_n = norm(text, tm[0], tm[1])
    q = [qk("attn.add_q_proj", "attn.norm_added_q.weight", txt_n), qk("attn.to_q", "attn.norm_q.weight", img_n)]
    k = [qk("attn.add_k_proj", "attn.norm_added_k.weight", txt_n), qk("attn.to_k", "attn.norm_k.weight", img_n)]
    v = [lin("attn.add_v_proj", txt_n), lin("attn.to_v", img_n)]
    result = _joint_attention(q, k, v, rope, heads, store)
    t_text = text.shape[0]
    ai = lin("attn.to_out", result[t_text:], "out_proj")
    at = lin("attn.to_add_out", result[:t_text], "out_proj")
    image = store((image + store(im[2] * ai, "gated")).astype(F32), "resid")
    text = store((text + store(tm[2] * at, "gated")).astype(F32), "resid")

    def feed_forward(prefix: str, value):
        if ff == "swiglu":
            return lin(f"{prefix}.linear_out", glu(lin(f"{prefix}.linear_in", value)), "out_proj")
        return ltx_feed_forward(params, prefix, value, store)

    image = store((image + store(im[5] * feed_forward("ff", norm(image, im[3], im[4])), "gated")).astype(F32), "resid")
    text = store((text + store(tm[5] * feed_forward("ff_context", norm(text, tm[3], tm[4])), "gated")).astype(F32),
                 "resid")
    return image, text


def flux_single_block(params: dict, value, modulation, rope, *, heads: int, width: int, bf16_graph: bool = False,
                      rounding_mode=None):
    """FLUX.2 ``SingleBlock.__call__`` (``kinomlx/models/flux2/transformer.py:201-220``) with
    ``SingleAttention`` (``:170-198``): one fused projection split [D, 2D, 3D], per-head QKNorm,
    adjacent-pair RoPE, ``to_out(concat[attention, swiglu(mlp)])``, gated residual.
    ``modulation`` is ``(3, D)``: shift, scale, gate. ``bf16_graph`` and ``rounding_mode`` as
    ``flux_double_block``."""
    store = rounding(rounding_mode or bf16_graph)
    x = np.asarray(value, dtype=F32)
    mod = np.asarray(modulation, dtype=F32)
    n = _flux_normalized(store)(x, mod[0], mod[1])
    fused = store(_lin(params, "attn.to_qkv_mlp_proj", n), "proj")
    q, k, v, mlp = fused[:, :width], fused[:, width : 2 * width], fused[:, 2 * width : 3 * width], fused[:, 3 * width :]
    q = store(_heads_norm(q, params["attn.norm_q.weight"], heads), "qk_norm")
    k = store(_heads_norm(k, params["attn.norm_k.weight"], heads), "qk_norm")
    attn = _joint_attention([q], [k], [v], rope, heads, store)
    out = store(_lin(params, "attn.to_out", np.concatenate([attn, _flux_swiglu(store)(mlp)], axis=-1)), "out_proj")
    return store((x + store(mod[2] * out, "gated")).astype(F32), "resid")


def config1_double_block(params: dict, image, text, image_mod, text_mod, rope, *, heads: int,
                         bf16_graph: bool = False, rounding_mode=None):
    """This build's config-1 block: the FLUX.2 double-stream structure with LTX's GELU-tanh
    feed-forward (biases on the feed-forward only) and Krea-style per-axis RoPE tables."""
    return flux_double_block(params, image, text, image_mod, text_mod, rope, heads=heads, ff="gelu",
                             bf16_graph=bf16_graph, rounding_mode=rounding_mode)


def krea_attention(params: dict, prefix: str, value, *, heads: int, kv_heads: int, eps: float, rotary=None,
                   store=_keep) -> np.ndarray:
    """``Krea2Attention.__call__`` without a mask (``kinomlx/models/krea2/transformer/model.py:134-196``):
    Q/K/V/gate projections, zero-centred per-head RMSNorm on Q and K, adjacent-pair RoPE with
    ``(T, Dh)`` tables, grouped-query SDPA (query head ``h`` reads K/V head ``h // (H / Hkv)``,
    scale ``Dh ** -0.5``), ``attended * sigmoid(gate)`` over the full width, ``to_out``."""
    x = np.asarray(value, dtype=F32)
    tokens, hidden = x.shape
    dh = hidden // heads
    q = store(_lin(params, f"{prefix}.to_q", x)).reshape(tokens, heads, dh)
    k = store(_lin(params, f"{prefix}.to_k", x)).reshape(tokens, kv_heads, dh)
    v = store(_lin(params, f"{prefix}.to_v", x)).reshape(tokens, kv_heads, dh)
    g = store(_lin(params, f"{prefix}.to_gate", x))
    q = store(rms_norm(q, params[f"{prefix}.norm_q.weight"], eps, weight_offset=1.0))
    k = store(rms_norm(k, params[f"{prefix}.norm_k.weight"], eps, weight_offset=1.0))
    if rotary is not None:
        cos, sin = rotary
        q = store(pair_rope(q, cos[:, None, :], sin[:, None, :]))
        k = store(pair_rope(k, cos[:, None, :], sin[:, None, :]))
    group = heads // kv_heads
    k_full = np.repeat(k, group, axis=1).reshape(tokens, hidden)
    v_full = np.repeat(v, group, axis=1).reshape(tokens, hidden)
    out = store(attention(q.reshape(tokens, hidden), k_full, v_full, heads=heads))
    out = store(out * store(sigmoid(g)))
    return store(_lin(params, f"{prefix}.to_out", out))


def krea_block(params: dict, value, modulation, rotary, *, heads: int, kv_heads: int, eps: float = 1e-6,
               bf16_graph: bool = False) -> np.ndarray:
    """``Krea2TransformerBlock.__call__`` (``kinomlx/models/krea2/transformer/model.py:310-348``).

    ``modulation`` is the ``(6, D)`` sum ``time_modulation + scale_shift_table`` in the official
    chunk order (prescale, preshift, pregate, postscale, postshift, postgate; ``:288-307``).
    ``norm1``/``norm2`` are zero-centred RMSNorms with weights (``:29-46``); the feed-forward is
    ``down(silu(gate(x)) * up(x))`` (``:199-214``). ``bf16_graph=True`` rounds every array the
    MLX graph materialises to bf16, as ``ltx_video_block`` does."""
    store = rounding(bf16_graph)
    x = np.asarray(value, dtype=F32)
    mod = np.asarray(modulation, dtype=F32)
    pre_s, pre_sh, pre_g, post_s, post_sh, post_g = mod
    one = F32(1.0)

    def modulated(v, norm_name, scale, shift):
        n = store(rms_norm(v, params[norm_name], eps, weight_offset=1.0))
        return store((store(store(one + scale) * n) + shift).astype(F32))

    attn = krea_attention(params, "attn", modulated(x, "norm1.weight", pre_s, pre_sh), heads=heads,
                          kv_heads=kv_heads, eps=eps, rotary=rotary, store=store)
    x = store((x + store(pre_g * attn)).astype(F32))
    f = modulated(x, "norm2.weight", post_s, post_sh)
    hidden = store(store(silu(store(_lin(params, "ff.gate", f)))) * store(_lin(params, "ff.up", f)))
    ff = store(_lin(params, "ff.down", hidden))
    return store((x + store(post_g * ff)).astype(F32))


def _ltx_first_branches(params: dict, pre: str, x, context, pe, *, heads: int, eps: float, store):
    """Self-attention then text cross-attention of one stream (``transformer.py:244-308``)."""
    ada = np.asarray(params[f"{pre}ada"], dtype=F32)
    prompt = np.asarray(params[f"{pre}prompt"], dtype=F32)

    def _adaln(v, scale, shift):
        return store((store(rms_norm(v, eps=eps)) * (F32(1.0) + scale) + shift).astype(F32))

    value = np.asarray(x, dtype=F32)
    attended = ltx_attention(params, f"{pre}attn1", _adaln(value, ada[1], ada[0]), heads=heads, pe=pe, eps=eps,
                             store=store)
    value = store(gated_residual(value, attended, ada[2]))
    query = _adaln(value, ada[7], ada[6])
    ctx = store(modulate(context, prompt[1], prompt[0]))
    cross = ltx_attention(params, f"{pre}attn2", query, heads=heads, context=ctx, eps=eps, store=store)
    return store((value + store(gate(cross, ada[8]))).astype(F32)), _adaln


def ltx_av_block(params: dict, video_x, audio_x, video_context, audio_context, pe, audio_pe, cross_pe,
                 audio_cross_pe, *, heads: int, audio_heads: int, eps: float = 1e-6, bf16_graph: bool = False):
    """``BasicAVTransformerBlock.__call__`` with both streams enabled
    (``kinomlx/models/ltx2/transformer/transformer.py:225-421``): each stream's self- and text
    cross-attention, then the audio -> video and video -> audio cross-attention from the
    RMS-normalized bases of both streams (``:310-371``), then each stream's feed-forward.

    ``params`` holds the video block's names as ``ltx_video_block`` (``ada`` (9, Dv),
    ``prompt`` (2, Dv)), the audio stream's under an ``audio_`` prefix (``audio_attn1.*``,
    ``audio_attn2.*``, ``audio_ff.*``, ``audio_ada``, ``audio_prompt``), the cross-attentions
    ``audio_to_video_attn.*`` / ``video_to_audio_attn.*`` and the ``(5, D)`` rows ``av_video`` /
    ``av_audio`` = table + cross timesteps (``:188-199``): scale a2v, shift a2v, scale v2a,
    shift v2a, gate. Returns ``(video, audio)``, tokens leading."""
    store = rounding(bf16_graph)
    v, _adaln = _ltx_first_branches(params, "", video_x, video_context, pe, heads=heads, eps=eps, store=store)
    a, _ = _ltx_first_branches(params, "audio_", audio_x, audio_context, audio_pe, heads=audio_heads, eps=eps,
                               store=store)
    av_v = np.asarray(params["av_video"], dtype=F32)
    av_a = np.asarray(params["av_audio"], dtype=F32)
    v_norm, a_norm = store(rms_norm(v, eps=eps)), store(rms_norm(a, eps=eps))
    a2v = ltx_attention(params, "audio_to_video_attn", store(modulate(v_norm, av_v[0], av_v[1])), heads=audio_heads,
                        context=store(modulate(a_norm, av_a[0], av_a[1])), pe=cross_pe, k_pe=audio_cross_pe, eps=eps,
                        store=store)
    v2a = ltx_attention(params, "video_to_audio_attn", store(modulate(a_norm, av_a[2], av_a[3])), heads=audio_heads,
                        context=store(modulate(v_norm, av_v[2], av_v[3])), pe=audio_cross_pe, k_pe=cross_pe, eps=eps,
                        store=store)
    v = store(gated_residual(v, a2v, av_v[4]))
    a = store(gated_residual(a, v2a, av_a[4]))
    ada, audio_ada = np.asarray(params["ada"], dtype=F32), np.asarray(params["audio_ada"], dtype=F32)
    v = store(gated_residual(v, ltx_feed_forward(params, "ff", _adaln(v, ada[4], ada[3]), store), ada[5]))
    a = store(gated_residual(a, ltx_feed_forward(params, "audio_ff", _adaln(a, audio_ada[4], audio_ada[3]), store),
                             audio_ada[5]))
    return v, a
