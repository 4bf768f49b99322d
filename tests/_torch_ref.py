"""FP32 PyTorch evaluation of the LTX-2 video block and the FLUX.2 blocks (test infrastructure).

The same composition as ``oracle.ltx_video_block`` written with torch operations, so that the
full-size (9216-token) block can be evaluated in FP32 on the GPU in seconds, where the numpy
oracle would take minutes. ``tests/test_blocks_cpu.py`` pins it against the numpy oracle.
"""

import torch


def _keep(x, site="graph"):
    return x


def bf16_store(x, site="graph"):
    """Round an FP32 tensor to bf16 values (kept in FP32): the reference's materialised arrays."""
    return x.to(torch.bfloat16).float()


def fp16_store(x, site="graph"):
    """Round an FP32 tensor to fp16 values (kept in FP32): the reference's FP16 graph."""
    return x.to(torch.float16).float()


# This build's 16-bit storage points (the same names as ``oracle.blocks.KX_SITES``).
KX_SITES = frozenset({"norm", "proj", "gate", "qk", "attn_gated", "ctx", "act"})


def _kx_store(x, site="graph"):
    return x.to(torch.bfloat16).float() if site in KX_SITES else x


def _kx_store16(x, site="graph"):
    return x.to(torch.float16).float() if site in KX_SITES else x


def rounding(mode, half=torch.bfloat16):
    """``None``/``False``: FP32; ``True``/``"graph"``: the reference's graph in ``half`` (bf16 or
    fp16: every materialised array rounded to it); ``"kx"``: only where the MI355X path stores its
    16-bit type (as ``oracle.blocks.rounding``)."""
    if not mode:
        return _keep
    if mode is True or mode == "graph":
        return fp16_store if half == torch.float16 else bf16_store
    if mode == "kx":
        return _kx_store16 if half == torch.float16 else _kx_store
    raise ValueError(f"unknown rounding mode {mode!r}")


def _lin(p, name, x):
    out = x @ p[f"{name}.weight"].T
    bias = p.get(f"{name}.bias")
    return out if bias is None else out + bias


def _rms(x, w=None, eps=1e-6):
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    return y if w is None else y * w


def _split_rope(x, cos, sin):
    t, width = x.shape
    heads, half = cos.shape[1], cos.shape[3]
    xh = x.reshape(t, heads, 2 * half).transpose(0, 1)
    c, s = cos[0], sin[0]
    first, second = xh[..., :half], xh[..., half:]
    out = torch.cat([first * c - second * s, first * s + second * c], -1)
    return out.transpose(0, 1).reshape(t, width)


def _attention(q, k, v, heads):
    t, width = q.shape
    dh = width // heads
    qh = q.reshape(t, heads, dh).transpose(0, 1)
    kh = k.reshape(k.shape[0], heads, dh).transpose(0, 1)
    vh = v.reshape(v.shape[0], heads, dh).transpose(0, 1)
    out = torch.empty_like(qh)
    kt = kh.transpose(1, 2).contiguous()
    for start in range(0, t, 2048):
        sc = qh[:, start:start + 2048] @ kt * dh ** -0.5
        out[:, start:start + 2048] = torch.softmax(sc, -1) @ vh
    return out.transpose(0, 1).reshape(t, width)


def _ltx_attention(p, prefix, x, heads, context=None, pe=None, st=_keep):
    source = x if context is None else context
    gate = st(2 * st(torch.sigmoid(st(_lin(p, f"{prefix}.to_gate_logits", x), "gate_logits")), "gate_sigmoid"),
              "gate")
    v = st(_lin(p, f"{prefix}.to_v", source), "proj")
    q = st(_rms(st(_lin(p, f"{prefix}.to_q", x), "proj"), p[f"{prefix}.q_norm.weight"]), "qk_norm")
    k = st(_rms(st(_lin(p, f"{prefix}.to_k", source), "proj"), p[f"{prefix}.k_norm.weight"]), "qk_norm")
    if pe is not None:
        q, k = _split_rope(q, *pe), _split_rope(k, *pe)
    q, k = st(q, "qk"), st(k, "qk")
    o = st(_attention(q, k, v, heads), "attn")
    t, width = o.shape
    o = st((o.reshape(t, heads, width // heads) * gate[:, :, None]).reshape(t, width), "attn_gated")
    return st(_lin(p, f"{prefix}.to_out", o), "out_proj")


def ltx_video_block(p, x, context, pe, heads, bf16_graph=False, rounding_mode=None, half=torch.bfloat16):
    """``p``: fp32 tensors named as in ``oracle.ltx_video_block`` (dense weights);
    ``bf16_graph`` / ``rounding_mode`` round at the same sites as the oracle's modes, to ``half``."""
    st = rounding(rounding_mode or bf16_graph, half)
    ada, prompt = p["ada"], p["prompt"]
    n = st(st(_rms(x), "norm_raw") * (1 + ada[1]) + ada[0], "norm")
    x = st(x + _ltx_attention(p, "attn1", n, heads, pe=pe, st=st) * ada[2], "resid")
    q = st(st(_rms(x), "norm_raw") * (1 + ada[7]) + ada[6], "norm")
    ctx = st(context * (1 + prompt[1]) + prompt[0], "ctx")
    x = st(x + st(_ltx_attention(p, "attn2", q, heads, context=ctx, st=st) * ada[8], "gated"), "resid")
    n = st(st(_rms(x), "norm_raw") * (1 + ada[4]) + ada[3], "norm")
    h = st(torch.nn.functional.gelu(st(_lin(p, "ff.proj_in", n), "ff_in"), approximate="tanh"), "act")
    return st(x + st(_lin(p, "ff.proj_out", h), "out_proj") * ada[5], "resid")


def _layer_norm(x, eps=1e-6):
    mean = x.mean(-1, keepdim=True)
    c = x - mean
    return c * torch.rsqrt((c * c).mean(-1, keepdim=True) + eps)


def _pair_rope(x, cos, sin, heads):
    """Adjacent-pair rotation of ``(T, H * Dh)`` rows by ``(T, Dh)`` tables."""
    t, width = x.shape
    xh = x.reshape(t, heads, width // (2 * heads), 2)
    c = cos.reshape(t, 1, -1, 2)[..., 0]
    s = sin.reshape(t, 1, -1, 2)[..., 0]
    x0, x1 = xh[..., 0], xh[..., 1]
    return torch.stack([x0 * c - x1 * s, x1 * c + x0 * s], -1).reshape(t, width)


def _heads_rms(x, w, heads):
    t, width = x.shape
    return _rms(x.reshape(t, heads, width // heads), w).reshape(t, width)


def _swiglu(x, st):
    half = x.shape[-1] // 2
    return st(st(torch.nn.functional.silu(x[..., :half]), "act_silu") * x[..., half:], "act")


def flux_double_block(p, image, text, im, tm, rope, heads, ff="swiglu", bf16_graph=False, rounding_mode=None):
    """Torch form of ``oracle.flux_double_block`` (same names, same rounding sites)."""
    st = rounding(rounding_mode or bf16_graph)

    def norm(x, shift, scale):
        return st(st(_layer_norm(x), "norm_raw") * (1 + scale) + shift, "norm")

    def lin(name, x, site="proj"):
        return st(_lin(p, name, x), site)

    def qk(name, norm_name, x):
        return st(_heads_rms(lin(name, x), p[norm_name], heads), "qk_norm")

    img_n, txt_n = norm(image, im[0], im[1]), norm(text, tm[0], tm[1])
    q = torch.cat([qk("attn.add_q_proj", "attn.norm_added_q.weight", txt_n),
                   qk("attn.to_q", "attn.norm_q.weight", img_n)])
    k = torch.cat([qk("attn.add_k_proj", "attn.norm_added_k.weight", txt_n),
                   qk("attn.to_k", "attn.norm_k.weight", img_n)])
    v = torch.cat([lin("attn.add_v_proj", txt_n), lin("attn.to_v", img_n)])
    q, k = st(_pair_rope(q, *rope, heads), "qk"), st(_pair_rope(k, *rope, heads), "qk")
    result = st(st(_attention(q, k, v, heads), "attn"), "attn_gated")
    tt = text.shape[0]
    image = st(image + st(im[2] * lin("attn.to_out", result[tt:], "out_proj"), "gated"), "resid")
    text = st(text + st(tm[2] * lin("attn.to_add_out", result[:tt], "out_proj"), "gated"), "resid")

    def feed_forward(prefix, x):
        if ff == "swiglu":
            return lin(f"{prefix}.linear_out", _swiglu(lin(f"{prefix}.linear_in", x), st), "out_proj")
        h = st(torch.nn.functional.gelu(lin(f"{prefix}.proj_in", x, "ff_in"), approximate="tanh"), "act")
        return lin(f"{prefix}.proj_out", h, "out_proj")

    image = st(image + st(im[5] * feed_forward("ff", norm(image, im[3], im[4])), "gated"), "resid")
    text = st(text + st(tm[5] * feed_forward("ff_context", norm(text, tm[3], tm[4])), "gated"), "resid")
    return image, text


def flux_single_block(p, x, mod, rope, heads, width, bf16_graph=False, rounding_mode=None):
    """Torch form of ``oracle.flux_single_block``."""
    st = rounding(rounding_mode or bf16_graph)
    n = st(st(_layer_norm(x), "norm_raw") * (1 + mod[1]) + mod[0], "norm")
    fused = st(_lin(p, "attn.to_qkv_mlp_proj", n), "proj")
    q = st(_heads_rms(fused[:, :width], p["attn.norm_q.weight"], heads), "qk_norm")
    k = st(_heads_rms(fused[:, width:2 * width], p["attn.norm_k.weight"], heads), "qk_norm")
    q, k = st(_pair_rope(q, *rope, heads), "qk"), st(_pair_rope(k, *rope, heads), "qk")
    attn = st(st(_attention(q, k, fused[:, 2 * width:3 * width], heads), "attn"), "attn_gated")
    out = st(_lin(p, "attn.to_out", torch.cat([attn, _swiglu(fused[:, 3 * width:], st)], -1)), "out_proj")
    return st(x + st(mod[2] * out, "gated"), "resid")
