"""FP32 torch-CPU restatement of the config-1 block: TEST INFRASTRUCTURE, not product code.

The benchmark's CPU baseline, on torch's CPU kernels with ``torch.set_num_threads``: the same op
sequence and FP32 arithmetic as ``oracle.blocks.config1_double_block`` (the FLUX.2 double-stream
block, ``kinomlx/models/flux2/transformer.py:88-167``, with LTX's GELU-tanh feed-forward,
``kinomlx/models/ltx2/transformer/feed_forward.py:80-97``), without any bf16 rounding. Only
``tests/`` and ``bench.py``'s ``cpu_baseline`` use it; ``tests/test_oracle.py`` pins it to the
numpy restatement on the config-1 block.
"""

from __future__ import annotations

import torch

F = torch.nn.functional


def to_torch(params: dict) -> dict[str, torch.Tensor]:
    """The numpy parameter arrays as FP32 CPU tensors."""
    return {name: torch.as_tensor(value, dtype=torch.float32) for name, value in params.items()}


def _linear(p: dict, name: str, x: torch.Tensor) -> torch.Tensor:
    """``addmm(bias, x, W^T)`` (``kinomlx/kernels/mpp_linear.py:469-506``)."""
    bias = p.get(f"{name}.bias")
    return F.linear(x, p[f"{name}.weight"], bias)


def _normalized(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``layer_norm(x) * (1 + scale) + shift`` (``flux2/transformer.py:56-60``)."""
    return F.layer_norm(x, (x.shape[-1],), eps=eps) * (1.0 + scale) + shift


def _heads_norm(x: torch.Tensor, weight: torch.Tensor, heads: int, eps: float = 1e-6) -> torch.Tensor:
    """Per-head RMSNorm ``x * rsqrt(mean(x^2) + eps) * w`` (``flux2/transformer.py:68-85``)."""
    t, width = x.shape
    h = x.reshape(t, heads, width // heads)
    h = h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps) * weight
    return h.reshape(t, width)


def _pair_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int) -> torch.Tensor:
    """``(x0, x1) -> (x0 c0 - x1 s0, x1 c1 + x0 s1)`` per head (``flux2/transformer.py:25-29``)."""
    t, width = x.shape
    h = x.reshape(t, heads, width // heads)
    pairs = h.reshape(t, heads, -1, 2)
    perpendicular = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).reshape(h.shape)
    return (h * cos[:, None, :] + perpendicular * sin[:, None, :]).reshape(t, width)


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int) -> torch.Tensor:
    """Non-causal softmax attention, scale ``Dh ** -0.5`` (``flux2/kv.py:48-54``)."""
    t, width = q.shape
    dh = width // heads

    def split(x):
        return x.reshape(x.shape[0], heads, dh).transpose(0, 1)

    out = F.scaled_dot_product_attention(split(q)[None], split(k)[None], split(v)[None])
    return out[0].transpose(0, 1).reshape(t, width)


def _gelu_approx(x: torch.Tensor) -> torch.Tensor:
    """tanh GELU with the inner argument clamped to +-10 (``kinomlx/kernels/fused_ops.py:27-35``)."""
    inner = (0.7978845608028654 * (x + 0.044715 * (x * x * x))).clamp(-10.0, 10.0)
    return 0.5 * x * (1.0 + torch.tanh(inner))


def config1_double_block(p: dict, image: torch.Tensor, text: torch.Tensor, image_mod: torch.Tensor,
                         text_mod: torch.Tensor, rope: tuple[torch.Tensor, torch.Tensor], *, heads: int):
    """``oracle.blocks.config1_double_block`` in FP32 on torch's CPU kernels: ``(image, text)``."""
    im, tm = image_mod, text_mod
    img_n = _normalized(image, im[0], im[1])
    txt_n = _normalized(text, tm[0], tm[1])

    def qk(name, norm_name, value):
        return _heads_norm(_linear(p, name, value), p[norm_name], heads)

    q = torch.cat((qk("attn.add_q_proj", "attn.norm_added_q.weight", txt_n),
                   qk("attn.to_q", "attn.norm_q.weight", img_n)))
    k = torch.cat((qk("attn.add_k_proj", "attn.norm_added_k.weight", txt_n),
                   qk("attn.to_k", "attn.norm_k.weight", img_n)))
    v = torch.cat((_linear(p, "attn.add_v_proj", txt_n), _linear(p, "attn.to_v", img_n)))
    cos, sin = rope
    result = _attention(_pair_rope(q, cos, sin, heads), _pair_rope(k, cos, sin, heads), v, heads)
    t_text = text.shape[0]
    image = image + im[2] * _linear(p, "attn.to_out", result[t_text:])
    text = text + tm[2] * _linear(p, "attn.to_add_out", result[:t_text])

    def feed_forward(prefix, value):
        return _linear(p, f"{prefix}.proj_out", _gelu_approx(_linear(p, f"{prefix}.proj_in", value)))

    image = image + im[5] * feed_forward("ff", _normalized(image, im[3], im[4]))
    text = text + tm[5] * feed_forward("ff_context", _normalized(text, tm[3], tm[4]))
    return image, text
