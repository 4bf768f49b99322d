"""Operator-level CPU restatement of the reference's DiT-block math (test infrastructure only).

Each function names the reference file:line whose MLX arithmetic it restates. Arrays are numpy
float32 unless stated; bfloat16 data is carried as float32 values that bf16 represents exactly.
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32

__all__ = [
    "adaln",
    "attention",
    "bf16_bits",
    "dequantize_affine",
    "dequantize_mxfp8",
    "e4m3_decode",
    "e4m3_encode",
    "e8m0_scale",
    "mxfp8_linear",
    "pack_bytes",
    "quantize_mxfp8",
    "unpack_bytes",
    "flux_rotary_positions",
    "fractional_positions",
    "frequency_grid",
    "from_bf16_bits",
    "gate",
    "gated_residual",
    "gelu_approx",
    "krea_apply_rotary",
    "krea_rms_norm",
    "krea_rotary",
    "layer_norm",
    "linear",
    "modulate",
    "normalized",
    "pack_affine",
    "pair_rope",
    "precompute_freqs_cis",
    "quantize_affine",
    "quantized_linear",
    "rms_norm",
    "silu",
    "split_rope",
    "swiglu",
    "to_bf16",
    "unpack_affine",
    "E2M1_MAX",
    "dequantize_fp4",
    "e2m1_decode",
    "e2m1_encode",
    "fp4_linear",
    "pack_nibbles",
    "quantize_mxfp4",
    "quantize_nvfp4",
    "unpack_nibbles",
]


# ---------------------------------------------------------------------------------------------
# bfloat16 helpers (round-to-nearest-even, the rounding of every bf16 store on both sides)


def bf16_bits(value: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even; NaNs stay quiet NaNs."""
    u = np.ascontiguousarray(value, dtype=F32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    quiet = ((u >> 16) | 0x40) & 0xFFFF
    return np.where(nan, quiet, rounded).astype(np.uint16)


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def to_bf16(value: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return from_bf16_bits(bf16_bits(value))


def _f32(value) -> np.ndarray:
    return np.asarray(value, dtype=F32)


# ---------------------------------------------------------------------------------------------
# Norms and modulation


def rms_norm(value, weight=None, eps: float = 1e-6, *, weight_offset: float = 0.0) -> np.ndarray:
    """RMSNorm over the last axis with FP32 opmath.

    Weighted form: ``x * rsqrt(mean(x^2) + eps) * (w + weight_offset)``
    (``kinomlx/kernels/fused_ops.py:141-193`` reduction and affine order, ``:412-457`` policy).
    Unweighted form: ``mx.fast.rms_norm(x, None, eps)`` (``fused_ops.py:437-441``).
    """
    x = _f32(value)
    mean_square = np.mean(x * x, axis=-1, keepdims=True, dtype=F32)
    inverse = F32(1.0) / np.sqrt(mean_square + F32(eps))
    out = x * inverse
    if weight is not None:
        out = out * (_f32(weight) + F32(weight_offset))
    return out.astype(F32)


def layer_norm(value, eps: float = 1e-6) -> np.ndarray:
    """Non-affine LayerNorm, ``mx.fast.layer_norm(x, None, None, eps)``
    (``kinomlx/models/flux2/transformer.py:56-57``)."""
    x = _f32(value)
    mean = np.mean(x, axis=-1, keepdims=True, dtype=F32)
    centred = x - mean
    variance = np.mean(centred * centred, axis=-1, keepdims=True, dtype=F32)
    return (centred / np.sqrt(variance + F32(eps))).astype(F32)


def adaln(value, scale, shift, eps: float = 1e-6) -> np.ndarray:
    """LTX AdaLN: ``rms_norm(x) * (1 + scale) + shift``
    (``kinomlx/models/ltx2/transformer/transformer.py:16-23``)."""
    return (rms_norm(value, eps=eps) * (F32(1.0) + _f32(scale)) + _f32(shift)).astype(F32)


def modulate(value, scale, shift) -> np.ndarray:
    """``x * (1 + scale) + shift`` (``transformer.py:33-34``)."""
    return (_f32(value) * (F32(1.0) + _f32(scale)) + _f32(shift)).astype(F32)


def gated_residual(value, residual, gate_value) -> np.ndarray:
    """``x + r * gate`` (``transformer.py:26-30``)."""
    return (_f32(value) + _f32(residual) * _f32(gate_value)).astype(F32)


def gate(value, gate_value) -> np.ndarray:
    """``x * gate`` (``transformer.py:37-38``)."""
    return (_f32(value) * _f32(gate_value)).astype(F32)


def normalized(value, shift, scale, eps: float = 1e-6) -> np.ndarray:
    """FLUX.2 modulation: ``layer_norm(x) * (1 + scale) + shift``
    (``kinomlx/models/flux2/transformer.py:56-57``)."""
    return (layer_norm(value, eps) * (F32(1.0) + _f32(scale)) + _f32(shift)).astype(F32)


def krea_rms_norm(value, weight, eps: float) -> np.ndarray:
    """Zero-centred RMSNorm ``x * rsqrt(mean(x^2) + eps) * (w + 1)``
    (``kinomlx/models/krea2/transformer/model.py:29-46``)."""
    return rms_norm(value, weight, eps, weight_offset=1.0)


# ---------------------------------------------------------------------------------------------
# Activations


def gelu_approx(value) -> np.ndarray:
    """tanh GELU with the inner argument clamped to +-10, FP32
    (``kinomlx/kernels/fused_ops.py:27-35``)."""
    x = _f32(value)
    inner = F32(0.7978845608028654) * (x + F32(0.044715) * (x * x * x))
    inner = np.clip(inner, F32(-10.0), F32(10.0))
    return (F32(0.5) * x * (F32(1.0) + np.tanh(inner))).astype(F32)


def silu(value) -> np.ndarray:
    """``x / (1 + exp(-x))`` in FP32 (``kinomlx/kernels/fused_ops.py:40-45``)."""
    x = _f32(value)
    with np.errstate(over="ignore"):
        return (x / (F32(1.0) + np.exp(-x))).astype(F32)


def swiglu(value) -> np.ndarray:
    """``silu(gate) * content`` over the two halves of the last axis
    (``kinomlx/models/flux2/transformer.py:63-65``)."""
    x = _f32(value)
    half = x.shape[-1] // 2
    return (silu(x[..., :half]) * x[..., half:]).astype(F32)


# ---------------------------------------------------------------------------------------------
# Rotary embeddings


def split_rope(value, cos, sin) -> np.ndarray:
    """Split-half rotation of flattened-head activations by head-major FP32 tables.

    ``value`` is ``(B, T, H * 2 * half)``; ``cos``/``sin`` are ``(B or 1, H, T, half)``. For each
    head and ``i < half``: ``o[i] = x[i]c - x[i+half]s`` and ``o[i+half] = x[i]s + x[i+half]c``
    with each product rounded in FP32 before the difference/sum
    (``kinomlx/kernels/split_rope.py:35-56``; graph ``kinomlx/models/ltx2/transformer/rope.py:18-61``).
    """
    x = _f32(value)
    c = _f32(cos)
    s = _f32(sin)
    batch, tokens, width = x.shape
    _, heads, t2, half = c.shape
    if t2 != tokens or width != heads * 2 * half:
        raise ValueError("split RoPE shape mismatch")
    xh = x.reshape(batch, tokens, heads, 2 * half).transpose(0, 2, 1, 3)
    first = xh[..., :half]
    second = xh[..., half:]
    first_c = first * c
    second_s = second * s
    first_s = first * s
    second_c = second * c
    out = np.concatenate([first_c - second_s, first_s + second_c], axis=-1)
    return out.transpose(0, 2, 1, 3).reshape(batch, tokens, width).astype(F32)


def frequency_grid(theta: float, position_dims: int, inner_dim: int) -> np.ndarray:
    """``theta ** (j / (n - 1)) * pi / 2`` for ``j < n = inner_dim // (2 * position_dims)``, in host
    double precision, then narrowed to FP32 (``kinomlx/models/ltx2/transformer/rope.py:75-92``)."""
    count = inner_dim // (2 * position_dims)
    if count <= 0:
        raise ValueError("RoPE dimension is too small for its position axes")
    exponents = (0.0,) if count == 1 else tuple(j / (count - 1) for j in range(count))
    return np.array([math.pow(theta, e) * math.pi / 2 for e in exponents], dtype=np.float64).astype(
        F32
    )


def fractional_positions(positions, max_pos, *, use_middle_indices_grid: bool) -> np.ndarray:
    """Positions ``(B, axes, T[, 2])`` -> ``(B, T, axes)`` fractions of ``max_pos``
    (``kinomlx/models/ltx2/transformer/rope.py:95-112``)."""
    p = np.asarray(positions)
    if p.shape[1] != len(max_pos):
        raise ValueError("position axes must match max_pos")
    if use_middle_indices_grid:
        if p.ndim != 4 or p.shape[-1] != 2:
            raise ValueError("middle-position RoPE expects (B, axes, T, 2) bounds")
        p = (_f32(p[..., 0]) + _f32(p[..., 1])) / F32(2.0)
    elif p.ndim == 4:
        p = p[..., 0]
    scale = np.asarray(max_pos, dtype=F32)[None, :, None]
    return (_f32(p) / scale).transpose(0, 2, 1)


def precompute_freqs_cis(
    indices_grid,
    *,
    dim: int,
    theta: float = 10000.0,
    max_pos=(20, 2048, 2048),
    use_middle_indices_grid: bool = False,
    num_attention_heads: int = 32,
) -> tuple[np.ndarray, np.ndarray]:
    """Split-RoPE cosine/sine tables ``(B, H, T, dim / (2H))`` in FP32
    (``kinomlx/models/ltx2/transformer/rope.py:115-176``).

    ``scaled = 2 * fraction - 1``; ``freq[b, t, j * axes + a] = scaled[b, t, a] * grid[j]``
    (frequency-major, axis-minor); front-padded with ``cos = 1``, ``sin = 0`` up to ``dim / 2``.
    """
    if dim % num_attention_heads:
        raise ValueError("RoPE dimension must divide evenly across attention heads")
    grid_in = np.asarray(indices_grid)
    fractional = fractional_positions(grid_in, tuple(max_pos), use_middle_indices_grid=use_middle_indices_grid)
    grid = frequency_grid(theta, grid_in.shape[1], dim)
    scaled = fractional * F32(2.0) - F32(1.0)
    frequencies = scaled[..., None] * grid[None, None, None, :]  # (B, T, axes, n)
    frequencies = frequencies.transpose(0, 1, 3, 2).reshape(frequencies.shape[0], frequencies.shape[1], -1)
    expected = dim // 2
    padding = expected - frequencies.shape[-1]
    if padding < 0:
        raise ValueError("RoPE frequency grid exceeds half the model dimension")
    cos = np.cos(frequencies).astype(F32)
    sin = np.sin(frequencies).astype(F32)
    if padding:
        cos = np.concatenate([np.ones((*cos.shape[:-1], padding), F32), cos], axis=-1)
        sin = np.concatenate([np.zeros((*sin.shape[:-1], padding), F32), sin], axis=-1)
    batch, tokens, _ = cos.shape
    cos = cos.reshape(batch, tokens, num_attention_heads, -1).transpose(0, 2, 1, 3)
    sin = sin.reshape(batch, tokens, num_attention_heads, -1).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def pair_rope(value, cos, sin) -> np.ndarray:
    """Adjacent-pair rotation ``(x0, x1) -> (x0 c0 - x1 s0, x1 c1 + x0 s1)`` in FP32, cast back
    (``kinomlx/models/flux2/transformer.py:25-29``; Krea ``model.py:69-92``).

    ``value`` is ``(..., Dh)``; ``cos``/``sin`` broadcast against it.
    """
    x = _f32(value)
    pairs = x.reshape(*x.shape[:-1], -1, 2)
    perpendicular = np.stack([-pairs[..., 1], pairs[..., 0]], axis=-1).reshape(x.shape)
    return (x * _f32(cos) + perpendicular * _f32(sin)).astype(F32)


def flux_rotary_positions(ids) -> tuple[np.ndarray, np.ndarray]:
    """FLUX.2 tables from ``(B, T, 4)`` ids: ``freq_i = 2000^(-2i/32)``, ``i < 16`` per axis,
    angles repeated pairwise to ``(B, T, 1, 128)`` (``kinomlx/models/flux2/transformer.py:17-22``)."""
    frequency = (F32(2000.0) ** (-np.arange(0, 32, 2, dtype=F32) / F32(32))).astype(F32)
    ids = _f32(ids)
    angles = (ids[..., None] * frequency).reshape(*ids.shape[:-1], 64)
    angles = np.repeat(angles, 2, axis=-1)
    return np.cos(angles)[:, :, None].astype(F32), np.sin(angles)[:, :, None].astype(F32)


def krea_rotary(position_ids, *, theta: float, axes_dims) -> tuple[np.ndarray, np.ndarray]:
    """Per-axis ``1 / theta^(2i/d_axis)`` frequencies, adjacent-pair repetition, axes concatenated
    in declared order (``kinomlx/models/krea2/transformer/model.py:49-66``)."""
    positions = _f32(position_ids)
    if positions.ndim != 3 or positions.shape[-1] != len(axes_dims):
        raise ValueError("position_ids must have shape [batch, sequence, position_axes]")
    parts = []
    for axis, dims in enumerate(axes_dims):
        frequencies = (F32(1.0) / (F32(theta) ** (np.arange(0, dims, 2, dtype=F32) / F32(dims)))).astype(F32)
        angles = positions[..., axis, None] * frequencies
        parts.append(np.repeat(angles, 2, axis=-1))
    combined = np.concatenate(parts, axis=-1)
    return np.cos(combined).astype(F32), np.sin(combined).astype(F32)


def krea_apply_rotary(queries, keys, cos, sin) -> tuple[np.ndarray, np.ndarray]:
    """Krea adjacent-pair RoPE on head-major ``(B, H, T, Dh)`` with ``(B, T, Dh)`` tables
    (``kinomlx/models/krea2/transformer/model.py:69-92``)."""
    c = _f32(cos)[:, None, :, :]
    s = _f32(sin)[:, None, :, :]
    return pair_rope(queries, c, s), pair_rope(keys, c, s)


# ---------------------------------------------------------------------------------------------
# Attention and linear products


def attention(q, k, v, *, heads: int, scale: float | None = None, bias=None) -> np.ndarray:
    """Non-causal softmax attention on token-major flattened heads.

    ``q`` is ``(Tq, H * Dh)``, ``k``/``v`` are ``(Tk, H * Dh)``; output ``(Tq, H * Dh)``.
    ``softmax(q k^T * Dh^-0.5 + bias) v`` per head, FP32 scores and accumulation (contract of
    ``kinomlx/models/ltx2/kernels/dense_attention.py:87-153``; SDPA
    ``kinomlx/models/ltx2/transformer/attention.py:144-185``). ``bias`` (optional, additive, the
    SDPA mask) broadcasts as ``(H | 1, Tq | 1, Tk)``; a row whose biases are all the dtype
    minimum keeps equal scores, as in the reference.
    """
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    tq, width = q.shape
    tk = k.shape[0]
    dh = width // heads
    sc = F32(dh ** -0.5 if scale is None else scale)
    out = np.empty((tq, width), F32)
    if bias is not None:
        bias = np.broadcast_to(_f32(bias), (heads, tq, tk))
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        qh = q[:, sl]
        kh = k[:, sl]
        vh = v[:, sl]
        for start in range(0, tq, 2048):
            stop = min(tq, start + 2048)
            scores = (qh[start:stop] @ kh.T) * sc
            if bias is not None:
                scores = (scores + bias[h, start:stop]).astype(F32)
            scores -= scores.max(axis=-1, keepdims=True)
            np.exp(scores, out=scores)
            denom = scores.sum(axis=-1, keepdims=True, dtype=F32)
            out[start:stop, sl] = (scores @ vh) / denom
    return out


def linear(value, weight, bias=None) -> np.ndarray:
    """``addmm(bias, x, W^T)`` for an ``(out, in)`` weight: FP32 products and sums, bias added in
    FP32 (``kinomlx/kernels/mpp_linear.py:1-6``, ``:469-506``; ``kinomlx/modeling/layers.py``)."""
    x = _f32(value)
    out = x @ _f32(weight).T
    if bias is not None:
        out = out + _f32(bias)
    return out.astype(F32)


# ---------------------------------------------------------------------------------------------
# Group-wise affine int4 / int8 weights
#
# The arithmetic of ``mx.quantize`` / ``mx.quantized_matmul`` lives in MLX (mlx>=0.32.4,
# ``pyproject.toml:28``), not in the reference tree. Call sites: ``kinomlx/models/ltx2/
# preparation.py:152`` and ``kinomlx/models/ltx2/weights/quantization.py:28-44``; defaults
# ``kinomlx/models/ltx2/weights/tensors.py:185-203`` (affine -> group 64, 4 bits). The packed
# format restated here: ``(N, K * bits / 32)`` uint32 words, element ``j`` of a word at bits
# ``[bits*j, bits*(j+1))`` (little-endian nibble/byte order), bf16 scale and bias per group of
# ``group_size`` along K, ``w = scale * q + bias``.


def pack_affine(codes: np.ndarray, bits: int) -> np.ndarray:
    """``(N, K)`` integer codes -> ``(N, K * bits / 32)`` little-endian uint32 words."""
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    per_word = 32 // bits
    c = np.asarray(codes, dtype=np.uint32)
    n, k = c.shape
    if k % per_word:
        raise ValueError("K must fill whole words")
    c = c.reshape(n, k // per_word, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * bits)[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def unpack_affine(words: np.ndarray, bits: int) -> np.ndarray:
    """``(N, W)`` uint32 words -> ``(N, W * 32 / bits)`` integer codes (uint32)."""
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    per_word = 32 // bits
    w = np.asarray(words, dtype=np.uint32)
    shifts = (np.arange(per_word, dtype=np.uint32) * bits)[None, None, :]
    mask = np.uint32((1 << bits) - 1)
    return ((w[..., None] >> shifts) & mask).reshape(w.shape[0], -1)


def quantize_affine(weight, group_size: int = 64, bits: int = 4):
    """This build's deterministic affine quantizer (stands in for ``mx.quantize``).

    Per group: ``scale = bf16((max - min) / (2^bits - 1))`` (1 for a constant group),
    ``bias = bf16(min)``, ``q = clip(rint((w - bias) / scale), 0, 2^bits - 1)``. Returns
    ``(words uint32 (N, K*bits/32), scales float32 (N, K/group), biases float32 (N, K/group))``
    with scales and biases holding bf16 values.
    """
    w = _f32(weight)
    n, k = w.shape
    if k % group_size:
        raise ValueError("K must be a multiple of the group size")
    levels = (1 << bits) - 1
    groups = w.reshape(n, k // group_size, group_size)
    lo = groups.min(axis=-1)
    hi = groups.max(axis=-1)
    scale = (hi - lo) / F32(levels)
    scale = np.where(scale > 0, scale, F32(1.0)).astype(F32)
    scale_bf = to_bf16(scale)
    scale_bf = np.where(scale_bf > 0, scale_bf, F32(1.0)).astype(F32)
    bias_bf = to_bf16(lo)
    codes = np.rint((groups - bias_bf[..., None]) / scale_bf[..., None])
    codes = np.clip(codes, 0, levels).astype(np.uint32).reshape(n, k)
    return pack_affine(codes, bits), scale_bf, bias_bf


def dequantize_affine(words, scales, biases, *, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """Bit-exact dequantisation ``bf16(fp32(scale) * q + fp32(bias))`` -> ``(N, K)`` float32.

    A bf16 scale (8 significant bits) times ``q < 256`` is exact in FP32, so the only roundings
    are the FP32 add and the final round-to-nearest-even into bf16.
    """
    codes = unpack_affine(words, bits).astype(F32)
    n, k = codes.shape
    s = np.repeat(_f32(scales), group_size, axis=1)[:, :k]
    b = np.repeat(_f32(biases), group_size, axis=1)[:, :k]
    return to_bf16(s * codes + b)


def quantized_linear(value, words, scales, biases, bias=None, *, group_size: int = 64, bits: int = 4):
    """``quantized_matmul(x, w, scales, biases, transpose=True) + bias`` with the bit-exact bf16
    dequantised weight and FP32 accumulation (``kinomlx/models/ltx2/weights/quantization.py:28-44``)."""
    weight = dequantize_affine(words, scales, biases, group_size=group_size, bits=bits)
    return linear(value, weight, bias)


# ---------------------------------------------------------------------------------------------
# MX block-scaled fp8 (``mode="mxfp8"``: group 32, 8 bits; ``kinomlx/models/ltx2/weights/
# tensors.py:185-203``, ``preparation.py:139-157``, ``weights/quantization.py:17-44``). The
# arithmetic lives in MLX (``mx.quantize`` / ``mx.quantized_matmul``, not vendored): the format
# follows the OCP Microscaling (MX) v1.0 specification. Elements are FP8 E4M3 (OCP "FN": 1 sign,
# 4 exponent bits with bias 7, 3 mantissa bits; exponent 0 is subnormal m * 2^-9; 0x7F / 0xFF
# are NaN; no infinities; the largest finite value is 448), four per uint32 word little-endian
# (element j at bits [8j, 8j+8)); each run of 32 elements along the quantized axis shares one
# E8M0 scale byte S (2^(S - 127); 255 is NaN). Dequantisation is exact in bf16: an E4M3 value has
# 4 significant bits and the scale is a power of two.

E4M3_MAX = 448.0


def e4m3_decode(codes) -> np.ndarray:
    """FP8 E4M3 (OCP) bytes -> float32, exactly (NaN for 0x7F / 0xFF)."""
    c = np.asarray(codes, dtype=np.uint32)
    sign = np.where((c >> 7) & 1, -1.0, 1.0)
    e = ((c >> 3) & 15).astype(np.int64)
    m = (c & 7).astype(np.float64)
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return (sign * mag).astype(F32)


def e4m3_encode(value) -> np.ndarray:
    """float -> FP8 E4M3 bytes, round to nearest even, saturating at +-448 (values already scaled
    into the element range; NaN -> 0x7F; the sign survives underflow to zero)."""
    v = np.asarray(value, dtype=np.float64)
    a = np.nan_to_num(np.abs(v), nan=0.0, posinf=E4M3_MAX)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -30)))
    e = np.maximum(e, -6.0)  # below 2^-6 the spacing stays 2^-9 (subnormals)
    quantum = np.exp2(e - 3.0)
    q = np.minimum(np.rint(a / quantum) * quantum, E4M3_MAX)
    # re-derive the fields from the rounded magnitude (rounding may carry into the exponent)
    qe = np.floor(np.log2(np.maximum(q, 2.0 ** -30)))
    normal = q >= 2.0 ** -6
    exp_field = np.where(normal, qe + 7.0, 0.0)
    mant = np.where(normal, (q / np.exp2(qe) - 1.0) * 8.0, q / 2.0 ** -9)
    code = (exp_field.astype(np.uint32) << 3) | np.rint(mant).astype(np.uint32)
    code = np.where(q == 0, 0, code) | np.where(np.signbit(v), 0x80, 0).astype(np.uint32)
    return np.where(np.isnan(v), 0x7F, code).astype(np.uint8)


def e8m0_scale(scales) -> np.ndarray:
    """E8M0 scale bytes -> float32 powers of two 2^(S - 127) (NaN for 255)."""
    s = np.asarray(scales, dtype=np.int64)
    return np.where(s == 255, np.nan, np.exp2((s - 127).astype(np.float64))).astype(F32)


def pack_bytes(codes: np.ndarray) -> np.ndarray:
    """``(R, C)`` bytes -> ``(R, C / 4)`` little-endian uint32 words."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    return c.view("<u4").reshape(c.shape[0], c.shape[1] // 4)


def unpack_bytes(words: np.ndarray) -> np.ndarray:
    """``(R, W)`` uint32 words -> ``(R, 4 W)`` bytes."""
    w = np.ascontiguousarray(words, dtype="<u4")
    return w.view(np.uint8).reshape(w.shape[0], w.shape[1] * 4)


def quantize_mxfp8(weight, group_size: int = 32):
    """``(R, C)`` -> ``(words (R, C/4) uint32, scales (R, C/group_size) uint8)`` along the last
    axis, by the OCP MX conversion: shared exponent ``floor(log2(amax)) - 8`` (8 = the exponent of
    E4M3's largest normal), clamped to the E8M0 range; elements RNE to E4M3 with saturation. This
    build's deterministic quantizer (MLX's own exponent choice is not reproduced: parity
    unpinned); a group of zeros gets S = 0."""
    w = np.asarray(weight, dtype=np.float64)
    r, c = w.shape
    if c % group_size or group_size % 4:
        raise ValueError("mxfp8 quantization needs the last axis a multiple of the group size")
    g = w.reshape(r, c // group_size, group_size)
    amax = np.abs(g).max(axis=-1)
    exp = np.floor(np.log2(np.maximum(amax, 2.0 ** -200))) - 8.0
    exp = np.clip(exp, -127.0, 127.0)
    exp = np.where(amax == 0, -127.0, exp)
    scaled = g / np.exp2(exp)[..., None]
    codes = e4m3_encode(scaled).reshape(r, c)
    return pack_bytes(codes), (exp + 127.0).astype(np.uint8)


def dequantize_mxfp8(words, scales, *, group_size: int = 32) -> np.ndarray:
    """Bit-exact dequantisation along the last axis: ``bf16(e4m3(q) * 2^(S-127))`` -> float32
    ``(R, 4 W)``; the product is exact, so the bf16 rounding is the identity for any S in 1..254
    whose result stays above the bf16 normal range."""
    codes = unpack_bytes(words)
    vals = e4m3_decode(codes).astype(np.float64)
    s = np.repeat(e8m0_scale(scales).astype(np.float64), group_size, axis=1)[:, : codes.shape[1]]
    return to_bf16((vals * s).astype(F32))


# ---------------------------------------------------------------------------------------------
# FP4 weights: mxfp4 (OCP MX v1.0) and nvfp4, the modes the reference routes feed-forward layers to
# (``kinomlx/models/ltx2/settings.py:39``, defaults ``kinomlx/models/ltx2/weights/tensors.py:190-195``:
# mxfp4 (32, 4), nvfp4 (16, 4); packed by ``mx.quantize(w, group_size, 4, mode)``,
# ``kinomlx/models/ltx2/preparation.py:152``). The arithmetic lives in MLX (not vendored): the
# formats are the published ones. E2M1 elements: sign bit 3, exponent bits 2-1 (bias 1), mantissa
# bit 0 -> magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6; eight per little-endian uint32 (element j at bits
# [4j, 4j + 4)). mxfp4 scales are E8M0 bytes (2^(S - 127)) per 32; nvfp4 scales are E4M3 bytes per 16.

E2M1_MAX = 6.0
_E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e2m1_decode(codes) -> np.ndarray:
    """FP4 E2M1 codes (0..15) -> float32, from the field definition (exponent e, mantissa m:
    subnormal ``m / 2`` for e = 0, else ``(1 + m / 2) * 2^(e - 1)``)."""
    c = np.asarray(codes, dtype=np.uint32)
    e = ((c >> 1) & 3).astype(np.float64)
    m = (c & 1).astype(np.float64)
    mag = np.where(e == 0, m * 0.5, (1.0 + m * 0.5) * np.exp2(e - 1.0))
    return np.where((c >> 3) & 1, -mag, mag).astype(F32)


def e2m1_encode(value) -> np.ndarray:
    """float -> E2M1 codes: round to nearest even on the E2M1 grid (the quantum is 0.5 below 2, 1 in
    [2, 4) and 2 from 4 on; a tie keeps the even mantissa), saturating at +-6; the sign survives
    (negative zero is code 8); NaN gives 0."""
    v = np.asarray(value, dtype=np.float64)
    a = np.nan_to_num(np.abs(v), nan=0.0, posinf=E2M1_MAX)
    e = np.clip(np.floor(np.log2(np.maximum(a, 2.0 ** -30))), 0.0, 2.0)
    quantum = np.exp2(e - 1.0)
    q = np.minimum(np.rint(a / quantum) * quantum, E2M1_MAX)
    code = np.searchsorted(_E2M1_GRID, q).astype(np.uint32)
    sign = np.where(np.signbit(v) & ~np.isnan(v), 8, 0).astype(np.uint32)
    return (code | sign).astype(np.uint8)


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """``(R, C)`` 4-bit codes -> ``(R, C / 8)`` little-endian uint32 words."""
    return pack_affine(np.asarray(codes, dtype=np.int64), 4)


def unpack_nibbles(words: np.ndarray) -> np.ndarray:
    """``(R, W)`` uint32 words -> ``(R, 8 W)`` 4-bit codes."""
    return unpack_affine(words, 4)


def quantize_mxfp4(weight, group_size: int = 32):
    """``(R, C)`` -> ``(words (R, C/8) uint32, scales (R, C/32) uint8)`` by the OCP MX conversion:
    shared exponent ``floor(log2(amax)) - 2`` (2: the exponent of E2M1's largest normal, 6 = 1.5 *
    2^2), clamped to the E8M0 range (-127 for an all-zero group), elements E2M1 of ``w * 2^-X``. This
    build's quantizer (MLX's own scale choice: parity unpinned)."""
    w = np.asarray(weight, dtype=np.float64)
    r, c = w.shape
    if c % group_size:
        raise ValueError("mxfp4 quantization needs the last axis a multiple of the group size")
    g = w.reshape(r, c // group_size, group_size)
    amax = np.abs(g).max(axis=-1)
    exp = np.clip(np.floor(np.log2(np.maximum(amax, 2.0 ** -200))) - 2.0, -127.0, 127.0)
    exp = np.where(amax == 0, -127.0, exp)
    codes = e2m1_encode(g / np.exp2(exp)[..., None]).reshape(r, c)
    return pack_nibbles(codes), (exp + 127.0).astype(np.uint8)


def quantize_nvfp4(weight, group_size: int = 16):
    """``(R, C)`` -> ``(words (R, C/8) uint32, scales (R, C/16) uint8)``: per group the E4M3 scale
    ``s = E4M3(fp32(amax / 6))`` (RNE, saturating at 448) and elements E2M1 of ``fp32(w / s)`` (IEEE
    fp32 division; zero codes when s is 0). This build's quantizer (NVIDIA's two-level form with a
    per-tensor scale, and MLX's own choice: parity unpinned)."""
    w = np.asarray(weight, dtype=F32)
    r, c = w.shape
    if c % group_size:
        raise ValueError("nvfp4 quantization needs the last axis a multiple of the group size")
    g = w.reshape(r, c // group_size, group_size)
    amax = np.abs(g).max(axis=-1).astype(F32)
    sbytes = e4m3_encode((amax / F32(6.0)).astype(F32)) & 0x7F
    s = e4m3_decode(sbytes)
    with np.errstate(divide="ignore", invalid="ignore"):
        scaled = (g / s[..., None]).astype(F32)
    codes = np.where(s[..., None] > 0, e2m1_encode(scaled), 0).reshape(r, c)
    return pack_nibbles(codes), sbytes.astype(np.uint8)


def dequantize_fp4(words, scales, *, mode: str) -> np.ndarray:
    """Bit-exact dequantisation along the last axis: ``bf16(e2m1(q) * scale)`` -> float32 ``(R, 8 W)``
    (``mode`` ``"mxfp4"``: E8M0 scales per 32; ``"nvfp4"``: E4M3 scales per 16). The product has at
    most 6 significant bits, so the bf16 rounding is the identity in the normal range."""
    codes = unpack_nibbles(words)
    vals = e2m1_decode(codes).astype(np.float64)
    group = 16 if mode == "nvfp4" else 32
    sv = e4m3_decode(scales) if mode == "nvfp4" else e8m0_scale(scales)
    s = np.repeat(sv.astype(np.float64), group, axis=1)[:, : codes.shape[1]]
    return to_bf16((vals * s).astype(F32))


def fp4_linear(value, words, scales, bias=None, *, mode: str):
    """``quantized_matmul(x, w, scales, transpose=True, group_size, bits=4, mode) + bias`` for an
    mxfp4 / nvfp4 ``(out, in / 8)`` packed weight."""
    return linear(value, dequantize_fp4(words, scales, mode=mode), bias)


def mxfp8_linear(value, words, scales, bias=None, *, group_size: int = 32, transposed: bool = True):
    """``quantized_matmul(x, w, scales, transpose=transposed, group_size, bits=8, mode="mxfp8")
    + bias``: with ``transposed`` the packed weight is ``(out, in / 4)`` grouped along ``in``
    (``nn.QuantizedLinear``); without, it was built from ``weight.T`` and is ``(in, out / 4)``
    grouped along ``out`` (``_PretransposedQuantizedLinear``, ``quantization.py:17-44``)."""
    w = dequantize_mxfp8(words, scales, group_size=group_size)
    return linear(value, w if transposed else np.ascontiguousarray(w.T), bias)
