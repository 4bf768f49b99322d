"""Weight-quantized linear layers on MI355X: group-wise affine int4/int8 and mxfp8.

Replaces ``nn.QuantizedLinear`` / ``mx.quantized_matmul(..., mode=...)`` and
``_PretransposedQuantizedLinear`` as the LTX-2 loader installs them
(``kinomlx/models/ltx2/weights/quantization.py:17-44``, ``:199-274``; defaults
``kinomlx/models/ltx2/weights/tensors.py:185-203``: affine -> group 64, 4 bits, mxfp8 -> group 32,
8 bits; quantizer call ``kinomlx/models/ltx2/preparation.py:139-157``).

Format: ``weight`` uint32 words ``(out, in * bits / 32)`` (stored in an int32 tensor), element
``j`` of a word at bits ``[bits*j, bits*(j+1))``; ``scales`` and ``biases`` bf16 ``(out, in /
group_size)``; ``w = scale * q + bias``. The kernel dequantizes inside its MFMA mainloop with
``bf16(fp32(scale) * q + fp32(bias))`` — exact product, one FP32 add, one round-to-nearest-even.

``QuantizedLinear`` holds the packed weight in HBM and, on each GPU call, dequantizes it
(bit-exact, one HBM-bound pass of ``kx_dequant_affine_bf16`` / ``kx_dequant_mxfp8_bf16``) into a
transient bf16 buffer that the dense GEMM multiplies: at the block's row counts the product is
compute-bound, the dense MFMA kernel is the fastest one, and the pass costs 2-3 % of the product
(23 us for a 12288 x 4096 weight against 0.82 ms for 9216 rows). ``quantized_matmul`` is the
allocation-free form: the GEMM dequantizes inside its mainloop (``kx_qgemm_affine_bf16``,
``kx_qgemm_mxfp8_bf16``). Layers of at most 64 outputs keep one dequantized copy.

``quantize`` is this build's deterministic quantizer (MLX's own scale/bias selection is not
reproduced): per group ``scale = bf16((max - min) / (2^bits - 1))``, ``bias = bf16(min)``,
``q = clip(round((w - bias) / scale), 0, 2^bits - 1)``.

mxfp8 (OCP MX): ``weight`` uint32 words ``(out, in / 4)`` of four FP8 E4M3 codes (element ``j`` in
byte ``j``), ``scales`` uint8 ``(out, in / 32)`` E8M0 exponents, no biases; ``w = e4m3(q) *
2^(s - 127)``, exact in bf16. The GEMM converts the codes inside its mainloop. The pretransposed
layout of ``transformer_quantize="mxfp8-blocks-pretranspose"`` (packed from ``weight.T``: words
``(in, out / 4)``, scales ``(in, out / 32)``, groups along the output axis) shares no group with
the ``(out, in)`` layout the GEMM streams, so ``PretransposedQuantizedLinear`` dequantizes it
once, exactly, to the bf16 ``(out, in)`` weight and runs the dense GEMM. ``quantize_mxfp8`` is
the OCP MX conversion (shared exponent ``floor(log2(max |w|)) - 8``, elements rounded to nearest
even and saturated at 448); MLX's own exponent choice is not reproduced.

mxfp4 / nvfp4 (the reference's feed-forward modes, ``video_ff_quantize_specs``,
``kinomlx/models/ltx2/settings.py:39``): ``weight`` uint32 words ``(out, in / 8)`` of eight FP4 E2M1
codes (element ``j`` at bits ``[4j, 4j + 4)``), ``scales`` uint8 ``(out, in / 32)`` E8M0 exponents
(mxfp4) or ``(out, in / 16)`` E4M3 values (nvfp4), no biases; ``w = e2m1(q) * scale``, exact in bf16.
Each GPU call dequantizes (``kx_dequant_fp4_bf16``) and runs the dense GEMM. ``quantize_fp4`` is this
build's conversion (mxfp4: OCP MX shared exponent ``floor(log2(max |w|)) - 2``; nvfp4: E4M3 scale of
``max |w| / 6``; E2M1 round to nearest even, saturated at 6); MLX's own scale choice is not
reproduced.
"""

from __future__ import annotations

import torch

from .. import _lib
from .mpp_linear import ACTIVATIONS

DEFAULT_GROUP_SIZE = 64
DEFAULT_BITS = 4
# (group_size, bits) per mode (``weights/tensors.py:185-203``)
_DEFAULTS = {"affine": (64, 4), "mxfp4": (32, 4), "mxfp8": (32, 8), "nvfp4": (16, 4)}
KERNEL_MODES = ("affine", "mxfp8", "mxfp4", "nvfp4")
# modes whose scales are uint8 exponent / E4M3 bytes and that carry no biases
SCALED_MODES = ("mxfp8", "mxfp4", "nvfp4")
FP4_MODES = ("mxfp4", "nvfp4")


def quant_defaults(mode: str, group_size: int | None, bits: int | None) -> tuple[int, int]:
    """(group_size, bits) with the mode's defaults filled in (``weights/tensors.py:185-203``)."""
    if mode not in _DEFAULTS:
        raise ValueError(f"Unsupported FF quantization mode: {mode}")
    g0, b0 = _DEFAULTS[mode]
    g = g0 if group_size is None else group_size
    b = b0 if bits is None else bits
    if g <= 0 or b <= 0:
        raise ValueError("quantization group size and bits must be positive")
    return g, b


def _check_mode(mode: str, group_size: int, bits: int) -> None:
    """A mode, group size and width this build has kernels for."""
    quant_defaults(mode, group_size, bits)
    if mode not in KERNEL_MODES:
        raise NotImplementedError(f"{mode} quantized linears have no MI355X kernel")
    if mode in SCALED_MODES:
        if (group_size, bits) != _DEFAULTS[mode]:
            want = _DEFAULTS[mode]
            raise ValueError(f"{mode} takes group size {want[0]} and {want[1]} bits, got {group_size} and {bits}")
    else:
        _check_format(group_size, bits)


def _check_format(group_size: int, bits: int) -> None:
    if bits not in (4, 8):
        raise ValueError(f"affine quantization on MI355X takes 4 or 8 bits, got {bits}")
    if group_size != 64:
        raise ValueError(f"affine quantization on MI355X takes group size 64, got {group_size}")


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """``(N, K)`` integer codes -> ``(N, K * bits / 32)`` little-endian words (int32 storage)."""
    per_word = 32 // bits
    n, k = codes.shape
    c = codes.to(torch.int64).reshape(n, k // per_word, per_word)
    shifts = torch.arange(per_word, device=codes.device, dtype=torch.int64) * bits
    words = (c << shifts).sum(dim=-1)  # disjoint bit fields: the sum is the bitwise or
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32)


def unpack(words: torch.Tensor, bits: int) -> torch.Tensor:
    """``(N, W)`` words -> ``(N, W * 32 / bits)`` codes (int64)."""
    per_word = 32 // bits
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per_word, device=words.device, dtype=torch.int64) * bits
    return ((w[..., None] >> shifts) & ((1 << bits) - 1)).reshape(words.shape[0], -1)


def quantize(weight: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE, bits: int = DEFAULT_BITS,
             mode: str = "affine") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(out, in)`` weight -> ``(words, scales, biases)`` in the packed affine format.

    On the GPU this is the quantize-on-load kernel (``kx_quantize_affine_bf16``) on the bf16
    weight. A weight still in host memory (a checkpoint prepared on a machine without a GPU,
    synthetic test weights) is packed by the same arithmetic in torch on the host: the two are
    bit-identical on bf16 weights (tested). The kernel reads bf16: a GPU weight in another dtype
    is cast to bf16 first, as the reference casts to the transformer dtype before quantizing
    (``preparation.py:146-147``)."""
    quant_defaults(mode, group_size, bits)
    _check_format(group_size, bits)
    n, k = (int(v) for v in weight.shape)
    if k % group_size:
        raise ValueError("the input width must be a multiple of the group size")
    if weight.is_cuda:
        w = weight.to(torch.bfloat16)
        if w.stride(-1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
            w = w.contiguous()
        words = torch.empty((n, k * bits // 32), dtype=torch.int32, device=w.device)
        scales = torch.empty((n, k // group_size), dtype=torch.bfloat16, device=w.device)
        biases = torch.empty_like(scales)
        if n:
            _lib.launch_quantize(w, words, scales, biases, group_size=group_size, bits=bits)
        return words, scales, biases
    w = weight.float()
    levels = (1 << bits) - 1
    groups = w.reshape(n, k // group_size, group_size)
    lo = groups.amin(dim=-1)
    hi = groups.amax(dim=-1)
    scale = (hi - lo) / levels
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    scale_bf = scale.to(torch.bfloat16)
    scale_bf = torch.where(scale_bf > 0, scale_bf, torch.ones_like(scale_bf))
    bias_bf = lo.to(torch.bfloat16)
    codes = torch.round((groups - bias_bf.float()[..., None]) / scale_bf.float()[..., None])
    codes = codes.clamp(0, levels).to(torch.int64).reshape(n, k)
    return pack(codes, bits), scale_bf.contiguous(), bias_bf.contiguous()


def _out_buffer(out: torch.Tensor | None, n: int, k: int, device) -> torch.Tensor:
    if out is None:
        return torch.empty((n, k), dtype=torch.bfloat16, device=device)
    if out.shape != (n, k) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"dequantize: out must be a contiguous bf16 ({n}, {k}) tensor")
    return out


def dequantize(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
               group_size: int = DEFAULT_GROUP_SIZE, bits: int = DEFAULT_BITS,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Packed affine weight -> bf16 ``(out, in)`` through the kernel's own dequantization (into
    ``out`` when given)."""
    _check_format(group_size, bits)
    n = int(words.shape[0])
    k = int(words.shape[1]) * 32 // bits
    out = _out_buffer(out, n, k, words.device)
    _lib.launch_dequant(words.contiguous(), scales.contiguous(), biases.contiguous(), out, n=n, k=k,
                        group_size=group_size, bits=bits)
    return out


def quantize_mxfp8(weight: torch.Tensor, group_size: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """``(out, in)`` weight -> mxfp8 ``(words (out, in / 4) int32, scales (out, in / 32) uint8)``.

    On the GPU: the quantize-on-load kernel (``kx_quantize_mxfp8_bf16``) on the bf16 weight. A
    host weight is converted by the same arithmetic in torch (the E4M3 rounding is torch's
    round-to-nearest-even ``float8_e4m3fn`` cast after clamping to +-448): bit-identical on bf16
    weights (tested)."""
    if group_size != 32:
        raise ValueError(f"mxfp8 takes group size 32, got {group_size}")
    n, k = (int(v) for v in weight.shape)
    if k % 32:
        raise ValueError(f"mxfp8 groups the last axis by 32: cannot quantize a {n} x {k} matrix")
    if weight.is_cuda:
        w = weight.to(torch.bfloat16)
        if w.stride(-1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
            w = w.contiguous()
        words = torch.empty((n, k // 4), dtype=torch.int32, device=w.device)
        scales = torch.empty((n, k // 32), dtype=torch.uint8, device=w.device)
        if n:
            _lib.launch_quantize_mxfp8(w, words, scales)
        return words, scales
    w = weight.to(torch.bfloat16).float().reshape(n, k // 32, 32)
    amax = w.abs().amax(dim=-1)
    _, e = torch.frexp(amax)
    x = torch.where(amax > 0, (e.to(torch.int64) - 9).clamp(-127, 127), torch.full_like(e, -127, dtype=torch.int64))
    scaled = torch.ldexp(w, (-x)[..., None].to(torch.float32))
    codes = scaled.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(n, k)
    return codes.contiguous().view(torch.int32), (x + 127).to(torch.uint8).contiguous()


def dequantize_mxfp8(words: torch.Tensor, scales: torch.Tensor, *, transposed: bool = False,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """mxfp8 weight -> bf16 ``(out, in)``, exactly: ``words`` ``(out, in / 4)``, or with
    ``transposed`` the pretransposed ``(in, out / 4)`` packing of ``weight.T``."""
    rows, cols = int(words.shape[0]), int(words.shape[1]) * 4
    n, k = (cols, rows) if transposed else (rows, cols)
    out = _out_buffer(out, n, k, words.device)
    _lib.launch_dequant_mxfp8(words.contiguous(), scales.contiguous(), out, n=n, k=k, transposed=transposed)
    return out


def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """float32 -> E2M1 codes (int64): the round-to-nearest-even decision boundaries of the grid
    0, 0.5, 1, 1.5, 2, 3, 4, 6 (ties to the even mantissa), saturated at 6, sign in bit 3; NaN -> 0."""
    a = torch.nan_to_num(x.abs(), nan=0.0)
    code = ((a > 0.25).long() + (a >= 0.75).long() + (a > 1.25).long() + (a >= 1.75).long() + (a > 2.5).long()
            + (a >= 3.5).long() + (a > 5.0).long())
    return code | ((torch.signbit(x) & ~torch.isnan(x)).long() << 3)


def quantize_fp4(weight: torch.Tensor, mode: str = "mxfp4") -> tuple[torch.Tensor, torch.Tensor]:
    """``(out, in)`` weight -> FP4 ``(words (out, in / 8) int32, scales (out, in / G) uint8)``:
    ``mode`` ``"mxfp4"`` (G = 32, E8M0 scales) or ``"nvfp4"`` (G = 16, E4M3 scales). On the GPU:
    the quantize-on-load kernel (``kx_quantize_fp4_bf16``) on the bf16 weight; a host weight is
    converted by the same arithmetic in torch (bit-identical on bf16 weights, tested)."""
    if mode not in FP4_MODES:
        raise ValueError(f"quantize_fp4 takes mode mxfp4 or nvfp4, got {mode}")
    group = _DEFAULTS[mode][0]
    n, k = (int(v) for v in weight.shape)
    if k % group:
        raise ValueError(f"{mode} groups the last axis by {group}: cannot quantize a {n} x {k} matrix")
    kind = _lib.KX_FP4_NV if mode == "nvfp4" else _lib.KX_FP4_MX
    if weight.is_cuda:
        w = weight.to(torch.bfloat16)
        if w.stride(-1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
            w = w.contiguous()
        words = torch.empty((n, k // 8), dtype=torch.int32, device=w.device)
        scales = torch.empty((n, k // group), dtype=torch.uint8, device=w.device)
        if n:
            _lib.launch_quantize_fp4(w, words, scales, group_size=group, scale_kind=kind)
        return words, scales
    w = weight.to(torch.bfloat16).float().reshape(n, k // group, group)
    amax = w.abs().amax(dim=-1)
    if mode == "nvfp4":
        sc = (amax / 6.0).clamp(max=448.0).to(torch.float8_e4m3fn)
        sbytes = sc.view(torch.uint8) & 0x7F
        s = sc.float().abs()
        codes = torch.where(s[..., None] > 0, _e2m1_codes(w / s[..., None]), torch.zeros_like(w, dtype=torch.int64))
    else:
        _, e = torch.frexp(amax)
        x = torch.where(amax > 0, (e.to(torch.int64) - 3).clamp(-127, 127), torch.full_like(e, -127, dtype=torch.int64))
        codes = _e2m1_codes(torch.ldexp(w, (-x)[..., None].to(torch.float32)))
        sbytes = (x + 127).to(torch.uint8)
    return pack(codes.reshape(n, k), 4), sbytes.contiguous()


def dequantize_fp4(words: torch.Tensor, scales: torch.Tensor, mode: str = "mxfp4", *,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """FP4 weight -> bf16 ``(out, in)``, exactly (``kx_dequant_fp4_bf16``)."""
    if mode not in FP4_MODES:
        raise ValueError(f"dequantize_fp4 takes mode mxfp4 or nvfp4, got {mode}")
    group = _DEFAULTS[mode][0]
    n, k = int(words.shape[0]), int(words.shape[1]) * 8
    out = _out_buffer(out, n, k, words.device)
    _lib.launch_dequant_fp4(words.contiguous(), scales.contiguous(), out, n=n, k=k, group_size=group,
                            scale_kind=_lib.KX_FP4_NV if mode == "nvfp4" else _lib.KX_FP4_MX)
    return out


def tile_weights(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *,
                 bits: int = DEFAULT_BITS, group_size: int = DEFAULT_GROUP_SIZE) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed affine weights -> the kernel's tiled layout ``(wt, sbt)`` (uint8 tensors)."""
    _check_format(group_size, bits)
    n = int(words.shape[0])
    k = int(words.shape[1]) * 32 // bits
    if k % 128:
        raise ValueError("the tiled quantized layout needs an input width that is a multiple of 128")
    npad = (n + 255) // 256 * 256
    wt = torch.empty(npad * k * bits // 8, dtype=torch.uint8, device=words.device)
    sbt = torch.empty(npad * (k // 128) * 8, dtype=torch.uint8, device=words.device)
    _lib.launch_tile_weights(words.contiguous(), scales.contiguous(), biases.contiguous(), wt, sbt, n=n, k=k,
                             group_size=group_size, bits=bits)
    return wt, sbt


def _prepare_call(value, n, k, bias, activation, residual, gate, out_dtype, out=None):
    """Shared argument handling of the reference-layout and tiled-layout products."""
    if value.dtype != torch.bfloat16:
        raise ValueError(f"quantized_matmul takes bfloat16 activations on MI355X, got {value.dtype}")
    if int(value.shape[-1]) != k:
        raise ValueError(f"input width {value.shape[-1]} does not match the packed width {k}")
    a = value.reshape(-1, k)
    if a.stride(-1) != 1 or a.data_ptr() % 16 or a.stride(0) % 8:
        a = a.contiguous()
    if out is None:
        out = torch.empty((*value.shape[:-1], n), dtype=out_dtype or value.dtype, device=value.device)
    elif out.shape[-1] != n or out.numel() != a.shape[0] * n:
        raise ValueError(f"out must hold {a.shape[0]} rows of width {n}")
    flags = ACTIVATIONS[activation]
    if bias is not None:
        flags |= _lib.EPI_BIAS
        bias = bias.to(torch.bfloat16).contiguous()
    resid2 = gate32 = None
    if residual is not None:
        flags |= _lib.EPI_GATED_RESIDUAL
        resid2 = residual.reshape(-1, n)
        gate32 = gate.float()
        if gate32.stride(-1) != 1 or gate32.data_ptr() % 16:
            gate32 = gate32.contiguous()
    return a, out, flags, bias, resid2, gate32


def quantized_matmul(
    value: torch.Tensor,
    weight: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor,
    *,
    transpose: bool = True,
    group_size: int = DEFAULT_GROUP_SIZE,
    bits: int = DEFAULT_BITS,
    mode: str = "affine",
    bias: torch.Tensor | None = None,
    activation: str | None = None,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``value @ dequant(weight)^T (+ bias)`` with dequantization inside the MFMA mainloop;
    ``activation``/``residual``/``gate``/``out``/``out_dtype`` as ``mpp_linear.fused_linear``.
    ``mode="mxfp8"`` takes ``biases=None``; with ``transpose=False`` (mxfp8 only: the packing of
    ``weight.T``) the weight is dequantized for the call and multiplied by the dense GEMM."""
    _check_mode(mode, group_size, bits)
    if mode in FP4_MODES:
        # no in-mainloop FP4 product: the exact dequantization, then the dense GEMM
        from .mpp_linear import fused_linear

        if biases is not None or not transpose:
            raise ValueError(f"{mode} weights carry no biases and take the (out, in) packing")
        n, k = int(weight.shape[0]), int(weight.shape[1]) * 8
        dense = dequantize_fp4(weight, scales, mode, out=dequant_workspace(n, k, value.device))
        return fused_linear(value, dense, None if bias is None else bias.to(torch.bfloat16), activation=activation,
                            residual=residual, gate=gate, out=out, out_dtype=out_dtype)
    if mode == "mxfp8":
        if biases is not None:
            raise ValueError("mxfp8 weights carry no biases")
        if not transpose:
            from .mpp_linear import fused_linear

            n, k = int(weight.shape[1]) * 4, int(weight.shape[0])
            dense = dequantize_mxfp8(weight, scales, transposed=True, out=dequant_workspace(n, k, value.device))
            return fused_linear(value, dense, None if bias is None else bias.to(torch.bfloat16), activation=activation,
                                residual=residual, gate=gate, out=out, out_dtype=out_dtype)
        n = int(weight.shape[0])
        k = int(weight.shape[1]) * 4
        a, out, flags, bias, resid2, gate32 = _prepare_call(value, n, k, bias, activation, residual, gate,
                                                            out_dtype, out)
        if a.shape[0]:
            _lib.launch_qgemm_mxfp8(a, weight, scales, out.view(-1, n), n=n, k=k, bias=bias, flags=flags,
                                    resid=resid2, gate=gate32)
        return out
    if not transpose:
        raise ValueError("the MI355X affine quantized linear takes the (out, in) packing (transpose=True)")
    n = int(weight.shape[0])
    k = int(weight.shape[1]) * 32 // bits
    if scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError("scales and biases must be (out, in / group_size)")
    a, out, flags, bias, resid2, gate32 = _prepare_call(value, n, k, bias, activation, residual, gate, out_dtype,
                                                        out)
    if a.shape[0] == 0:
        return out
    _lib.launch_qgemm(
        a, weight, scales, biases, out.view(-1, n), n=n, k=k, group_size=group_size, bits=bits,
        bias=bias, flags=flags, resid=resid2, gate=gate32,
    )
    return out


# One dequantization buffer per (device, stream), grown to the largest quantized weight called on
# it and kept: each GPU call of a quantized layer writes its bf16 weight there and the dense GEMM
# reads it, so a block's calls reuse one allocation (134 MB for the LTX-2 feed-forward weights)
# instead of taking a new one from the caching allocator per call. Calls on one stream run in
# order, so a call's dequantization never overwrites a weight that an earlier GEMM still reads.
_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}


def dequant_workspace(n: int, k: int, device: torch.device) -> torch.Tensor:
    """A bf16 ``(n, k)`` view of the current stream's dequantization buffer on ``device``."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch.cuda.current_stream(index).cuda_stream)
    buf = _WORKSPACE.get(key)
    if buf is None or buf.numel() < n * k:
        buf = torch.empty(n * k, dtype=torch.bfloat16, device=torch.device("cuda", index))
        _WORKSPACE[key] = buf
    return buf[: n * k].view(n, k)


class QuantizedLinear:
    """``nn.QuantizedLinear`` counterpart: packed affine weight with bf16 scales/biases, or an
    mxfp8 weight with uint8 scales (``biases`` None); optional bf16 bias;
    ``layer(x) = quantized_matmul(x, ...) + bias`` (bias fused in the epilogue)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None,
                 bias: torch.Tensor | None = None, *, group_size: int | None = None,
                 bits: int | None = None, mode: str = "affine") -> None:
        group_size, bits = quant_defaults(mode, group_size, bits)
        _check_mode(mode, group_size, bits)
        if (biases is None) != (mode in SCALED_MODES):
            raise ValueError("affine weights carry biases and mxfp8 / mxfp4 / nvfp4 weights none")
        # the kernels reinterpret the scale bits: bf16 scale / bias pairs (affine), scale bytes
        # (mxfp8 / mxfp4: E8M0, nvfp4: E4M3)
        if mode in SCALED_MODES and scales.dtype != torch.uint8:
            raise ValueError(f"{mode} scales must be uint8 bytes, got {scales.dtype}")
        if mode == "affine" and (scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16):
            raise ValueError(f"affine scales and biases must be bfloat16, got {scales.dtype} and {biases.dtype}")
        self.weight = weight
        self.scales = scales
        self.biases = biases
        self.bias = bias
        self.group_size = group_size
        self.bits = bits
        self.mode = mode
        # layers of at most 64 outputs (the gate logits) keep their weight dequantized once, by the
        # bit-exact dequantization kernel, and run the memory-bound dense GEMV: per-lane
        # dequantization from global memory made that GEMV latency-bound
        self._dense = None
        if weight.is_cuda and int(weight.shape[0]) <= 64:
            self._dense = self.dequantized()

    def dequantized(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """The bf16 ``(out, in)`` weight, exactly (a new buffer, or ``out``)."""
        if self.mode == "mxfp8":
            return dequantize_mxfp8(self.weight, self.scales, out=out)
        if self.mode in FP4_MODES:
            return dequantize_fp4(self.weight, self.scales, self.mode, out=out)
        return dequantize(self.weight, self.scales, self.biases, group_size=self.group_size, bits=self.bits,
                          out=out)

    @classmethod
    def from_linear(cls, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                    group_size: int | None = None, bits: int | None = None,
                    mode: str = "affine") -> "QuantizedLinear":
        group_size, bits = quant_defaults(mode, group_size, bits)
        if mode == "mxfp8":
            _check_mode(mode, group_size, bits)
            words, scales = quantize_mxfp8(weight, group_size)
            return cls(words, scales, None, bias, group_size=group_size, bits=bits, mode=mode)
        if mode in FP4_MODES:
            _check_mode(mode, group_size, bits)
            words, scales = quantize_fp4(weight, mode)
            return cls(words, scales, None, bias, group_size=group_size, bits=bits, mode=mode)
        words, scales, biases = quantize(weight, group_size, bits)
        return cls(words, scales, biases, bias, group_size=group_size, bits=bits)

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[1]) * 32 // self.bits

    def __call__(self, value: torch.Tensor, *, activation: str | None = None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if self.weight.is_cuda and value.is_cuda:
            from .mpp_linear import fused_linear

            if int(value.shape[-1]) != self.in_features:
                raise ValueError(f"input width {value.shape[-1]} does not match the packed width {self.in_features}")
            weight = self._dense
            if weight is None:
                weight = self.dequantized(dequant_workspace(self.out_features, self.in_features, value.device))
            bias = None if self.bias is None else self.bias.to(torch.bfloat16)
            return fused_linear(value, weight, bias, activation=activation, residual=residual, gate=gate,
                                out=out, out_dtype=out_dtype)
        return quantized_matmul(
            value, self.weight, self.scales, self.biases, group_size=self.group_size,
            bits=self.bits, mode=self.mode, bias=self.bias, activation=activation,
            residual=residual, gate=gate, out=out, out_dtype=out_dtype,
        )


class PretransposedQuantizedLinear:
    """``_PretransposedQuantizedLinear`` counterpart (``quantization.py:17-44``): an mxfp8 weight
    packed from ``weight.T`` (words ``(in, out / 4)``, scales ``(in, out / 32)``), multiplied as
    ``mx.quantized_matmul(x, w, scales, transpose=False) + bias``. Its groups run along the output
    axis, so it is dequantized once, exactly, to the bf16 ``(out, in)`` weight, and each call is
    the dense GEMM with the bias (and any activation / gated residual) in its epilogue."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None, *,
                 group_size: int | None = None, bits: int | None = None, mode: str = "mxfp8") -> None:
        group_size, bits = quant_defaults(mode, group_size, bits)
        if mode != "mxfp8":
            raise NotImplementedError(f"pretransposed {mode} weights have no MI355X path (mxfp8 does)")
        _check_mode(mode, group_size, bits)
        self.weight = weight
        self.scales = scales
        self.bias = bias
        self.group_size = group_size
        self.bits = bits
        self.mode = mode
        self._dense = dequantize_mxfp8(weight, scales, transposed=True) if weight.is_cuda else None

    @classmethod
    def from_linear(cls, weight: torch.Tensor, bias: torch.Tensor | None = None) -> "PretransposedQuantizedLinear":
        """Pack ``weight.T`` as the reference's ``mxfp8-blocks-pretranspose`` preparation does
        (``preparation.py:139-157``)."""
        words, scales = quantize_mxfp8(weight.t().contiguous())
        return cls(words, scales, bias)

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[1]) * 4

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[0])

    def __call__(self, value: torch.Tensor, *, activation: str | None = None,
                 residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        from .mpp_linear import fused_linear

        if self._dense is None:
            raise RuntimeError("the pretransposed quantized linear runs on the GPU: move its weight to cuda first")
        bias = None if self.bias is None else self.bias.to(torch.bfloat16)
        return fused_linear(value, self._dense, bias, activation=activation, residual=residual, gate=gate, out=out,
                            out_dtype=out_dtype)


__all__ = [
    "FP4_MODES",
    "KERNEL_MODES",
    "PretransposedQuantizedLinear",
    "QuantizedLinear",
    "dequant_workspace",
    "dequantize",
    "dequantize_fp4",
    "dequantize_mxfp8",
    "pack",
    "quant_defaults",
    "quantize",
    "quantize_fp4",
    "quantize_mxfp8",
    "quantized_matmul",
    "tile_weights",
    "unpack",
]
