"""Dense bf16 / fp16 linear products on gfx950 MFMA, behind the reference's ``mpp_linear`` surface.

Mirror of ``kinomlx/kernels/mpp_linear.py`` (``linear``, ``applies``, ``supports``,
``available``, ``prepare``, ``restore``, ``fp16_operand``, ``Operand``, ``set_enabled``,
``enabled``, ``linear_rows``), computing ``addmm(bias, x, W^T)``: FP32 accumulation in
``v_mfma_f32_32x32x16_bf16`` (``_f16`` for float16 operands, the reference's ``half`` MPP GEMMs,
``mpp_linear.py:145-294``), bias added in FP32, one rounding to the input's type
(``mpp_linear.py:1-6``).

MI355X has native bf16 MFMA, so the M1's scaled-FP16 operand conversion has no counterpart:
``fp16_operand``/``prepare`` return the operand unchanged (``Operand(values, None)``) and
``restore`` gives the weight back. ``prepare`` of an ``(in, out)`` weight (``transposed=False``)
stores the ``(out, in)`` copy the kernel reads, so later calls skip the transpose.

``fused_linear`` exposes the kernel's epilogues (activation, gated residual) to the block code:
``c = residual + gate * act(x W^T + bias)`` in one pass.
"""

from __future__ import annotations

from math import prod
from typing import NamedTuple

import torch

from .. import _lib

MIN_ROWS = 1
MIN_WIDTH = 8
_DTYPES = (torch.bfloat16, torch.float16)
_enabled = True

ACTIVATIONS = {
    None: 0,
    "gelu_tanh": _lib.EPI_ACT_GELU_TANH,
    "silu": _lib.EPI_ACT_SILU,
    "sigmoid2": _lib.EPI_ACT_SIGMOID2,
    "sigmoid": _lib.EPI_ACT_SIGMOID,
}


class Operand(NamedTuple):
    """The values ``linear`` multiplies for one operand; ``peak`` is always None on MI355X (no
    scaled-FP16 conversion), kept for the reference's signature."""

    values: torch.Tensor
    peak: torch.Tensor | None


def set_enabled(enabled: bool) -> None:
    """Use the MFMA kernel wherever it applies (the default)."""
    global _enabled
    _enabled = bool(enabled)


def enabled() -> bool:
    """Whether the MFMA products are switched on."""
    return _enabled


def supports(rows: int, k: int, n: int, *, transposed: bool, dtype: torch.dtype) -> bool:
    """Whether the kernel computes a ``rows x k`` by ``k x n`` product: bf16 or fp16, ``k`` a
    multiple of 8 (16-byte rows), 32-bit counts."""
    del transposed
    return (
        dtype in _DTYPES and rows >= MIN_ROWS and n >= 1 and k >= MIN_WIDTH and k % 8 == 0
        and rows < 2**31 and n < 2**31 and k < 2**30
    )


def available(*, transposed: bool, bias: bool, dtype: torch.dtype = torch.bfloat16) -> bool:
    """Whether the kernel is built, a GPU is visible and the dtype is supported."""
    del transposed, bias
    return dtype in _DTYPES and _lib.available()


def _weight(weight: torch.Tensor | Operand) -> torch.Tensor:
    return weight.values if isinstance(weight, Operand) else weight


def applies(value: torch.Tensor, weight: torch.Tensor | Operand, bias: torch.Tensor | None, *,
            transposed: bool) -> bool:
    """Whether ``linear`` computes this product (contract of ``mpp_linear.py:455-466``)."""
    array = _weight(weight)
    if not _enabled or value.dim() < 2 or array.dim() != 2:
        return False
    dtype = value.dtype
    if dtype not in _DTYPES or array.dtype != dtype:
        return False
    k = int(value.shape[-1])
    n, inner = (int(s) for s in (array.shape if transposed else array.shape[::-1]))
    if inner != k:
        return False
    if bias is not None and (bias.dtype != dtype or bias.dim() != 1 or int(bias.shape[0]) != n):
        return False
    rows = prod(int(s) for s in value.shape[:-1])
    return supports(rows, k, n, transposed=transposed, dtype=dtype) and available(
        transposed=transposed, bias=bias is not None, dtype=dtype
    )


def fp16_operand(value: torch.Tensor) -> Operand:
    """The operand as the kernel multiplies it: unchanged (bf16 and fp16 are native on MI355X)."""
    return Operand(value, None)


def prepare(weight: torch.Tensor, *, transposed: bool = True) -> Operand:
    """The weight as the kernel reads it: ``(out, in)`` contiguous rows."""
    values = weight if transposed else weight.t()
    return Operand(values.contiguous(), None)


def restore(prepared: Operand) -> torch.Tensor:
    """The ``(out, in)`` weight a prepared operand holds."""
    return prepared.values


def _as_out_in(weight: torch.Tensor | Operand, transposed: bool) -> torch.Tensor:
    if isinstance(weight, Operand):
        return weight.values
    w = weight if transposed else weight.t()
    if w.stride(-1) != 1 or w.data_ptr() % 16 or w.stride(0) % 8:
        w = w.contiguous()
    return w


def _rows_view(value: torch.Tensor) -> torch.Tensor:
    v = value.reshape(-1, value.shape[-1]) if value.dim() != 2 else value
    if v.stride(-1) != 1 or v.data_ptr() % 16 or v.stride(0) % 8:
        v = v.contiguous()
    return v


def fused_linear(
    value: torch.Tensor,
    weight: torch.Tensor | Operand,
    bias: torch.Tensor | None = None,
    *,
    activation: str | None = None,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``residual + gate * act(value @ W^T + bias)`` in one MFMA pass (``(out, in)`` weight).

    ``gate`` is an fp32 row vector ``(n,)``, one per batch ``(B, 1, n)`` or per row; without
    ``residual`` the epilogue stops after the activation. ``residual`` may be of the input's
    16-bit type or fp32 and the output (``out_dtype``, default the input dtype) likewise: a
    residual stream can be carried in fp32 between blocks' branches so that it is rounded once, not
    once per add.
    """
    w = _as_out_in(weight, True)
    dtype = value.dtype
    if dtype not in _DTYPES or w.dtype != dtype:
        raise ValueError(f"the MFMA linear multiplies float16 or bfloat16 inputs by weights of that dtype, "
                         f"got {dtype}, {w.dtype}")
    n, k = (int(s) for s in w.shape)
    if int(value.shape[-1]) != k:
        raise ValueError(f"linear input width {value.shape[-1]} does not match weight width {k}")
    a = _rows_view(value)
    if out is None:
        out = torch.empty((*value.shape[:-1], n), dtype=out_dtype or dtype, device=value.device)
    if a.shape[0] == 0:
        return out
    flags = ACTIVATIONS[activation]
    if bias is not None:
        if bias.dtype != dtype or bias.shape != (n,):
            raise ValueError(f"bias must be {dtype} of shape ({n},)")
        flags |= _lib.EPI_BIAS
        bias = bias.contiguous()
    resid2 = None
    gate32 = None
    if residual is not None:
        if gate is None:
            raise ValueError("a gated residual needs a gate")
        flags |= _lib.EPI_GATED_RESIDUAL
        resid2 = residual.reshape(-1, n)
        gate32 = gate.float()
        if gate32.stride(-1) != 1 or gate32.data_ptr() % 16:
            gate32 = gate32.contiguous()
    out2 = out.view(-1, n)  # a view: a strided `out` is written in place, never via a copy
    _lib.launch_gemm(a, w, out2, bias=bias, flags=flags, resid=resid2, gate=gate32)
    return out


def linear(
    value: torch.Tensor,
    weight: torch.Tensor | Operand,
    bias: torch.Tensor | None,
    *,
    transposed: bool,
    operand: Operand | None = None,
) -> torch.Tensor:
    """``addmm(bias, value, weight.T)`` for an ``(out, in)`` weight with ``transposed``, or
    ``addmm(bias, value, weight)`` for an ``(in, out)`` weight (``mpp_linear.py:469-506``)."""
    dtype = value.dtype
    array = _weight(weight)
    if array.dtype != dtype:
        raise ValueError(f"the MFMA linear multiplies a {dtype} input by a weight of that dtype, not {array.dtype}")
    k = int(value.shape[-1])
    n = int(array.shape[0] if (transposed or isinstance(weight, Operand)) else array.shape[1])
    rows = prod(int(s) for s in value.shape[:-1])
    if not supports(rows, k, n, transposed=transposed, dtype=dtype):
        raise ValueError(f"the MFMA linear does not take a {rows} x {k} by {k} x {n} {dtype} product")
    if operand is not None and operand.values.shape != value.shape:
        raise ValueError("operand must be fp16_operand(value)")
    w = weight if isinstance(weight, Operand) else _as_out_in(weight, transposed)
    return fused_linear(value, w, bias)


def linear_rows(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """``residual + addmm(bias, value, weight.T)`` for ``(rows, k)`` rows and an ``(n, k)``
    weight; any row count (``mpp_linear.py:593-613``). The residual is added after the
    product's rounding, as a separate addition would."""
    product = fused_linear(value, weight, bias)
    if residual is None:
        return product
    if residual.shape != product.shape:
        raise ValueError("residual must match the product's shape")
    ones = torch.ones(product.shape[-1], dtype=torch.float32, device=product.device)
    return _residual_add(residual, product, ones)


def _residual_add(base: torch.Tensor, addend: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    out = torch.empty(base.shape, dtype=base.dtype, device=base.device)
    _lib.launch_gated_residual(base, addend, out, gate)
    return out


__all__ = [
    "ACTIVATIONS",
    "MIN_ROWS",
    "MIN_WIDTH",
    "Operand",
    "applies",
    "available",
    "enabled",
    "fp16_operand",
    "fused_linear",
    "linear",
    "linear_rows",
    "prepare",
    "restore",
    "set_enabled",
    "supports",
]
