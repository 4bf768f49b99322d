"""LTX-2 GELU feed-forward on MI355X (mirror of
``kinomlx/models/ltx2/transformer/feed_forward.py``).

``project_out(gelu_approx(project_in(x)))`` with the tanh GELU computed in the up-projection
GEMM's epilogue (FP32, clamped inner argument) — the ``(T, 4D)`` activation is written once,
already activated, instead of being written, read, activated and written again.
"""

from __future__ import annotations

import torch

from .attention import Linear


class GELUApprox:
    """Input projection followed by approximate GELU (``feed_forward.py:11-34``)."""

    def __init__(self, dim_in: int, dim_out: int, *, bias: bool = True) -> None:
        self.dim_in = dim_in
        self.dim_out = dim_out
        self.bias = bias
        self.proj: Linear | None = None

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        if value.shape[-1] != self.dim_in:
            raise ValueError(f"GELU projection expects width {self.dim_in}, got {value.shape[-1]}")
        out = self.proj(value, activation="gelu_tanh")
        if out.shape[-1] != self.dim_out:
            raise ValueError(f"GELU projection produced width {out.shape[-1]}, expected {self.dim_out}")
        return out


class FeedForward:
    """Linear-GELU-linear MLP (``feed_forward.py:37-97``)."""

    def __init__(self, dim: int, *, dim_out: int | None = None, mult: int = 4, bias: bool = True) -> None:
        if mult <= 0:
            raise ValueError("feed-forward multiplier must be positive")
        self.dim = dim
        self.output_dim = dim if dim_out is None else dim_out
        self.inner_dim = dim * mult
        self.project_in = GELUApprox(dim, self.inner_dim, bias=bias)
        self.project_out: Linear | None = None

    def __call__(self, value: torch.Tensor, *, residual: torch.Tensor | None = None,
                 gate: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """``project_out(gelu(project_in(x)))``; with ``residual``/``gate`` the block's gated
        residual is formed in the down-projection's epilogue (``out_dtype`` as ``Attention``)."""
        if value.shape[-1] != self.dim:
            raise ValueError(f"feed-forward expects width {self.dim}, got {value.shape[-1]}")
        hidden = self.project_in(value)
        out = self.project_out(hidden, residual=residual, gate=gate, out_dtype=out_dtype)
        if out.shape[-1] != self.output_dim:
            raise ValueError(f"feed-forward produced width {out.shape[-1]}, expected {self.output_dim}")
        return out


__all__ = ["FeedForward", "GELUApprox"]
