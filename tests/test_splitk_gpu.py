"""Split-K GEMM on the GPU (kx_gemm_splitk_bf16): few-row products with every epilogue against
the FP32 oracle, and the dispatch rule that routes them there."""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import _lib, workloads
from kinomlx_amd.kernels.mpp_linear import fused_linear
from tests.conftest import cosine, max_abs

pytestmark = pytest.mark.gpu


def _bf(shape, seed, std=1.0):
    return workloads.bf16(workloads.normal(seed, "splitk", shape, std))


def test_dispatch_rule():
    assert _lib.splitk_splits(127, 2048, 2048) == 8
    assert _lib.splitk_splits(127, 2048, 8192) == 16
    assert _lib.splitk_splits(9216, 4096, 4096) == 1  # enough tiles
    assert _lib.splitk_splits(127, 32, 4096) == 1      # the skinny kernel's shape
    assert _lib.splitk_splits(127, 2048, 512) == 1     # too little K


@pytest.mark.parametrize("m,n,k", [(127, 2048, 2048), (127, 2048, 8192), (127, 4096, 2048), (200, 1024, 4096)])
@pytest.mark.parametrize("epi", ["plain", "bias_gelu", "gated_f32", "out_f32"])
def test_splitk_matches_oracle(device, m, n, k, epi):
    assert _lib.splitk_splits(m, n, k) > 1
    x, w, b = _bf((m, k), 1), _bf((n, k), 2, 0.02), _bf((n,), 3, 0.02)
    kwargs = {}
    ref = oracle.linear(x.float().numpy(), w.float().numpy(), b.float().numpy() if epi == "bias_gelu" else None)
    if epi == "bias_gelu":
        kwargs = dict(activation="gelu_tanh")
        ref = oracle.gelu_approx(ref)
    if epi == "gated_f32":
        resid = workloads.normal(4, "resid", (m, n))
        gate = workloads.normal(5, "gate", (n,), 0.5)
        kwargs = dict(residual=resid.to(device), gate=gate.to(device), out_dtype=torch.float32)
        ref = resid.numpy() + gate.numpy() * ref
    if epi == "out_f32":
        kwargs = dict(out_dtype=torch.float32)
    got = fused_linear(x.to(device), w.to(device), b.to(device) if epi == "bias_gelu" else None, **kwargs)
    out = got.float().cpu().numpy()
    assert cosine(out, ref) > 0.99999
    bound = 2e-3 if got.dtype == torch.float32 else 2 ** -7 * max(1.0, np.abs(ref).max())
    assert max_abs(out, ref) <= bound, (max_abs(out, ref), bound)
