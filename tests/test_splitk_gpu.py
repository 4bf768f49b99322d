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


@pytest.mark.parametrize("m,n,k", [(4864, 4096, 8192), (4352, 4096, 8192), (6400, 4096, 8192)])
@pytest.mark.parametrize("epi", ["plain", "gated_f32"])
def test_tail_split_matches_oracle(device, m, n, k, epi):
    """A long-K product split into whole rounds of 256x256 tiles plus K slices of the tail rows
    (768 tail rows take the 256x256 slices, 256 tail rows the small-M slices, 2304 tail rows over
    half a round take 8 slices in 5 rounds): the head rows, the rows either side of the split and
    every tail row against the FP32 oracle."""
    rows, splits = _lib.tail_split(m, n, k)
    x, w = _bf((m, k), 11), _bf((n, k), 12, 0.02)
    sample = np.r_[0:64, rows - 64:m]
    ref = oracle.linear(x[sample].float().numpy(), w.float().numpy())
    kwargs = {}
    if epi == "gated_f32":
        resid = workloads.normal(13, "resid", (m, n))
        gate = workloads.normal(14, "gate", (n,), 0.5)
        kwargs = dict(residual=resid.to(device), gate=gate.to(device), out_dtype=torch.float32)
        ref = resid[sample].numpy() + gate.numpy() * ref
    timer = _lib.LaunchTimer()
    _lib.set_timer(timer)
    try:
        got = fused_linear(x.to(device), w.to(device), None, **kwargs)
    finally:
        _lib.set_timer(None)
    launches = [(name, args) for name, args, _ in timer.durations_ms()]
    # the tail's K slices first (its rows are the input's most recently written), then the head
    assert [name for name, _ in launches] == ["kx_gemm_splitk_bf16", "kx_gemm_bf16"]
    assert launches[1][1][7] == rows and launches[0][1][7] == m - rows and launches[0][1][18] == splits
    out = got.float().cpu().numpy()[sample]
    assert cosine(out, ref) > 0.99999
    bound = 2e-3 if got.dtype == torch.float32 else 2 ** -7 * max(1.0, np.abs(ref).max())
    assert max_abs(out, ref) <= bound, (max_abs(out, ref), bound)


def test_tail_split_keeps_plain_tiling_for_a_per_batch_gate(device):
    """A gate that changes with the row block indexes rows from the product's first row: such a
    product keeps the one plain launch."""
    m, n, k = 4864, 4096, 8192
    x, w = _bf((m, k), 15), _bf((n, k), 16, 0.02)
    resid = workloads.normal(17, "resid", (2, m // 2, n)).to(device)
    gate = workloads.normal(18, "gate", (2, 1, n), 0.5).to(device)
    timer = _lib.LaunchTimer()
    _lib.set_timer(timer)
    try:
        got = fused_linear(x.view(2, m // 2, k).to(device), w.to(device), None, residual=resid, gate=gate,
                           out_dtype=torch.float32)
    finally:
        _lib.set_timer(None)
    assert [name for name, _, _ in timer.durations_ms()] == ["kx_gemm_bf16"]
    sample = np.r_[0:32, m // 2 - 32:m // 2 + 32, m - 32:m]
    ref = oracle.linear(x[sample].float().numpy(), w.float().numpy())
    g = gate.cpu().numpy()[np.where(sample < m // 2, 0, 1), 0]
    ref = resid.view(m, n)[sample].cpu().numpy() + g * ref
    out = got.view(m, n).float().cpu().numpy()[sample]
    assert max_abs(out, ref) <= 2e-3, max_abs(out, ref)


def test_tail_split_of_a_batched_input_equals_the_flat_product(device):
    """A 3-D ``(B, T, K)`` input whose flattened rows take the tail split: the tail's first row is
    found from the flattened row stride, not the batch axis, so the result equals the 2-D product
    bit for bit."""
    m, n, k = 4864, 4096, 8192
    assert _lib.tail_split(m, n, k) is not None
    x, w = _bf((m, k), 19), _bf((n, k), 20, 0.02)
    resid = workloads.normal(21, "resid", (m, n)).to(device)
    gate = workloads.normal(22, "gate", (n,), 0.5).to(device)
    xd, wd = x.to(device), w.to(device)
    flat = fused_linear(xd, wd, None, residual=resid, gate=gate, out_dtype=torch.float32)
    batched = fused_linear(xd.view(2, m // 2, k), wd, None, residual=resid.view(2, m // 2, n), gate=gate,
                           out_dtype=torch.float32)
    assert batched.shape == (2, m // 2, n)
    assert torch.equal(batched.view(m, n), flat)


def test_input_above_the_cache_size_is_tiled_newest_rows_first(device):
    """An input over 128 MiB (here 9216 x 8192 bf16, 151 MB) makes the kernel visit its tile rows
    last to first; the tile order changes no result: the first, middle and last rows against the
    FP32 oracle, and the whole product bit-equal to the same rows computed in two halves (each
    under the size, so in the ascending order)."""
    m, n, k = 9216, 512, 8192
    assert m * k * 2 > 128 << 20 and (m // 2) * k * 2 <= 128 << 20
    x, w = _bf((m, k), 21), _bf((n, k), 22, 0.02)
    xd, wd = x.to(device), w.to(device)
    got = fused_linear(xd, wd, None)
    halves = torch.cat([fused_linear(xd[: m // 2], wd, None), fused_linear(xd[m // 2:], wd, None)])
    assert torch.equal(got, halves)
    sample = np.r_[0:64, m // 2 - 32:m // 2 + 32, m - 64:m]
    ref = oracle.linear(x[sample].float().numpy(), w.float().numpy())
    out = got.float().cpu().numpy()[sample]
    assert cosine(out, ref) > 0.99999 and max_abs(out, ref) <= 2 ** -7 * max(1.0, np.abs(ref).max())
