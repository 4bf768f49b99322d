"""The no-allocation split-K entry point (kx_gemm_splitk_noalloc_bf16) through the C ABI: its
output equals kx_gemm_splitk_bf16's (caller workspace) bit for bit, on two calls in a row with the
second smaller (the static scratch keeps the first call's partial products), with and without an
epilogue; sizes beyond the static scratch are refused before any GPU work."""

import ctypes

import pytest
import torch

from kinomlx_amd import _lib, workloads

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _bf(shape, seed, std=1.0):
    return workloads.bf16(workloads.normal(seed, "noalloc", shape, std))


def _run(name, x, w, out, splits, *, bias=None, flags=0, resid=None, gate=None, workspace=None):
    m, k = x.shape
    n = w.shape[0]
    args = [x.data_ptr(), k, w.data_ptr(), k, None if bias is None else bias.data_ptr(), out.data_ptr(), n, m, n, k,
            flags, None if resid is None else resid.data_ptr(), 0 if resid is None else n,
            None if gate is None else gate.data_ptr(), 1, 0]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel() * 4]
    args += [splits, torch.cuda.current_stream().cuda_stream]
    rc = getattr(_lib.load(), name)(*args)
    assert rc == _lib.KX_OK, _lib.load().kx_last_error().decode()


def _pair(device, m, n, k, epilogue):
    splits = _lib.splitk_splits(m, n, k)
    assert splits > 1
    x, w = _bf((m, k), 1).to(device), _bf((n, k), 2, 0.02).to(device)
    kw = {}
    out_dtype = torch.bfloat16
    if epilogue:
        kw = dict(bias=_bf((n,), 3, 0.02).to(device),
                  resid=workloads.normal(4, "resid", (m, n)).to(device),
                  gate=workloads.normal(5, "gate", (n,), 0.5).to(device),
                  flags=_lib.EPI_BIAS | _lib.EPI_GATED_RESIDUAL | _lib.EPI_RESID_F32 | _lib.EPI_OUT_F32)
        out_dtype = torch.float32
    ref = torch.full((m, n), float("nan"), dtype=out_dtype, device=device)
    got = torch.full((m, n), float("nan"), dtype=out_dtype, device=device)
    work = torch.empty(splits * m * n, dtype=torch.float32, device=device)
    _run("kx_gemm_splitk_bf16", x, w, ref, splits, workspace=work, **kw)
    _run("kx_gemm_splitk_noalloc_bf16", x, w, got, splits, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("epilogue", [False, True])
def test_noalloc_matches_workspace_entry_point_twice_in_a_row(device, epilogue):
    # the first call fills more of the scratch than the second reads
    _pair(device, 200, 2048, 4096, epilogue)
    _pair(device, 127, 1024, 2048, epilogue)


def test_noalloc_largest_product_size(device):
    # the largest split-K product the dispatch rule makes still fits the static scratch
    m, n, k = 127, 4096, 4096
    splits = _lib.splitk_splits(m, n, k)
    assert splits * m * n * 4 <= SCRATCH_BYTES
    _pair(device, m, n, k, False)


def test_noalloc_refuses_more_than_the_scratch(device):
    # real, correctly shaped operands: a product whose partial products (2 x 1024 x 4096 fp32 =
    # 32 MiB) exceed the scratch is refused with an error, whatever order the checks run in
    lib = _lib.load()
    m, n, k, splits = 1024, 4096, 4096, 2
    assert splits * m * n * 4 > SCRATCH_BYTES
    x, w = _bf((m, k), 6).to(device), _bf((n, k), 7, 0.02).to(device)
    out = torch.zeros((m, n), dtype=torch.bfloat16, device=device)
    rc = lib.kx_gemm_splitk_noalloc_bf16(x.data_ptr(), k, w.data_ptr(), k, None, out.data_ptr(), n, m, n, k, 0, None,
                                         0, None, 1, 0, splits, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == _lib.KX_ERR_INVALID
    assert "exceeds" in lib.kx_last_error().decode()
    assert not out.any()  # nothing was launched
    assert ctypes.sizeof(ctypes.c_void_p) == 8
