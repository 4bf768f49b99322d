"""The FP32 torch block reference used at full size is pinned against the numpy oracle. CPU."""

import numpy as np
import torch

import oracle
from kinomlx_amd import workloads
from tests import _torch_ref
from tests._blocks import ltx_case
from tests.conftest import max_abs


def test_torch_reference_matches_oracle_ltx_block():
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    p, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
    got = _torch_ref.ltx_video_block(tp, torch.from_numpy(x), torch.from_numpy(ctx),
                                     tuple(torch.from_numpy(t) for t in pe), heads=2).numpy()
    assert max_abs(got, ref) < 1e-4


def test_torch_reference_bf16_graph_matches_oracle_bf16_graph():
    """Both restatements of the reference's bf16 execution round at the same points: they agree
    up to rare one-ulp rounding flips, far below the bf16 graph's own error against FP32."""
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    p, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    fp32 = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=2, bf16_graph=True)
    tp = {k: torch.from_numpy(np.asarray(v)) for k, v in op.items()}
    got = _torch_ref.ltx_video_block(tp, torch.from_numpy(x), torch.from_numpy(ctx),
                                     tuple(torch.from_numpy(t) for t in pe), heads=2, bf16_graph=True).numpy()
    assert np.mean(got == ref) > 0.95
    assert max_abs(got, ref) < 0.5 * max_abs(ref, fp32)


def test_bf16_graph_rounds_every_output_and_stays_close_to_fp32():
    """The bf16-graph mode returns bf16 values and differs from FP32 by rounding noise only
    (cosine > 0.9999); dropping a rounding point would leave non-bf16 values."""
    spec = workloads.LTXSpec(grid=(2, 3, 4), text_tokens=5, dim=256, heads=2, head_dim=128)
    _, op, inputs, pe = ltx_case(spec)
    x = inputs["x"][0].float().numpy()
    ctx = inputs["context"][0].float().numpy()
    fp32 = oracle.ltx_video_block(op, x, ctx, pe, heads=2)
    graph = oracle.ltx_video_block(op, x, ctx, pe, heads=2, bf16_graph=True)
    assert np.array_equal(graph, oracle.to_bf16(graph))
    assert not np.array_equal(fp32, oracle.to_bf16(fp32))
    cos = float(graph.ravel() @ fp32.ravel() / np.linalg.norm(graph) / np.linalg.norm(fp32))
    assert cos > 0.9999
    assert 0 < max_abs(graph, fp32) < 0.1
