"""Block parity on the GPU: the MI355X LTX-2 video block against the FP32 oracle on the same
seeded inputs, and at the full 9216-token north-star shape against the FP32 torch evaluation of
the same block (pinned to the oracle in ``test_blocks_cpu.py``).

Tolerance (north star): cosine similarity >= 0.9995 and max abs error <= 2e-2 between the bf16
block output and the FP32 evaluation. The absolute bar is met wherever a bf16 output can meet
it; the synthetic D = 4096 blocks reach |y| ~ 26, where one bf16 rounding of the output alone
is worth up to 0.0625 and the reference's own bf16 execution (``oracle.ltx_video_block(...,
bf16_graph=True)``) misses 2e-2 several times over. There the bar is the reference's own error:
max abs error <= max(2e-2, max abs error of the reference's bf16 graph on the same inputs).
"""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.ltx2.transformer import TransformerArgs
from tests import _torch_ref
from tests._blocks import device_tables, ltx_case
from tests.conftest import cosine, max_abs

pytestmark = pytest.mark.gpu

COS_MIN = 0.9995
MAX_ABS = 2e-2


def _check_block(got, ref, graph):
    """cosine >= 0.9995; max abs <= max(2e-2, the reference bf16 graph's own max abs error)."""
    assert np.all(np.isfinite(got))
    c, m, g = cosine(got, ref), max_abs(got, ref), max_abs(graph, ref)
    print(f"cosine {c:.7f} max_abs {m:.4g} (reference bf16 graph {g:.4g}) max|ref| {np.abs(ref).max():.3f}")
    assert c >= COS_MIN, c
    assert m <= max(MAX_ABS, g), (m, g)
    return m, g


def _run_block(spec, p, inputs, pe, device):
    block = workloads.build_ltx_block(spec, p, device)
    args = TransformerArgs(
        x=inputs["x"].to(device), context=inputs["context"].to(device), timesteps=p["timesteps"].to(device),
        positional_embeddings=device_tables(pe, device),
    )
    out, _ = block(args)
    torch.cuda.synchronize()
    return out.x[0].float().cpu().numpy()


@pytest.mark.parametrize(
    "spec",
    [
        workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128),
        workloads.LTXSpec(grid=(2, 4, 16), text_tokens=32, dim=4096, heads=32, head_dim=128),
        workloads.LTXSpec(grid=(3, 5, 7), text_tokens=9, dim=1024, heads=16, head_dim=64),
        workloads.LTXSpec(grid=(2, 4, 16), text_tokens=32, dim=4096, heads=32, head_dim=128, bits=4),
        workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128, bits=8),
    ],
    ids=["d1024", "d4096", "d1024-h64-ragged", "d4096-int4", "d1024-int8"],
)
def test_ltx_block_matches_oracle(device, spec):
    p, op, inputs, pe = ltx_case(spec)
    got = _run_block(spec, p, inputs, pe, device)
    x, ctx = inputs["x"][0].float().numpy(), inputs["context"][0].float().numpy()
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=spec.heads)
    graph = oracle.ltx_video_block(op, x, ctx, pe, heads=spec.heads, bf16_graph=True)
    m, _ = _check_block(got, ref, graph)
    if np.abs(ref).max() < 4.0:
        # outputs below 4: one bf16 rounding is at most 2^-7, so the literal bar applies
        assert m <= MAX_ABS, m


def test_ltx_block_unfused_projections_agree_with_fused(device):
    spec = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
    p, _, inputs, pe = ltx_case(spec)
    args = TransformerArgs(x=inputs["x"].to(device), context=inputs["context"].to(device),
                           timesteps=p["timesteps"].to(device), positional_embeddings=device_tables(pe, device))
    fused, _ = workloads.build_ltx_block(spec, p, device, fuse=True)(args)
    plain, _ = workloads.build_ltx_block(spec, p, device, fuse=False)(args)
    assert torch.equal(fused.x, plain.x)


def test_ltx_block_full_9216_tokens_matches_fp32_evaluation(device):
    """Config 3 at full size: 9216 video tokens, 256 text tokens, D = 4096, 32 x 128."""
    spec = workloads.CONFIGS[3]
    p, op, inputs, pe = ltx_case(spec)
    got = _run_block(spec, p, inputs, pe, device)
    tp = {k: torch.from_numpy(np.asarray(v)).to(device) for k, v in op.items()}
    pe_d = tuple(torch.from_numpy(t).to(device) for t in pe)
    x, ctx = inputs["x"][0].float().to(device), inputs["context"][0].float().to(device)
    with torch.no_grad():
        torch.backends.cuda.matmul.allow_tf32 = False
        ref = _torch_ref.ltx_video_block(tp, x, ctx, pe_d, heads=spec.heads).cpu().numpy()
        graph = _torch_ref.ltx_video_block(tp, x, ctx, pe_d, heads=spec.heads, bf16_graph=True).cpu().numpy()
    print("config3 full block:", end=" ")
    _check_block(got, ref, graph)
