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
