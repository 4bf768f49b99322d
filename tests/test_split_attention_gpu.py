"""Key-split attention on the GPU (kx_attention_split_fwd_bf16): few-query, many-key calls against
the oracle and against the unsplit kernel, with gates, biases, batches and ragged key counts."""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import _lib, workloads
from kinomlx_amd.ltx2.dense_attention import batched_attention
from tests.conftest import cosine, max_abs

pytestmark = pytest.mark.gpu


def _bf(shape, seed):
    return workloads.bf16(workloads.normal(seed, "split", shape))


def _unsplit(q, k, v, heads, dim, gate=None):
    out = torch.empty_like(q)
    b, tq, tk = q.shape[0], q.shape[1], k.shape[1]
    g = None if gate is None else gate.reshape(b * tq, heads)
    _lib._call("kx_attention_fwd_bf16", q.data_ptr(), q.stride(-2), k.data_ptr(), k.stride(-2), v.data_ptr(),
               v.stride(-2), out.data_ptr(), out.stride(-2), b, tq, tk, heads, dim, dim ** -0.5,
               None if g is None else g.data_ptr(), heads, _lib._stream())
    return out


@pytest.mark.parametrize("batch,heads,dim,tq,tk", [(1, 32, 64, 127, 5376), (2, 4, 128, 50, 2000), (1, 8, 64, 300, 1500)])
@pytest.mark.parametrize("gated", [False, True])
def test_split_matches_oracle_and_unsplit(device, batch, heads, dim, tq, tk, gated):
    assert _lib.attention_splits(batch, tq, tk, heads) > 1
    q, k, v = (_bf((batch, t, heads * dim), s).to(device) for s, t in ((1, tq), (2, tk), (3, tk)))
    gate = None
    if gated:
        gate = (torch.rand((batch, tq, heads), generator=torch.Generator().manual_seed(4)) * 2).to(torch.bfloat16)
        gate = gate.to(device)
    got = batched_attention(q, k, v, heads=heads, gate=gate)
    plain = _unsplit(q, k, v, heads, dim, gate)
    a, b = got.float().cpu().numpy(), plain.float().cpu().numpy()
    assert cosine(a, b) > 0.99999 and max_abs(a, b) <= 2 ** -7 * max(1.0, np.abs(b).max())
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ref = np.stack([oracle.attention(qn[i], kn[i], vn[i], heads=heads) for i in range(batch)])
    if gated:
        ref = (ref.reshape(batch, tq, heads, dim) * gate.float().cpu().numpy()[..., None]).reshape(ref.shape)
    assert cosine(a, ref) > 0.99999 and max_abs(a, ref) < 2e-2


def test_split_with_bias_and_fully_masked_rows(device):
    batch, heads, dim, tq, tk = 1, 8, 64, 100, 3000
    q, k, v = (_bf((batch, t, heads * dim), s).to(device) for s, t in ((5, tq), (6, tk), (7, tk)))
    mask = torch.zeros((batch, tq, tk), dtype=torch.bfloat16)
    mask[0, :, 2000:] = -3.3895313892515355e38  # a whole slice of keys removed for every query
    mask[0, 7, :] = -3.3895313892515355e38      # query 7 sees no key: the uniform average of V
    got = batched_attention(q, k, v, heads=heads, mask=mask.to(device)).float().cpu().numpy()
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ref = oracle.attention(qn[0], kn[0], vn[0], heads=heads, bias=mask.float().numpy()[0][None])
    assert cosine(got[0], ref) > 0.99999 and max_abs(got[0], ref) < 2e-2
    assert np.allclose(got[0, 7], vn[0].mean(0), atol=1e-2)
