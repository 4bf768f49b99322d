"""Masked attention on the GPU: the kernel's additive score bias against the oracle, every mask
shape the reference's SDPA takes, and the preprocessor's mask conversions."""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.ltx2.dense_attention import batched_attention
from tests.conftest import cosine, max_abs

pytestmark = pytest.mark.gpu

MIN = -3.3895313892515355e38


def _bf(shape, seed, scale=1.0):
    return (workloads.normal(seed, "mask", shape) * scale).to(torch.bfloat16)


def _oracle(q, k, v, heads, bias_np):
    return np.stack([oracle.attention(q[b].float().numpy(), k[b].float().numpy(), v[b].float().numpy(), heads=heads,
                                      bias=None if bias_np is None else bias_np[b]) for b in range(q.shape[0])])


@pytest.mark.parametrize("dim", [128, 64])
@pytest.mark.parametrize("kind", ["keys", "keys_bool", "full", "per_head", "shared2d"])
def test_masked_attention_matches_oracle(device, dim, kind):
    batch, heads, tq, tk = 2, 4, 150, 83  # ragged: tk not a multiple of the 64-key tile or of 4
    q, k, v = _bf((batch, tq, heads * dim), 1), _bf((batch, tk, heads * dim), 2), _bf((batch, tk, heads * dim), 3)
    g = torch.Generator().manual_seed(5)
    if kind == "keys":
        keep = torch.rand((batch, tk), generator=g) > 0.3
        mask = ((keep.float() - 1.0) * -MIN).to(torch.bfloat16)[:, None, None, :]
    elif kind == "keys_bool":
        mask = (torch.rand((batch, tk), generator=g) > 0.3)[:, None, None, :]
    elif kind == "full":
        mask = (torch.randn((batch, tq, tk), generator=g) * 2).to(torch.bfloat16)
    elif kind == "per_head":
        mask = (torch.randn((batch, heads, tq, tk), generator=g) * 2).to(torch.bfloat16)
    else:
        mask = (torch.randn((tq, tk), generator=g) * 2).to(torch.bfloat16)
    got = batched_attention(q.to(device), k.to(device), v.to(device), heads=heads, mask=mask.to(device))
    m = mask if mask.dtype != torch.bool else torch.where(mask, 0.0, float("-inf"))
    m4 = m.float()
    while m4.dim() < 4:
        m4 = m4[None] if m4.dim() == 2 else m4[:, None]
    bias_np = np.broadcast_to(m4.numpy(), (batch, heads, tq, tk))
    ref = _oracle(q, k, v, heads, bias_np)
    out = got.float().cpu().numpy()
    assert np.all(np.isfinite(out))
    # one bf16 rounding of outputs below ~4: the per-op bar of the attention kernel
    assert cosine(out, ref) > 0.99999 and max_abs(out, ref) < 2e-2, (cosine(out, ref), max_abs(out, ref))


def test_fully_masked_row_averages_values(device):
    heads, tq, tk, dim = 2, 40, 70, 128
    q, k, v = _bf((1, tq, heads * dim), 7), _bf((1, tk, heads * dim), 8), _bf((1, tk, heads * dim), 9)
    mask = torch.zeros((1, tq, tk), dtype=torch.bfloat16)
    mask[0, 3, :] = MIN  # every key of query 3 removed
    got = batched_attention(q.to(device), k.to(device), v.to(device), heads=heads, mask=mask.to(device))
    mean = v[0].float().mean(0).numpy()
    assert np.allclose(got[0, 3].float().cpu().numpy(), mean, atol=1e-2)


@pytest.mark.parametrize("dim", [64, 128])
def test_unmasked_bias_of_zero_matches_no_mask(device, dim):
    # D = 64 runs one key loop for both forms (bit-identical); at D = 128 the unbiased kernel is
    # software-pipelined over 32-key blocks (its running max moves per block, its row sums add per
    # 16 keys), so the two forms agree to the kernel's per-op bar rather than bit for bit
    heads, tq, tk = 4, 300, 200
    q, k, v = _bf((1, tq, heads * dim), 10), _bf((1, tk, heads * dim), 11), _bf((1, tk, heads * dim), 12)
    plain = batched_attention(q.to(device), k.to(device), v.to(device), heads=heads)
    zero = batched_attention(q.to(device), k.to(device), v.to(device), heads=heads,
                             mask=torch.zeros((1, 1, 1, tk), dtype=torch.bfloat16, device=device))
    if dim == 64:
        assert torch.equal(plain, zero)
    else:
        a, b = plain.float().cpu().numpy(), zero.float().cpu().numpy()
        assert cosine(a, b) > 0.99999 and max_abs(a, b) < 2e-2, (cosine(a, b), max_abs(a, b))


def test_preprocessor_mask_conversions(device):
    from kinomlx_amd.ltx2.model import LTXAVModel, ModalityPreprocessor

    pre = ModalityPreprocessor(model=LTXAVModel(num_layers=1, video_heads=8, video_head_dim=128,
                                                video_context_dim=1024), prefix="", inner_dim=1024, heads=8,
                               max_pos=(20, 2048, 2048), cross_dim=1024, cross_max_pos=20)
    keep = torch.tensor([[1, 0, 1]], device=device)
    bias = pre._context_mask(keep)
    assert bias.shape == (1, 1, 1, 3) and bias.dtype == torch.bfloat16
    assert bias[0, 0, 0, 0].item() == 0.0 and bias[0, 0, 0, 1].item() == pytest.approx(MIN, rel=1e-2)
    soft = torch.tensor([[[1.0, 0.5], [0.0, 0.25]]], device=device)
    log_bias = pre._self_attention_mask(soft, torch.bfloat16)
    assert log_bias.shape == (1, 1, 2, 2)
    assert log_bias[0, 0, 0, 0].item() == 0.0 and log_bias[0, 0, 0, 1].item() == pytest.approx(np.log(0.5), abs=1e-2)
    assert log_bias[0, 0, 1, 0].item() == pytest.approx(MIN, rel=1e-2)


def test_block_with_padded_text_mask_equals_the_unpadded_block(device):
    """A text context padded with masked tokens gives the block output of the unpadded context
    (the padding's keys are removed by the mask inside the kernel)."""
    from kinomlx_amd.ltx2.transformer import TransformerArgs
    from tests._blocks import device_tables, ltx_case

    spec = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=24, dim=1024, heads=8, head_dim=128)
    p, _, inputs, pe = ltx_case(spec)
    block = workloads.build_ltx_block(spec, p, device)
    keep = 17
    ctx = inputs["context"].to(device)
    mask = torch.zeros((1, 1, 1, spec.text_tokens), dtype=torch.bfloat16, device=device)
    mask[..., keep:] = MIN
    common = dict(x=inputs["x"].to(device), timesteps=p["timesteps"].to(device),
                  positional_embeddings=device_tables(pe, device))
    masked, _ = block(TransformerArgs(context=ctx, context_mask=mask, **common))
    short, _ = block(TransformerArgs(context=ctx[:, :keep].contiguous(), **common))
    a, b = masked.x.float().cpu().numpy(), short.x.float().cpu().numpy()
    assert cosine(a, b) > 0.999999 and max_abs(a, b) <= 2 ** -6 * max(1.0, np.abs(b).max())
