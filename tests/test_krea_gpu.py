"""Krea 2 block surface parity on the GPU (``kinomlx_amd.krea2``) against the FP32 oracle on the
same seeded inputs.

Bars: ``apply_rotary_embedding`` is bit-exact; the zero-centred norm within one bf16 ulp-level
relative L2; grouped-query attention within the reference's attention tolerance; the block at
the block bar (cosine >= 0.9995 and |got - ref| <= 2e-2 + ulp_bf16(ref) / 2 elementwise,
``assert_block_bar``), with the reference's own bf16 execution printed beside it.
"""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd.krea2 import transformer as krea
from kinomlx_amd.ltx2 import dense_attention
from tests._blocks import build_krea_block, krea_case
from tests.conftest import assert_block_bar, cosine, max_abs, rel_l2

pytestmark = pytest.mark.gpu
F32 = np.float32


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize(
    ("hidden", "heads", "kv_heads", "tokens", "ff"),
    [(512, 4, 2, 96, 1024), (384, 6, 2, 37, 768), (1024, 8, 8, 64, 2048)],
    ids=["gqa-d512-fused-norm-rope", "gqa-d384-h64-two-pass", "mha-d1024"],
)
def test_krea_block_matches_oracle(device, hidden, heads, kv_heads, tokens, ff):
    p, op, x, tmod, ids = krea_case(hidden, heads, kv_heads, tokens, ff)
    dh = hidden // heads
    rope = krea.Krea2RotaryEmbedding(theta=1000.0, axes_dims=(dh // 4, dh // 4, dh // 2))
    cos, sin = rope(ids.to(device))
    block = build_krea_block(p, hidden, heads, kv_heads, device)
    got = _np(block(x.to(device), time_modulation=tmod.to(device), rotary=(cos, sin), attention_mask=None)[0])
    mod = tmod[0].float().numpy().reshape(6, hidden) + op["scale_shift_table"]
    rot = (_np(cos)[0], _np(sin)[0])
    xn = x[0].float().numpy()
    ref = oracle.krea_block(op, xn, mod, rot, heads=heads, kv_heads=kv_heads)
    graph = oracle.krea_block(op, xn, mod, rot, heads=heads, kv_heads=kv_heads, bf16_graph=True)
    assert_block_bar(got, ref, "krea block", context=graph)


def test_krea_block_unfused_and_batched_agree(device):
    hidden, heads, kv_heads = 512, 4, 2
    p, _, x, tmod, ids = krea_case(hidden, heads, kv_heads, 40, 1024, batch=2)
    rope = krea.Krea2RotaryEmbedding(theta=1000.0, axes_dims=(32, 32, 64))
    tables = rope(ids.to(device))
    kwargs = dict(time_modulation=tmod.to(device), rotary=tables, attention_mask=None)
    fused = build_krea_block(p, hidden, heads, kv_heads, device)(x.to(device), **kwargs)
    plain = build_krea_block(p, hidden, heads, kv_heads, device, fuse=False)(x.to(device), **kwargs)
    # the fused projection norms and rotates Q/K in its epilogue; the unfused path's two passes
    # (the key width is not a multiple of 512) round the normalized keys once more
    assert rel_l2(_np(fused), _np(plain)) < 2e-3 and max_abs(_np(fused), _np(plain)) < 2e-2
    one = build_krea_block(p, hidden, heads, kv_heads, device)(
        x[1:].to(device), time_modulation=tmod[1:].to(device), rotary=tuple(t[1:] for t in tables),
        attention_mask=None)
    assert torch.equal(fused[1:], one)


def test_krea_rotary_tables_and_rotation(device):
    """``Krea2RotaryEmbedding`` against the oracle's tables; ``apply_rotary_embedding`` on
    head-major Q/K bit-exact with the FP32 product-then-sum order."""
    r = np.random.default_rng(91)
    ids = torch.from_numpy(r.integers(0, 50, (2, 11, 3)).astype(F32))
    rope = krea.Krea2RotaryEmbedding(theta=1000.0, axes_dims=(16, 16, 32))
    cos, sin = rope(ids.to(device))
    ref_cos, ref_sin = oracle.krea_rotary(ids.numpy(), theta=1000.0, axes_dims=(16, 16, 32))
    assert np.allclose(_np(cos), ref_cos, atol=3e-6) and np.allclose(_np(sin), ref_sin, atol=3e-6)
    q = oracle.to_bf16(r.standard_normal((2, 4, 11, 64)).astype(F32) * 2)
    k = oracle.to_bf16(r.standard_normal((2, 2, 11, 64)).astype(F32) * 2)
    gq, gk = krea.apply_rotary_embedding(torch.from_numpy(q).to(device).to(torch.bfloat16),
                                         torch.from_numpy(k).to(device).to(torch.bfloat16), cos, sin)
    rq, rk = oracle.krea_apply_rotary(q, k, _np(cos), _np(sin))
    assert np.array_equal(_np(gq), oracle.to_bf16(rq)) and np.array_equal(_np(gk), oracle.to_bf16(rk))


def test_krea_rms_norm_is_zero_centred(device):
    r = np.random.default_rng(92)
    x = oracle.to_bf16(r.standard_normal((7, 512)).astype(F32) * 3)
    w = (r.standard_normal(512) * 0.1).astype(F32)
    norm = krea.Krea2RMSNorm(512, 1e-6)
    norm.weight = torch.from_numpy(w).to(device)
    got = _np(norm(torch.from_numpy(x).to(device).to(torch.bfloat16)))
    ref = oracle.krea_rms_norm(x, w, 1e-6)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-6)


@pytest.mark.parametrize(("heads", "kv_heads", "dh"), [(8, 2, 128), (6, 3, 64), (4, 1, 128)])
def test_grouped_query_attention_kernel(device, heads, kv_heads, dh):
    """``kx_attention_gqa_fwd_bf16``: query head h reads K/V head h // (heads / kv_heads)."""
    r = np.random.default_rng(93 + heads)
    tq, tk = 300, 129
    q = oracle.to_bf16(r.standard_normal((tq, heads * dh)).astype(F32))
    k = oracle.to_bf16(r.standard_normal((tk, kv_heads * dh)).astype(F32))
    v = oracle.to_bf16(r.standard_normal((tk, kv_heads * dh)).astype(F32))
    dev = [torch.from_numpy(a).to(device).to(torch.bfloat16)[None] for a in (q, k, v)]
    got = _np(dense_attention.batched_attention(*dev, heads=heads, kv_heads=kv_heads)[0])
    group = heads // kv_heads
    kf = np.repeat(k.reshape(tk, kv_heads, dh), group, axis=1).reshape(tk, -1)
    vf = np.repeat(v.reshape(tk, kv_heads, dh), group, axis=1).reshape(tk, -1)
    ref = oracle.attention(q, kf, vf, heads=heads)
    assert rel_l2(got, ref) < 8e-3 and max_abs(got, ref) < 2e-2


def test_krea_key_mask_equals_the_truncated_sequence(device):
    """A boolean (batch, length) mask: the valid queries see only the valid keys, so their rows
    equal the block run on the valid prefix alone; the masked queries' attention is zero
    (``model.py:164-196``)."""
    hidden, heads, kv_heads, tokens, keep = 512, 4, 2, 80, 53
    p, _, x, tmod, ids = krea_case(hidden, heads, kv_heads, tokens, 1024)
    rope = krea.Krea2RotaryEmbedding(theta=1000.0, axes_dims=(32, 32, 64))
    cos, sin = rope(ids.to(device))
    block = build_krea_block(p, hidden, heads, kv_heads, device)
    mask = torch.zeros((1, tokens), dtype=torch.bool, device=device)
    mask[:, :keep] = True
    masked = _np(block(x.to(device), time_modulation=tmod.to(device), rotary=(cos, sin), attention_mask=mask)[0])
    short = _np(block(x[:, :keep].contiguous().to(device), time_modulation=tmod.to(device),
                      rotary=(cos[:, :keep].contiguous(), sin[:, :keep].contiguous()), attention_mask=None)[0])
    assert cosine(masked[:keep], short) > 0.999999 and max_abs(masked[:keep], short) <= 2 ** -6 * np.abs(short).max()
    with pytest.raises(ValueError, match="boolean"):
        block(x.to(device), time_modulation=tmod.to(device), rotary=(cos, sin), attention_mask=mask.float())
