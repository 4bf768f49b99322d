"""Pins of the oracle's additive-bias attention (the reference's masked SDPA) on the CPU."""

import numpy as np

import oracle
from oracle.ops import F32


def _qkv(seed=0, tq=7, tk=11, heads=2, dh=8):
    r = np.random.default_rng(seed)
    return [r.standard_normal(s).astype(F32) for s in ((tq, heads * dh), (tk, heads * dh), (tk, heads * dh))]


def test_zero_and_row_constant_bias_change_nothing():
    q, k, v = _qkv()
    base = oracle.attention(q, k, v, heads=2)
    assert np.array_equal(oracle.attention(q, k, v, heads=2, bias=np.zeros((1, 1, 11), F32)), base)
    row = np.random.default_rng(1).standard_normal((2, 7, 1)).astype(F32)  # softmax shift invariance
    assert np.allclose(oracle.attention(q, k, v, heads=2, bias=np.broadcast_to(row, (2, 7, 11))), base, atol=1e-5)


def test_masked_keys_equal_attention_over_the_kept_keys():
    q, k, v = _qkv()
    keep = np.array([1, 0, 1, 1, 0, 0, 1, 1, 1, 0, 1], bool)
    bias = np.where(keep, 0.0, -3.3895313892515355e38).astype(F32)[None, None]
    got = oracle.attention(q, k, v, heads=2, bias=bias)
    ref = oracle.attention(q, k[keep], v[keep], heads=2)
    assert np.allclose(got, ref, atol=1e-5)


def test_bias_matches_float64_brute_force_per_head_and_query():
    q, k, v = _qkv(tq=5, tk=6, heads=2, dh=4)
    bias = np.random.default_rng(2).standard_normal((2, 5, 6)).astype(F32)
    got = oracle.attention(q, k, v, heads=2, bias=bias)
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    for h in range(2):
        sl = slice(4 * h, 4 * h + 4)
        s = q64[:, sl] @ k64[:, sl].T / 2.0 + bias[h]
        p = np.exp(s - s.max(-1, keepdims=True))
        assert np.allclose(got[:, sl], (p / p.sum(-1, keepdims=True)) @ v64[:, sl], atol=1e-5)
