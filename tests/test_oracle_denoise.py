"""Pins of the oracle's steps either side of the block (``oracle/denoise.py``), on the CPU.

Each check is chosen so that a plausible mistake fails it: the reference's own known answers
(``tests/samplers/test_steps.py:10-71``, ``tests/models/ltx2/transformer/test_model.py:572-594``,
``tests/models/ltx2/test_state.py:99-124``, ``tests/models/ltx2/test_denoise.py:36-67``),
float64 closed forms, and weight choices (identity, scaled identity) under which a swapped
activation, a missing bias or a wrong row order changes the result.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.ops import F32, to_bf16


def _bf(x):
    return to_bf16(np.asarray(x, dtype=F32))


# ---- timestep features ----------------------------------------------------------------------


def _embedding64(t, dim, max_period=10000):
    half = dim // 2
    freqs = np.exp(-math.log(max_period) * np.arange(half, dtype=np.float64) / half)
    angles = np.asarray(t, dtype=np.float64)[:, None] * freqs[None]
    out = np.concatenate([np.cos(angles), np.sin(angles)], axis=-1)
    if dim % 2:
        out = np.pad(out, [(0, 0), (0, 1)])
    return out, angles


@pytest.mark.parametrize("dim", [256, 255, 8])
def test_timestep_embedding_matches_the_float64_closed_form(dim):
    t = np.array([0.0, 0.5, 1.0, 37.25, 999.0, 1000.0], dtype=F32)
    got = oracle.timestep_embedding(t, dim)
    ref, angles = _embedding64(t, dim)
    assert got.shape == (6, dim) and got.dtype == F32
    # fp32 exponent, exp and product: a few ulps of the angle, times |angle|
    tol = 1e-6 + 5e-7 * np.abs(np.concatenate([angles, angles], axis=-1))
    if dim % 2:
        tol = np.pad(tol, [(0, 0), (0, 1)], constant_values=1e-6)
    assert np.all(np.abs(got - ref) <= tol)


def test_timestep_embedding_structure():
    got = oracle.timestep_embedding(np.array([0.0, 2.0], dtype=F32), 9)
    assert np.array_equal(got[0, :4], np.ones(4, F32)) and np.array_equal(got[0, 4:], np.zeros(5, F32))
    assert got[1, 8] == 0.0  # odd width: one zero column
    # column 0 is cos(t) (frequency 1), column half is sin(t): cosines first, then sines
    assert got[1, 0] == pytest.approx(math.cos(2.0), abs=1e-7)
    assert got[1, 4] == pytest.approx(math.sin(2.0), abs=1e-7)
    with pytest.raises(ValueError):
        oracle.timestep_embedding(np.zeros((2, 2), F32))


def test_timestep_scale_is_an_fp32_product_before_the_features():
    t = np.array([0.123, 0.9, 0.0371], dtype=F32)
    scaled = (t * F32(1000.0)).astype(F32)
    assert np.array_equal(oracle.timestep_embedding(t, time_scale=1000.0), oracle.timestep_embedding(scaled))


# ---- AdaLN modulation producers -------------------------------------------------------------


def _silu64(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def _adaln_params(prefix, d, rows, w2_scale=2.0, b1=0.5, b2=-0.25):
    eye = np.eye(d, 256, dtype=F32)
    p = {
        f"{prefix}.emb.timestep_embedder.linear_1.weight": eye,
        f"{prefix}.emb.timestep_embedder.linear_1.bias": np.full(d, b1, F32),
        f"{prefix}.emb.timestep_embedder.linear_2.weight": (w2_scale * np.eye(d, dtype=F32)).astype(F32),
        f"{prefix}.emb.timestep_embedder.linear_2.bias": np.full(d, b2, F32),
        f"{prefix}.linear.weight": np.concatenate([(k + 1) * np.eye(d, dtype=F32) for k in range(rows)]).astype(F32),
        f"{prefix}.linear.bias": np.zeros(rows * d, F32),
    }
    return p


def test_adaln_single_order_of_layers_and_activations():
    """Identity-like weights: embedded = 2 * silu(bf16(features) + 0.5) - 0.25 and modulation row
    k = (k + 1) * silu(embedded). Swapping a SiLU past a linear, dropping a bias or reordering the
    modulation rows changes these values."""
    d, rows = 256, 3
    p = _adaln_params("a", d, rows)
    t = np.array([0.25, 0.75], dtype=F32)
    modulation, embedded = oracle.adaln_single(p, "a", t, time_scale=1000.0)
    features = _bf(oracle.timestep_embedding(t, time_scale=1000.0)).astype(np.float64)
    emb64 = 2.0 * _silu64(features + 0.5) - 0.25
    assert np.allclose(embedded, emb64, atol=2e-6)
    mod64 = np.concatenate([(k + 1) * _silu64(emb64) for k in range(rows)], axis=-1)
    assert modulation.shape == (2, rows * d)
    assert np.allclose(modulation, mod64, atol=1e-5)


# ---- output head ------------------------------------------------------------------------------


def _layer_norm64(x, eps=1e-6):
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


def test_output_head_modulation_rows_and_projection():
    rng = np.random.default_rng(3)
    d, c, t = 64, 16, 5
    table = _bf(rng.normal(0, 0.5, (2, d)))
    embedded = _bf(rng.normal(0, 0.5, (1, 1, d)))
    w = _bf(rng.normal(0, 0.1, (c, d)))
    b = _bf(rng.normal(0, 0.1, (c,)))
    p = {"scale_shift_table": table, "proj_out.weight": w, "proj_out.bias": b}
    x = _bf(rng.normal(0, 1, (1, t, d)))
    x[0, 0] = 3.0  # a constant row normalizes to 0, so its output is proj_out(shift)
    got = oracle.output_head(p, x, embedded)
    mod = _bf(table[None, None] + embedded[:, :, None, :]).astype(np.float64)
    shift, scale = mod[:, :, 0], mod[:, :, 1]
    ref = (_layer_norm64(x) * (1.0 + scale) + shift) @ w.astype(np.float64).T + b
    assert np.allclose(got, ref, atol=1e-4)
    assert np.allclose(got[0, 0], shift[0, 0] @ w.astype(np.float64).T + b, atol=1e-5)


# ---- X0 conversion, composite, Euler steps, finite check ---------------------------------------


def test_x0_known_answer_from_the_reference():
    """``test_model.py:572-594``: latent -1.640625, velocity -2.453125, timestep 0.090820007 ->
    bf16 -1.4140625 (the exact value, -1.41783..., lies near a bf16 midpoint)."""
    latent = np.full((1, 2, 4), -1.640625, F32)
    velocity = np.full((1, 2, 4), -2.453125, F32)
    got = to_bf16(oracle.to_denoised(latent, velocity, np.full((1, 2), 0.090820007, F32)))
    assert np.all(got == np.float32(-1.4140625))


def test_x0_inverts_the_flow_interpolation():
    """With x_t = (1 - t) x0 + t n and v = n - x0, latent - t v = x0 (float64 closed form), for
    per-batch and per-token timesteps."""
    rng = np.random.default_rng(0)
    x0, noise = rng.normal(size=(2, 6, 8)), rng.normal(size=(2, 6, 8))
    for t in (np.array([0.3, 0.8]), rng.uniform(0, 1, (2, 6))):
        tb = t[:, None, None] if t.ndim == 1 else t[..., None]
        latent = ((1 - tb) * x0 + tb * noise).astype(F32)
        velocity = (noise - x0).astype(F32)
        got = oracle.to_denoised(latent, velocity, t.astype(F32))
        assert np.allclose(got, x0, atol=1e-5)
    with pytest.raises(ValueError):
        oracle.to_denoised(latent, velocity, np.zeros((2, 6, 1), F32))


@pytest.mark.parametrize("mask_value", [0.0, 0.05, 0.5, 0.95, 1.0])
def test_composite_blends_once(mask_value):
    """``test_state.py:99-124`` values: mask 1 keeps the prediction exactly, mask 0 the clean
    latent exactly, fractions blend in FP32 with one rounding."""
    denoised = np.full((1, 2, 3), -8.0, F32)
    clean = np.full((1, 2, 3), 4.6875, F32)
    got = to_bf16(oracle.post_process_latent(denoised, clean, np.full((1, 2), mask_value, F32)))
    exact = -8.0 * mask_value + 4.6875 * (1.0 - mask_value)
    assert np.allclose(got, exact, rtol=2 ** -8)
    if mask_value in (0.0, 1.0):
        assert np.all(got == np.float32(exact))


def test_euler_velocity_step_narrows_before_the_add():
    """``test_steps.py:10-24``: bf16 sample and velocity 0.01, sigma 1 -> 0.1234567: the scaled
    velocity is rounded to bf16 before the add, which differs from one FP32 evaluation."""
    sample = _bf([0.01])
    velocity = _bf([0.01])
    got = oracle.euler_velocity_step(sample, velocity, 1.0, 0.1234567, bf16=True)
    delta = np.float32(0.1234567 - 1.0)
    full = to_bf16(sample + delta * velocity)
    assert got[0] != full[0]
    assert got[0] == to_bf16(sample + to_bf16(delta * velocity))[0]
    same = oracle.euler_velocity_step(sample, velocity, 0.5, 0.5, bf16=True)
    assert np.array_equal(same, sample)


def test_euler_step_known_answers():
    """``test_steps.py:27-71``."""
    assert np.allclose(oracle.euler_step(np.full(3, 10.0, F32), np.zeros(3, F32), 1.0, 0.5), 5.0)
    d = np.array([1.0, 1.0, 1.0], F32)
    assert np.array_equal(oracle.euler_step(np.array([3.0, -2.0, 7.5], F32), d, 0.5, 0.0), d)
    s = np.array([5.0, 7.0, -3.0], F32)
    assert np.array_equal(oracle.euler_step(s, np.zeros(3, F32), 0.5, 0.5), s)
    for sigma in (0.0, -0.5, float("nan")):
        with pytest.raises(ValueError, match="current sigma must be positive"):
            oracle.euler_step(np.ones(1, F32), np.zeros(1, F32), sigma, -1.0)


def test_euler_step_equals_the_velocity_form_in_float64():
    """denoised + (s'/s)(x - denoised) = x + (s' - s) v with v = (x - denoised) / s."""
    rng = np.random.default_rng(1)
    x, d = rng.normal(size=64).astype(F32), rng.normal(size=64).astype(F32)
    sigma, nxt = 0.8, 0.55
    v = (x.astype(np.float64) - d) / sigma
    assert np.allclose(oracle.euler_step(x, d, sigma, nxt), x + (nxt - sigma) * v, atol=1e-6)


def test_mixed_mask_step_from_the_reference():
    """``test_denoise.py:50-67``: mask (0.5, 1), latent 1, clean 4, zero X0 prediction, sigma 1 -> 0
    gives (2, 0): the composite keeps half the clean latent for token 0."""
    mask = np.array([[0.5, 1.0]], F32)
    latent = np.ones((1, 2, 3), F32)
    clean = np.full((1, 2, 3), 4.0, F32)
    prediction = oracle.post_process_latent(np.zeros((1, 2, 3), F32), clean, mask)
    out = oracle.euler_step(latent, prediction, 1.0, 0.0)
    assert np.array_equal(out[:, 0], np.full((1, 3), 2.0, F32))
    assert np.array_equal(out[:, 1], np.zeros((1, 3), F32))


def test_all_finite():
    assert oracle.all_finite(np.zeros(5, F32))
    for bad in (np.nan, np.inf, -np.inf):
        x = np.zeros(5, F32)
        x[4] = bad
        assert not oracle.all_finite(x)
