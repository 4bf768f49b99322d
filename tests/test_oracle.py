"""Pins the CPU oracle before it is trusted as the parity checker.

Each oracle function is checked against the reference's own known-answer tests where they exist,
and otherwise against what the mathematics fixes (float64 / library routines, closed forms,
invariants), chosen so that a dropped term, a wrong sign or index, or a transposed operand
fails. CPU only.
"""

import math

import numpy as np
import pytest
import torch
from scipy.special import expit

import oracle
from tests.conftest import max_abs, rel_l2

F32 = np.float32


def _rng(seed):
    return np.random.default_rng(seed)


# ---- bf16 rounding ---------------------------------------------------------------------------


def _nearest_bf16_by_search(x: float) -> float:
    """Round a float32 value to bf16 by enumerating its two bf16 neighbours (ties to even)."""
    bits = np.array([x], dtype=F32).view(np.uint32)[0]
    lo = (bits & 0xFFFF0000)
    hi = lo + 0x10000
    flo = np.array([lo], dtype=np.uint32).view(F32)[0]
    fhi = np.array([hi], dtype=np.uint32).view(F32)[0]
    dlo, dhi = abs(float(x) - float(flo)), abs(float(fhi) - float(x))
    if dlo < dhi:
        return float(flo)
    if dhi < dlo:
        return float(fhi)
    return float(flo) if ((lo >> 16) & 1) == 0 else float(fhi)


def test_bf16_rounding_is_nearest_even_by_exhaustive_neighbour_search():
    r = _rng(0)
    xs = np.concatenate([r.standard_normal(4000).astype(F32) * 10, (np.arange(1, 300, dtype=F32) + 0.5) / 128])
    got = oracle.to_bf16(xs)
    want = np.array([_nearest_bf16_by_search(float(x)) for x in xs], dtype=F32)
    assert np.array_equal(got, want)


# ---- RoPE --------------------------------------------------------------------------------------


def test_rope_grid_matches_reference_known_answer():
    """The reference's float64 grid test (tests/models/ltx2/transformer/test_primitives.py:115-132)."""
    positions = np.array([[[[0.0, 1.0]]]], dtype=F32)
    cos, sin = oracle.precompute_freqs_cis(
        positions, dim=8, theta=10000.0, max_pos=(20,), use_middle_indices_grid=True, num_attention_heads=2
    )
    grid = np.power(10000.0, np.linspace(0.0, 1.0, 4, dtype=np.float64))
    angles = (grid * np.pi / 2).astype(F32) * F32(2 * 0.5 / 20 - 1)
    assert np.allclose(cos, np.cos(angles).astype(F32).reshape(1, 2, 1, 2), atol=1e-6)
    assert np.allclose(sin, np.sin(angles).astype(F32).reshape(1, 2, 1, 2), atol=1e-6)


def test_rope_tables_interleave_axes_and_front_pad():
    """3 axes, dim 16, 2 heads: n = 16 // 6 = 2 frequencies x 3 axes = 6 entries, front-padded
    by 2 with (cos 1, sin 0); entry 2 + 3j + a holds axis a's j-th frequency."""
    positions = np.zeros((1, 3, 1, 2), dtype=F32)
    positions[0, :, 0, 0] = [2.0, 10.0, 30.0]
    positions[0, :, 0, 1] = [3.0, 11.0, 31.0]
    max_pos = (20, 2048, 2048)
    cos, sin = oracle.precompute_freqs_cis(positions, dim=16, max_pos=max_pos, use_middle_indices_grid=True,
                                           num_attention_heads=2)
    flat_cos = cos.transpose(0, 2, 1, 3).reshape(-1)
    flat_sin = sin.transpose(0, 2, 1, 3).reshape(-1)
    assert flat_cos[:2].tolist() == [1.0, 1.0] and flat_sin[:2].tolist() == [0.0, 0.0]
    grid = [math.pi / 2, 10000.0 * math.pi / 2]
    mids = [2.5, 10.5, 30.5]
    for j in range(2):
        for a in range(3):
            angle = (2 * mids[a] / max_pos[a] - 1) * grid[j]
            assert flat_cos[2 + 3 * j + a] == pytest.approx(math.cos(angle), abs=2e-3 if j else 1e-6)
            assert flat_sin[2 + 3 * j + a] == pytest.approx(math.sin(angle), abs=2e-3 if j else 1e-6)


def test_split_rope_is_complex_rotation_of_halves():
    r = _rng(1)
    b, h, t, half = 2, 3, 5, 8
    x = r.standard_normal((b, t, h * 2 * half)).astype(F32)
    ang = r.uniform(-4, 4, (1, h, t, half))
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    got = oracle.split_rope(x, cos, sin)
    xh = x.astype(np.float64).reshape(b, t, h, 2 * half).transpose(0, 2, 1, 3)
    z = (xh[..., :half] + 1j * xh[..., half:]) * (cos.astype(np.float64) + 1j * sin.astype(np.float64))
    want = np.concatenate([z.real, z.imag], -1).transpose(0, 2, 1, 3).reshape(x.shape)
    assert max_abs(got, want) < 1e-5
    # rotation preserves each pair's norm
    gh = got.reshape(b, t, h, 2 * half)
    n_in = xh.transpose(0, 2, 1, 3)[..., :half] ** 2 + xh.transpose(0, 2, 1, 3)[..., half:] ** 2
    n_out = gh[..., :half].astype(np.float64) ** 2 + gh[..., half:].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)


def test_split_rope_rounds_each_product_before_the_difference():
    """x1 = c = x2 = s = 1 + 2^-12: separately rounded products cancel to exactly 0, while a
    fused multiply-add or a float64 evaluation leaves 2^-24."""
    v = F32(1.0 + 2.0**-12)
    x = np.array([[[v, v]]], dtype=F32)  # one head, half = 1
    c = np.array([[[[v]]]], dtype=F32)
    out = oracle.split_rope(x, c, c)
    assert out[0, 0, 0] == 0.0
    assert out[0, 0, 1] == F32(F32(v * v) + F32(v * v))


def test_pair_rope_is_complex_rotation_of_adjacent_pairs():
    r = _rng(2)
    x = r.standard_normal((4, 3, 16)).astype(F32)
    ang = np.repeat(r.uniform(-3, 3, (4, 1, 8)), 2, axis=-1)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    got = oracle.pair_rope(x, cos, sin)
    z = (x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]) * np.exp(1j * ang[..., 0::2])
    want = np.stack([z.real, z.imag], -1).reshape(x.shape)
    assert max_abs(got, want) < 1e-5


def test_krea_rotary_axis_order_and_adjacent_pairs_match_reference_test():
    """tests/models/krea2/transformer/test_transformer.py:302-327."""
    cos, sin = oracle.krea_rotary(np.array([[[1.0, 2.0, 3.0]]], F32), theta=1000.0, axes_dims=(2, 2, 4))
    third = 3.0 / math.sqrt(1000.0)
    angles = (1.0, 1.0, 2.0, 2.0, 3.0, 3.0, third, third)
    assert np.allclose(cos[0, 0], [math.cos(a) for a in angles], atol=1e-6)
    assert np.allclose(sin[0, 0], [math.sin(a) for a in angles], atol=1e-6)
    q = np.arange(1.0, 9.0, dtype=F32).reshape(1, 1, 1, 8)
    rq, rk = oracle.krea_apply_rotary(q, q * 2, cos, sin)
    assert rq[0, 0, 0, 0] == pytest.approx(math.cos(1.0) - 2 * math.sin(1.0), abs=1e-6)
    assert rq[0, 0, 0, 1] == pytest.approx(math.sin(1.0) + 2 * math.cos(1.0), abs=1e-6)
    assert np.allclose(rk, rq * 2, atol=1e-6)


def test_flux_rotary_frequencies_follow_2000_power_law():
    ids = np.array([[[1.0, 2.0, 3.0, 4.0]]], F32)
    cos, sin = oracle.flux_rotary_positions(ids)
    assert cos.shape == (1, 1, 1, 128)
    for axis in range(4):
        for i in range(16):
            angle = ids[0, 0, axis] * 2000.0 ** (-2 * i / 32)
            k = 2 * (axis * 16 + i)
            assert cos[0, 0, 0, k] == pytest.approx(math.cos(angle), abs=1e-5)
            assert cos[0, 0, 0, k + 1] == cos[0, 0, 0, k]
            assert sin[0, 0, 0, k] == pytest.approx(math.sin(angle), abs=1e-5)


# ---- norms and modulation ------------------------------------------------------------------------


def test_rms_norm_matches_float64_textbook_within_reference_tolerance():
    r = _rng(3)
    x = (r.standard_normal((2, 5, 256)) * 3).astype(F32)
    w = (r.standard_normal(256) * 0.1 + 1.0).astype(F32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True) + 1e-6) * w
    assert rel_l2(oracle.rms_norm(x, w, 1e-6), want) <= 5e-5  # tests/kernels/test_fused_ops.py:68-84
    # the offset is added to the weight, not to the output
    assert np.array_equal(oracle.rms_norm(x, w, 1e-6, weight_offset=1.0), oracle.rms_norm(x, w + F32(1.0), 1e-6))
    # unweighted output has unit RMS
    y = oracle.rms_norm(x, None, 1e-9).astype(np.float64)
    assert np.allclose(np.sqrt(np.mean(y * y, -1)), 1.0, atol=1e-5)


def test_layer_norm_centres_and_scales():
    r = _rng(4)
    x = (r.standard_normal((3, 512)) * 5 + 7).astype(F32)
    y = oracle.layer_norm(x, 1e-6).astype(np.float64)
    assert np.allclose(y.mean(-1), 0, atol=1e-5)
    assert np.allclose(y.var(-1), 1, atol=1e-4)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + 1e-6)
    assert max_abs(y, want) < 1e-5


def test_adaln_scale_and_shift_rows_enter_as_stated():
    r = _rng(5)
    x = r.standard_normal((4, 64)).astype(F32)
    shift = r.standard_normal(64).astype(F32)
    # scale = -1 cancels the normalised value: the output is the shift itself
    assert np.array_equal(oracle.adaln(x, np.full(64, -1, F32), shift), np.broadcast_to(shift, x.shape))
    # scale = 0, shift = 0 is the plain RMSNorm
    zeros = np.zeros(64, F32)
    assert np.array_equal(oracle.adaln(x, zeros, zeros), oracle.rms_norm(x))
    # LayerNorm modulation likewise
    assert np.array_equal(oracle.normalized(x, shift, np.full(64, -1, F32)), np.broadcast_to(shift, x.shape))


def test_gated_residual_modulate_gate_closed_forms():
    x = np.array([[1.0, 2.0]], F32)
    r = np.array([[3.0, -4.0]], F32)
    g = np.array([0.5, 2.0], F32)
    assert oracle.gated_residual(x, r, g).tolist() == [[2.5, -6.0]]
    assert oracle.modulate(x, g, r).tolist() == [[4.5, 2.0]]
    assert oracle.gate(r, g).tolist() == [[1.5, -8.0]]


# ---- activations -------------------------------------------------------------------------------


def test_gelu_matches_torch_float64_tanh_gelu():
    x = np.linspace(-8, 8, 65536, dtype=F32)
    want = torch.nn.functional.gelu(torch.from_numpy(x.astype(np.float64)), approximate="tanh").numpy()
    assert max_abs(oracle.gelu_approx(x), want) < 2e-6
    big = np.linspace(-128, 128, 4097, dtype=F32)
    got = oracle.gelu_approx(big)
    assert np.all(np.isfinite(got))
    assert np.allclose(got[big > 8], big[big > 8]) and np.allclose(got[big < -8], 0, atol=1e-6)


def test_silu_matches_scipy_expit():
    x = np.linspace(-30, 30, 20001, dtype=F32)
    want = x.astype(np.float64) * expit(x.astype(np.float64))
    assert max_abs(oracle.silu(x), want) < 2e-6


def test_swiglu_gates_the_first_half_and_carries_the_second():
    g = np.array([[0.0, 50.0, -3.0]], F32)
    c = np.array([[7.0, 2.0, 1.0]], F32)
    out = oracle.swiglu(np.concatenate([g, c], -1))
    assert out[0, 0] == 0.0  # silu(0) = 0 whatever the content
    assert out[0, 1] == pytest.approx(100.0)  # silu(50) ~ 50
    assert out[0, 2] == pytest.approx(-3.0 * expit(-3.0))


# ---- attention and linear --------------------------------------------------------------------------


def _attention64(q, k, v, heads):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    dh = q.shape[1] // heads
    out = np.empty_like(q)
    for h in range(heads):
        s = slice(h * dh, (h + 1) * dh)
        sc = q[:, s] @ k[:, s].T / math.sqrt(dh)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        out[:, s] = (p / p.sum(-1, keepdims=True)) @ v[:, s]
    return out


@pytest.mark.parametrize(("tq", "tk", "dh"), [(7, 7, 64), (33, 5, 128), (40, 300, 64), (1, 17, 128)])
def test_attention_matches_float64_explicit_softmax(tq, tk, dh):
    r = _rng(tq * 31 + tk)
    heads = 2
    q, k, v = (r.standard_normal((t, heads * dh)).astype(F32) for t in (tq, tk, tk))
    assert max_abs(oracle.attention(q, k, v, heads=heads), _attention64(q, k, v, heads)) < 1e-5


def test_attention_invariants():
    r = _rng(6)
    heads, dh = 2, 64
    q = r.standard_normal((9, heads * dh)).astype(F32)
    v = r.standard_normal((5, heads * dh)).astype(F32)
    same_k = np.repeat(r.standard_normal((1, heads * dh)).astype(F32), 5, axis=0)
    # identical keys: uniform weights, output is the mean value row
    assert max_abs(oracle.attention(q, same_k, v, heads=heads), np.broadcast_to(v.mean(0), (9, heads * dh))) < 1e-5
    # one key: output is that value row
    assert max_abs(oracle.attention(q, v[:1], v[:1] * 3, heads=heads), np.broadcast_to(v[0] * 3, (9, heads * dh))) < 1e-5
    # keys/values permuted together: same output
    k = r.standard_normal((5, heads * dh)).astype(F32)
    perm = r.permutation(5)
    assert max_abs(oracle.attention(q, k, v, heads=heads), oracle.attention(q, k[perm], v[perm], heads=heads)) < 1e-5


def test_linear_is_x_times_weight_transpose_plus_bias():
    r = _rng(7)
    x = r.standard_normal((5, 24)).astype(F32)
    w = r.standard_normal((10, 24)).astype(F32)  # (out, in), non-square
    b = r.standard_normal(10).astype(F32)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert max_abs(oracle.linear(x, w, b), want) < 1e-4


# ---- affine int4 / int8 ------------------------------------------------------------------------


def test_pack_order_is_little_endian():
    assert oracle.pack_affine(np.arange(1, 9)[None], 4)[0, 0] == 0x87654321
    assert oracle.pack_affine(np.array([[1, 2, 3, 4]]), 8)[0, 0] == 0x04030201
    codes = _rng(8).integers(0, 16, (3, 64))
    assert np.array_equal(oracle.unpack_affine(oracle.pack_affine(codes, 4), 4), codes)
    codes = _rng(9).integers(0, 256, (3, 64))
    assert np.array_equal(oracle.unpack_affine(oracle.pack_affine(codes, 8), 8), codes)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_is_exact_product_one_add_one_rne_over_all_codes(bits):
    levels = 1 << bits
    r = _rng(bits)
    scales = oracle.to_bf16(np.abs(r.standard_normal(64)).astype(F32) * 0.01 + 1e-4)
    biases = oracle.to_bf16(r.standard_normal(64).astype(F32) * 0.05)
    n = 64
    k = 128 if bits == 4 else 512
    codes = np.tile(np.arange(levels), (n, k // levels))  # every code in every group of 64 (int4)
    words = oracle.pack_affine(codes, bits)
    groups = k // 64
    s = np.repeat(scales[:, None], groups, 1)
    b = np.repeat(biases[:, None], groups, 1)
    got = oracle.dequantize_affine(words, s, b, group_size=64, bits=bits)
    for row in range(0, n, 7):
        for col in range(k):
            exact = float(s[row, col // 64]) * float(codes[row, col])  # exact in float64 too
            assert float(F32(exact)) == exact  # the bf16 x code product is exact in fp32
            summed = F32(F32(exact) + F32(b[row, col // 64]))
            assert got[row, col] == _nearest_bf16_by_search(float(summed))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantizer_error_is_within_half_a_step(bits):
    r = _rng(10 + bits)
    w = (r.standard_normal((16, 256)) * 0.02).astype(F32)
    words, scales, biases = oracle.quantize_affine(w, 64, bits)
    deq = oracle.dequantize_affine(words, scales, biases, group_size=64, bits=bits)
    step = np.repeat(scales, 64, axis=1)
    # half a step plus the bf16 roundings of bias and result
    assert np.all(np.abs(deq - w) <= step * 0.5 + np.abs(w) * 2**-7 + np.repeat(np.abs(biases), 64, 1) * 2**-7 + 1e-7)


# ---- mxfp8 (OCP MX: E4M3 elements, E8M0 group scales) --------------------------------------------


def test_e4m3_and_e8m0_decode_match_torch_float8_over_all_codes():
    codes = np.arange(256)
    as_torch = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    for ours, dtype in ((oracle.e4m3_decode(codes), torch.float8_e4m3fn), (oracle.e8m0_scale(codes), torch.float8_e8m0fnu)):
        theirs = as_torch.view(dtype).float().numpy()
        assert np.array_equal(np.isnan(ours), np.isnan(theirs))
        assert np.array_equal(ours[~np.isnan(ours)], theirs[~np.isnan(theirs)])
    v = oracle.e4m3_decode(codes)
    assert v[0x7E] == 448 and v[0x01] == 2.0 ** -9 and v[0x38] == 1 and np.isnan(v[0x7F])


def test_e4m3_encode_is_torch_rne_below_saturation_and_saturates_at_448():
    r = _rng(30)
    v = (r.standard_normal(200000) * np.exp2(r.integers(-14, 9, 200000))).astype(F32)
    v = np.concatenate([np.clip(v, -460, 460), [0.0, -0.0, 2.0 ** -10, 3 * 2.0 ** -11, 1.5 * 2.0 ** -9, 2.5 * 2.0 ** -9, 240, 248]])
    theirs = torch.from_numpy(v.astype(F32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.e4m3_encode(v), theirs)
    assert list(oracle.e4m3_encode([464, 1e9, -1e9, np.inf])) == [0x7E, 0x7E, 0xFE, 0x7E]
    codes = np.arange(256)
    finite = ~np.isnan(oracle.e4m3_decode(codes))
    assert np.array_equal(oracle.e4m3_encode(oracle.e4m3_decode(codes))[finite], codes[finite])


def test_mxfp8_identity_matches_reference_binding_test():
    """``tests/models/ltx2/weights/test_family.py:262-283``: ``mx.quantize(eye(32), 32, 8,
    "mxfp8")`` bound as a quantized linear returns its input."""
    words, scales = oracle.quantize_mxfp8(np.eye(32, dtype=F32))
    assert words.shape == (32, 8) and words.dtype == np.uint32 and scales.shape == (32, 1)
    x = np.ones((1, 32), F32)
    assert np.array_equal(oracle.mxfp8_linear(x, words, scales), x)
    assert np.array_equal(oracle.mxfp8_linear(x, words, scales, transposed=False), x)


def test_mxfp8_scale_is_ocp_shared_exponent_and_error_within_half_an_element_step():
    r = _rng(31)
    w = (r.standard_normal((24, 256)) * np.exp2(r.integers(-6, 3, (24, 1)))).astype(F32)
    w[3, :32] = 0.0  # an all-zero group
    words, scales = oracle.quantize_mxfp8(w)
    groups = np.abs(w.reshape(24, 8, 32)).max(-1)
    expect = np.where(groups > 0, np.floor(np.log2(np.maximum(groups, 1e-30))) - 8 + 127, 0)
    assert np.array_equal(scales, expect.astype(np.uint8))
    deq = oracle.dequantize_mxfp8(words, scales)
    assert np.all(deq[3, :32] == 0)
    # one E4M3 step at |v| is 2^(floor(log2|v|) - 3) (2^-9 below the normal range), times the scale;
    # values scaled past 448 saturate there
    s = np.repeat(np.exp2(scales.astype(np.float64) - 127), 32, 1)
    scaled = np.abs(w) / s
    step = np.exp2(np.maximum(np.floor(np.log2(np.maximum(scaled, 1e-30))), -6) - 3) * s
    bound = np.where(scaled > 448, (scaled - 448) * s, step / 2) + np.abs(w) * 2.0 ** -9
    assert np.all(np.abs(deq - w) <= bound)


def test_mxfp8_pretransposed_layout_groups_the_output_axis():
    r = _rng(32)
    w = oracle.to_bf16((r.standard_normal((64, 96)) * 0.1).astype(F32))  # (out, in)
    x = oracle.to_bf16(r.standard_normal((5, 96)).astype(F32))
    plain = oracle.quantize_mxfp8(w)
    pre = oracle.quantize_mxfp8(np.ascontiguousarray(w.T))  # (in, out / 4), groups along out
    assert pre[0].shape == (96, 16) and pre[1].shape == (96, 2)
    ref_plain = oracle.linear(x, oracle.dequantize_mxfp8(*plain))
    ref_pre = oracle.linear(x, np.ascontiguousarray(oracle.dequantize_mxfp8(*pre).T))
    assert np.array_equal(oracle.mxfp8_linear(x, *plain), ref_plain)
    assert np.array_equal(oracle.mxfp8_linear(x, *pre, transposed=False), ref_pre)
    assert rel_l2(ref_pre, oracle.linear(x, w)) < 0.05


# ---- block compositions --------------------------------------------------------------------------


def _tiny_ltx_params(d=64, heads=2, seed=0):
    r = _rng(100 + seed)
    p = {}
    for a in ("attn1", "attn2"):
        for n in ("to_q", "to_k", "to_v", "to_out"):
            p[f"{a}.{n}.weight"] = (r.standard_normal((d, d)) * 0.1).astype(F32)
            p[f"{a}.{n}.bias"] = (r.standard_normal(d) * 0.1).astype(F32)
        p[f"{a}.to_gate_logits.weight"] = (r.standard_normal((heads, d)) * 0.1).astype(F32)
        p[f"{a}.to_gate_logits.bias"] = np.zeros(heads, F32)
        p[f"{a}.q_norm.weight"] = np.ones(d, F32)
        p[f"{a}.k_norm.weight"] = np.ones(d, F32)
    p["ff.proj_in.weight"] = (r.standard_normal((4 * d, d)) * 0.1).astype(F32)
    p["ff.proj_in.bias"] = np.zeros(4 * d, F32)
    p["ff.proj_out.weight"] = (r.standard_normal((d, 4 * d)) * 0.1).astype(F32)
    p["ff.proj_out.bias"] = np.zeros(d, F32)
    p["ada"] = (r.standard_normal((9, d)) * 0.5).astype(F32)
    p["prompt"] = (r.standard_normal((2, d)) * 0.5).astype(F32)
    return p


def _tiny_inputs(d=64, heads=2, t=6, tc=3):
    r = _rng(200)
    x = r.standard_normal((t, d)).astype(F32)
    ctx = r.standard_normal((tc, d)).astype(F32)
    pos = np.zeros((1, 3, t, 2), F32)
    pos[0, 2, :, 0] = np.arange(t)
    pos[0, 2, :, 1] = np.arange(t) + 1
    pe = oracle.precompute_freqs_cis(pos, dim=d, use_middle_indices_grid=True, num_attention_heads=heads)
    return x, ctx, pe


def test_ltx_block_gate_rows_switch_each_residual_branch():
    """Gates are ada rows 2 (self-attention), 8 (text) and 5 (feed-forward): zeroing exactly
    those returns the input; zeroing all but one changes the output only through that branch."""
    p = _tiny_ltx_params()
    x, ctx, pe = _tiny_inputs()
    off = dict(p, ada=p["ada"].copy())
    off["ada"][[2, 5, 8]] = 0
    assert np.array_equal(oracle.ltx_video_block(off, x, ctx, pe, heads=2), x)
    for keep in (2, 5, 8):
        only = dict(p, ada=p["ada"].copy())
        only["ada"][[g for g in (2, 5, 8) if g != keep]] = 0
        out = oracle.ltx_video_block(only, x, ctx, pe, heads=2)
        assert not np.array_equal(out, x)
        scrambled = dict(only)
        # perturb the weights of every branch except the kept one: the output must not move
        for prefix, g in (("attn1", 2), ("attn2", 8), ("ff", 5)):
            if g == keep:
                continue
            for key in [k for k in only if k.startswith(prefix) and k.endswith("weight")]:
                scrambled[key] = only[key] * F32(1.5)
        assert np.array_equal(oracle.ltx_video_block(scrambled, x, ctx, pe, heads=2), out)


def test_ltx_block_text_branch_reads_modulated_context():
    """With one text token the cross-attention weights are all 1, so the text branch is
    to_out(to_v(modulate(ctx)) * gate) + bias for every query: a row-constant term."""
    p = _tiny_ltx_params()
    x, ctx, pe = _tiny_inputs(tc=1)
    only = dict(p, ada=p["ada"].copy())
    only["ada"][[2, 5]] = 0
    out = oracle.ltx_video_block(only, x, ctx, pe, heads=2)
    query = oracle.adaln(x, only["ada"][7], only["ada"][6])
    gate = 2 / (1 + np.exp(-(query @ p["attn2.to_gate_logits.weight"].T + p["attn2.to_gate_logits.bias"])))
    c = oracle.modulate(ctx, p["prompt"][1], p["prompt"][0])
    v = c @ p["attn2.to_v.weight"].T + p["attn2.to_v.bias"]
    o = (np.repeat(v, x.shape[0], 0).reshape(x.shape[0], 2, -1) * gate[:, :, None]).reshape(x.shape)
    want = x + (o @ p["attn2.to_out.weight"].T + p["attn2.to_out.bias"]) * only["ada"][8]
    assert max_abs(out, want) < 1e-5


def test_flux_double_block_gates_and_stream_order():
    r = _rng(300)
    d, heads, dh = 64, 2, 32
    p = {}
    for name in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out", "to_add_out"):
        p[f"attn.{name}.weight"] = (r.standard_normal((d, d)) * 0.1).astype(F32)
    for name in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        p[f"attn.{name}.weight"] = np.ones(dh, F32)
    for prefix in ("ff", "ff_context"):
        p[f"{prefix}.linear_in.weight"] = (r.standard_normal((96, d)) * 0.1).astype(F32)
        p[f"{prefix}.linear_out.weight"] = (r.standard_normal((d, 48)) * 0.1).astype(F32)
    image = r.standard_normal((5, d)).astype(F32)
    text = r.standard_normal((3, d)).astype(F32)
    im = (r.standard_normal((6, d)) * 0.5).astype(F32)
    tm = (r.standard_normal((6, d)) * 0.5).astype(F32)
    rope = (np.ones((8, dh), F32), np.zeros((8, dh), F32))
    im0, tm0 = im.copy(), tm.copy()
    im0[[2, 5]] = 0
    tm0[[2, 5]] = 0
    i_out, t_out = oracle.flux_double_block(p, image, text, im0, tm0, rope, heads=heads)
    assert np.array_equal(i_out, image) and np.array_equal(t_out, text)
    # the image output depends on the text stream only through attention
    i1, _ = oracle.flux_double_block(p, image, text, im, tm, rope, heads=heads)
    tm_ff = tm.copy()
    tm_ff[[3, 4, 5]] += 1.0  # text feed-forward modulation only
    i2, t2 = oracle.flux_double_block(p, image, text, im, tm_ff, rope, heads=heads)
    assert np.array_equal(i1, i2) and not np.array_equal(t2, _)


def _krea_params(r, hidden, heads, kv_heads, ff=48):
    dh = hidden // heads
    p = {}
    for name, rows in (("to_q", hidden), ("to_k", kv_heads * dh), ("to_v", kv_heads * dh), ("to_gate", hidden),
                       ("to_out", hidden)):
        p[f"attn.{name}.weight"] = (r.standard_normal((rows, hidden)) * 0.2).astype(F32)
    p["attn.norm_q.weight"] = (r.standard_normal(dh) * 0.1).astype(F32)
    p["attn.norm_k.weight"] = (r.standard_normal(dh) * 0.1).astype(F32)
    p["norm1.weight"] = (r.standard_normal(hidden) * 0.1).astype(F32)
    p["norm2.weight"] = (r.standard_normal(hidden) * 0.1).astype(F32)
    p["ff.gate.weight"] = (r.standard_normal((ff, hidden)) * 0.2).astype(F32)
    p["ff.up.weight"] = (r.standard_normal((ff, hidden)) * 0.2).astype(F32)
    p["ff.down.weight"] = (r.standard_normal((hidden, ff)) * 0.2).astype(F32)
    return p


def test_krea_grouped_query_attention_reads_kv_head_h_over_group():
    """Grouped-query attention equals full multi-head attention whose K/V weights repeat each
    K/V head's rows for its group of query heads ``h // (H / Hkv)`` (MLX SDPA GQA semantics):
    an ``h % Hkv`` mapping or a transposed head order fails this."""
    r = _rng(401)
    hidden, heads, kv_heads, t = 32, 4, 2, 6
    dh = hidden // heads
    p = _krea_params(r, hidden, heads, kv_heads)
    x = r.standard_normal((t, hidden)).astype(F32)
    ang = r.uniform(-2, 2, (t, dh // 2)).astype(F32)
    rot = (np.repeat(np.cos(ang), 2, -1), np.repeat(np.sin(ang), 2, -1))
    got = oracle.krea_attention(p, "attn", x, heads=heads, kv_heads=kv_heads, eps=1e-6, rotary=rot)
    full = dict(p)
    for name in ("to_k", "to_v"):
        w = p[f"attn.{name}.weight"].reshape(kv_heads, dh, hidden)
        full[f"attn.{name}.weight"] = np.repeat(w, heads // kv_heads, axis=0).reshape(hidden, hidden)
    want = oracle.krea_attention(full, "attn", x, heads=heads, kv_heads=heads, eps=1e-6, rotary=rot)
    assert max_abs(got, want) < 1e-6
    swapped = dict(full)
    for name in ("to_k", "to_v"):  # the other head order really changes the result
        w = p[f"attn.{name}.weight"].reshape(kv_heads, dh, hidden)
        swapped[f"attn.{name}.weight"] = np.tile(w, (heads // kv_heads, 1, 1)).reshape(hidden, hidden)
    other = oracle.krea_attention(swapped, "attn", x, heads=heads, kv_heads=heads, eps=1e-6, rotary=rot)
    assert max_abs(got, other) > 1e-3


def test_krea_block_gates_and_modulation_order():
    """Zero pre/post gates (chunks 2 and 5 of the official order) leave x unchanged; the output
    gate is sigmoid over the full width (a zero to_gate weight halves the attention output)."""
    r = _rng(402)
    hidden, heads, kv_heads, t = 32, 4, 2, 5
    p = _krea_params(r, hidden, heads, kv_heads)
    x = r.standard_normal((t, hidden)).astype(F32)
    mod = (r.standard_normal((6, hidden)) * 0.3).astype(F32)
    mod0 = mod.copy()
    mod0[[2, 5]] = 0
    assert np.array_equal(oracle.krea_block(p, x, mod0, None, heads=heads, kv_heads=kv_heads), x)
    only_attn = mod.copy()
    only_attn[5] = 0
    pz = dict(p)
    pz["attn.to_gate.weight"] = np.zeros_like(p["attn.to_gate.weight"])
    half = oracle.krea_block(pz, x, only_attn, None, heads=heads, kv_heads=kv_heads) - x
    p_out = dict(pz)
    p_out["attn.to_out.weight"] = p["attn.to_out.weight"] * F32(2.0)
    full = oracle.krea_block(p_out, x, only_attn, None, heads=heads, kv_heads=kv_heads) - x
    assert max_abs(2 * half, full) < 1e-5
    assert max_abs(half, 0) > 1e-3


# ---- FP4 (mxfp4 / nvfp4) -------------------------------------------------------------------------


def test_e2m1_decode_is_the_published_table():
    """OCP MX v1.0 E2M1: codes 0..7 are 0, 0.5, 1, 1.5, 2, 3, 4, 6 (the standard's table, typed
    here, not derived from the oracle's field formula); bit 3 is the sign."""
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    got = oracle.e2m1_decode(np.arange(16))
    assert got[:8].tolist() == table
    assert (-got[8:]).tolist() == table and np.all(np.signbit(got[8:]))


def test_e2m1_encode_rounds_to_nearest_even_and_saturates():
    codes = np.arange(16)
    assert np.array_equal(oracle.e2m1_encode(oracle.e2m1_decode(codes)), codes)
    grid = oracle.e2m1_decode(np.arange(8)).astype(np.float64)
    # brute force: the nearest grid value, ties to the even code (codes 0, 2, 4, 6 have mantissa 0)
    r = np.random.default_rng(3)
    x = np.concatenate([r.uniform(-7, 7, 20000), (grid[:-1] + grid[1:]) / 2, -(grid[:-1] + grid[1:]) / 2])
    a = np.minimum(np.abs(x), 6.0)
    dist = np.abs(a[:, None] - grid[None, :])
    best = dist.min(axis=1, keepdims=True)
    cand = np.where(dist == best, np.arange(8)[None, :], 99)
    even = np.where(cand % 2 == 0, cand, 99).min(axis=1)
    expect = np.where(even < 99, even, cand.min(axis=1)) | np.where(np.signbit(x), 8, 0)
    assert np.array_equal(oracle.e2m1_encode(x), expect)
    assert oracle.e2m1_encode(np.array([7.0, 1e30, -6.5]))[:].tolist() == [7, 7, 15]
    assert oracle.e2m1_encode(np.array([np.nan]))[0] == 0


@pytest.mark.parametrize("mode,group", [("mxfp4", 32), ("nvfp4", 16)])
def test_fp4_identity_round_trips(mode, group):
    """The reference's binding test packs an identity and gets its input back
    (``tests/models/ltx2/weights/test_family.py:262-283``, mxfp8). mxfp4 represents 0 and 1 exactly
    (scale 2^-2, code 4); nvfp4's scale is E4M3(amax / 6), exact for amax = 6 (scale 1, code 6),
    so ``6 * eye`` round-trips there (1 / 6 has no E4M3 form: an nvfp4 identity does not)."""
    eye = np.eye(2 * group, dtype=np.float32) * (6.0 if mode == "nvfp4" else 1.0)
    q = oracle.quantize_mxfp4(eye) if mode == "mxfp4" else oracle.quantize_nvfp4(eye)
    assert np.array_equal(oracle.dequantize_fp4(*q, mode=mode), eye)
    x = np.random.default_rng(1).standard_normal((3, 2 * group)).astype(np.float32)
    assert np.array_equal(oracle.fp4_linear(x, *q, mode=mode), oracle.linear(x, eye))


def test_mxfp4_scale_is_the_ocp_shared_exponent_and_error_within_half_a_step():
    r = np.random.default_rng(2)
    w = (r.standard_normal((64, 128)) * np.exp2(r.integers(-8, 8, (64, 1)))).astype(np.float32)
    words, scales = oracle.quantize_mxfp4(w)
    g = w.reshape(64, 4, 32).astype(np.float64)
    amax = np.abs(g).max(-1)
    assert np.array_equal(scales.astype(np.int64) - 127, np.floor(np.log2(amax)).astype(np.int64) - 2)
    deq = oracle.dequantize_fp4(words, scales, mode="mxfp4").reshape(64, 4, 32).astype(np.float64)
    unit = np.exp2(scales.astype(np.float64) - 127)[..., None]  # 2^X: the element grid's unit
    # below 2 units the grid step is 0.5 unit, then 1, then 2 (saturation above 6 units cannot
    # happen: amax < 8 units)
    step = np.where(np.abs(g) < 2 * unit, 0.5 * unit, np.where(np.abs(g) < 4 * unit, unit, 2 * unit))
    assert np.all(np.abs(deq - g) <= step / 2 + np.maximum(0, np.abs(g) - 6 * unit))


def test_nvfp4_scale_is_the_e4m3_of_amax_over_6():
    r = np.random.default_rng(4)
    w = (r.standard_normal((16, 64)) * 0.05).astype(np.float32)
    words, scales = oracle.quantize_nvfp4(w)
    amax = np.abs(w.reshape(16, 4, 16)).max(-1)
    # torch's E4M3 (RNE) cast of amax / 6 is the scale byte
    import torch

    expect = torch.from_numpy((amax / np.float32(6.0)).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(scales, expect.numpy())
    deq = oracle.dequantize_fp4(words, scales, mode="nvfp4")
    s = np.repeat(oracle.e4m3_decode(scales).astype(np.float64), 16, axis=1)
    assert np.all(np.abs(deq - w) <= s * 1.0 + 1e-12)  # at most half the largest E2M1 step (2) per unit


def test_torch_cpu_config1_block_matches_the_numpy_restatement():
    """The CPU baseline's torch restatement (``oracle/torch_cpu.py``: torch's layer norm, linear
    and SDPA kernels) against the numpy oracle on the full config-1 block, both FP32: they agree
    to FP32 reassociation. A dropped term, a swapped gate or a transposed operand in either moves
    the relative L2 error to order 1."""
    from kinomlx_amd import workloads
    from oracle import torch_cpu

    spec = workloads.CONFIGS[1]
    p = workloads.flux_params(spec, 0)
    inputs = workloads.flux_inputs(spec, 0)
    op = {k: v.float().numpy() for k, v in p.items()}
    image, text = inputs["image"][0].float().numpy(), inputs["text"][0].float().numpy()
    cos, sin = (t.numpy() for t in workloads.flux_rope(spec))
    ri, rt = oracle.config1_double_block(op, image, text, op["image_mod"], op["text_mod"], (cos, sin),
                                         heads=spec.heads)
    tp = torch_cpu.to_torch(op)
    gi, gt = torch_cpu.config1_double_block(tp, torch.from_numpy(image), torch.from_numpy(text), tp["image_mod"],
                                            tp["text_mod"], (torch.from_numpy(cos), torch.from_numpy(sin)),
                                            heads=spec.heads)
    for got, ref in ((gi.numpy(), ri), (gt.numpy(), rt)):
        assert got.shape == ref.shape
        assert rel_l2(got, ref) < 1e-5
        assert max_abs(got, ref) <= 1e-4 * float(np.abs(ref).max())
