"""Kernel parity on the GPU: each HIP kernel (through the C ABI via the operator surface) against
the CPU oracle on the same seeded inputs.

Bars: bit-exact for the split/pair RoPE standalone kernels and the int4/int8 dequantization;
elsewhere the tolerance is written in each test (bf16 output vs the FP32 oracle).
"""

import os

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import _lib
from kinomlx_amd.kernels import fused_ops, mpp_linear, quantized, split_rope
from kinomlx_amd.ltx2 import attention as ltx_attention
from kinomlx_amd.ltx2 import dense_attention, transformer
from tests.conftest import cosine, max_abs, rel_l2

pytestmark = pytest.mark.gpu
F32 = np.float32


def _bf(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32)).to(device).to(torch.bfloat16)


def _f32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32)).to(device)


def _np(t):
    return t.float().cpu().numpy()


def _rng(seed):
    return np.random.default_rng(seed)


def _within_one_ulp(got, ref):
    """|got - ref| within one bf16 ulp of ref (2^-7 relative, plus a tiny absolute floor)."""
    return np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-6)


# ---- norms ---------------------------------------------------------------------------------------


@pytest.mark.parametrize("dim", [512, 1024, 4096, 1000])
@pytest.mark.parametrize("kind", ["rms", "layer"])
def test_modulated_norm_matches_oracle(device, dim, kind):
    r = _rng(dim)
    x = oracle.to_bf16((r.standard_normal((37, dim)) * 2 + 0.5).astype(F32))
    scale = (r.standard_normal(dim) * 0.5).astype(F32)
    shift = (r.standard_normal(dim) * 0.5).astype(F32)
    if kind == "rms":
        got = transformer.adaln(_bf(x, device), _f32(scale, device), _f32(shift, device), 1e-6)
        ref = oracle.adaln(x, scale, shift)
    else:
        got = transformer.layer_norm_modulate(_bf(x, device), _f32(shift, device), _f32(scale, device))
        ref = oracle.normalized(x, shift, scale)
    # one rounding of an FP32 result: within one bf16 ulp (reduction order may differ)
    assert _within_one_ulp(_np(got), ref)


def test_modulated_norm_per_token_and_per_batch_rows(device):
    r = _rng(11)
    b, t, d = 2, 9, 1024
    x = oracle.to_bf16(r.standard_normal((b, t, d)).astype(F32))
    per_batch = (r.standard_normal((b, 1, d)) * 0.3).astype(F32)
    per_token = (r.standard_normal((b, t, d)) * 0.3).astype(F32)
    got = transformer.adaln(_bf(x, device), _f32(per_batch, device), _f32(per_token, device), 1e-6)
    assert _within_one_ulp(_np(got), oracle.adaln(x, per_batch, per_token))


@pytest.mark.parametrize(("dim", "wdtype", "offset"), [(4096, "bf16", 0.0), (256, "f32", 0.0), (3840, "bf16", 1.0)])
def test_weighted_rms_norm_matches_oracle(device, dim, wdtype, offset):
    """Relative L2 <= 5e-5 before the bf16 store is the reference's bar
    (tests/kernels/test_fused_ops.py:68-84); after one bf16 rounding we bound each element by
    one ulp."""
    r = _rng(dim + 1)
    x = oracle.to_bf16((r.standard_normal((2, 5, dim)) * 4).astype(F32))
    w = (r.standard_normal(dim) * (0.02 if offset else 0.1) + (0.0 if offset else 1.0)).astype(F32)
    w = oracle.to_bf16(w) if wdtype == "bf16" else w
    wt = _bf(w, device) if wdtype == "bf16" else _f32(w, device)
    got = fused_ops.rms_norm(_bf(x, device), wt, 1e-6, weight_offset=offset)
    assert _within_one_ulp(_np(got), oracle.rms_norm(x, w, 1e-6, weight_offset=offset))


@pytest.mark.parametrize(("dim", "heads"), [(4096, 32), (1024, 16), (2048, 16), (1024, 8)])
@pytest.mark.parametrize("wdtype", ["bf16", "f32"])
def test_fused_norm_and_split_rope_matches_oracle(device, dim, heads, wdtype):
    """Full-width RMSNorm + split RoPE: 128-wide heads take the kernel whose lanes own both halves
    of a head, 64-wide heads the lane-exchange kernel; bf16 and fp32 norm weights."""
    r = _rng(dim + heads)
    t = 41
    dh = dim // heads
    x = oracle.to_bf16((r.standard_normal((1, t, dim)) * 3).astype(F32))
    w = (r.standard_normal(dim) * 0.05 + 1).astype(F32)
    if wdtype == "bf16":
        w = oracle.to_bf16(w)
    pos = np.zeros((1, 3, t, 2), F32)
    pos[0, 0, :, 0] = np.arange(t) // 7
    pos[0, 1, :, 0] = np.arange(t) % 7
    pos[0, 2, :, 0] = np.arange(t) % 5
    pos[..., 1] = pos[..., 0] + 1
    cos, sin = oracle.precompute_freqs_cis(pos, dim=dim, use_middle_indices_grid=True, num_attention_heads=heads)
    norm = ltx_attention.RMSNorm(dim, weight=_bf(w, device) if wdtype == "bf16" else _f32(w, device))
    # token-major storage viewed head-major, as precompute_freqs_cis returns it
    cos_d = _f32(cos.transpose(0, 2, 1, 3), device).transpose(1, 2)
    sin_d = _f32(sin.transpose(0, 2, 1, 3), device).transpose(1, 2)
    got = _np(ltx_attention.norm_rope(_bf(x, device), norm, (cos_d, sin_d), heads))
    ref = oracle.split_rope(oracle.rms_norm(x, w, 1e-6), cos, sin)
    assert rel_l2(got, ref) < 4e-3 and max_abs(got, ref) < 2e-2 * max(1.0, np.abs(ref).max() / 4)
    assert dh in (64, 128)


@pytest.mark.parametrize(("dim", "batch", "table_batch", "wdtype"),
                         [(4096, 1, 1, torch.bfloat16), (1024, 2, 2, torch.float32), (2048, 2, 1, torch.bfloat16)])
def test_fused_qk_norm_rope_is_bit_identical_to_two_passes(device, dim, batch, table_batch, wdtype):
    """kx_qk_rmsnorm_rope_bf16 (Q and K rows of one fused projection, tables read once) against
    two kx_rmsnorm_rope_bf16 passes: the same arithmetic per row, so the same bits."""
    heads, t = dim // 128, 37
    r = _rng(dim + batch)
    qkv = torch.from_numpy((r.standard_normal((batch, t, 3 * dim)) * 2).astype(F32)).to(device).to(torch.bfloat16)
    wq = torch.from_numpy((r.standard_normal(dim) * 0.05 + 1).astype(F32)).to(device).to(wdtype)
    wk = torch.from_numpy((r.standard_normal(dim) * 0.05 + 1).astype(F32)).to(device).to(wdtype)
    qn, kn = ltx_attention.RMSNorm(dim, weight=wq), ltx_attention.RMSNorm(dim, weight=wk)
    ang = r.uniform(-3, 3, (table_batch, heads, t, 64)).astype(F32)
    cos = torch.from_numpy(np.ascontiguousarray(np.cos(ang).transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    sin = torch.from_numpy(np.ascontiguousarray(np.sin(ang).transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    q_raw, k_raw = qkv[..., :dim], qkv[..., dim:2 * dim]
    fused = ltx_attention.norm_rope_qk(q_raw, k_raw, qn, kn, (cos, sin), heads)
    assert fused is not None
    assert torch.equal(fused[0], ltx_attention.norm_rope(q_raw, qn, (cos, sin), heads))
    assert torch.equal(fused[1], ltx_attention.norm_rope(k_raw, kn, (cos, sin), heads))


@pytest.mark.parametrize(("norm_width", "rope_kind"), [(128, "pair"), (64, "pair"), (128, "none")])
def test_per_head_norm_and_pair_rope_matches_oracle(device, norm_width, rope_kind):
    r = _rng(norm_width)
    t, heads = 23, 4096 // norm_width if norm_width == 128 else 16
    dim = heads * norm_width
    x = oracle.to_bf16((r.standard_normal((t, dim)) * 2).astype(F32))
    w = oracle.to_bf16((r.standard_normal(norm_width) * 0.05 + 1).astype(F32))
    ang = np.repeat(r.uniform(-3, 3, (t, norm_width // 2)), 2, axis=-1).astype(F32)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    out = torch.empty((t, dim), dtype=torch.bfloat16, device=device)
    kind = _lib.KX_ROPE_PAIR if rope_kind == "pair" else _lib.KX_ROPE_NONE
    _lib.launch_rmsnorm_rope(
        _bf(x, device), out, _bf(w, device), 1e-6, 0.0, norm_width=norm_width, rope_kind=kind,
        cos=_f32(cos, device), sin=_f32(sin, device), table_ld=norm_width, table_hs=0, tokens=t, head_dim=norm_width,
    )
    normed = oracle.rms_norm(x.reshape(t, heads, norm_width), w, 1e-6)
    ref = oracle.pair_rope(normed, cos[:, None], sin[:, None]) if rope_kind == "pair" else normed
    got = _np(out).reshape(t, heads, norm_width)
    assert rel_l2(got, ref) < 4e-3 and cosine(got, ref) > 0.99999


# ---- RoPE (bit-exact) -------------------------------------------------------------------------


def _tables(batch, heads, tokens, half, token_major, seed=0):
    count = batch * tokens * heads * half
    angles = np.arange(count, dtype=F32) * F32(0.2718281)
    if token_major:
        angles = angles.reshape(batch, tokens, heads, half).transpose(0, 2, 1, 3)
    else:
        angles = angles.reshape(batch, heads, tokens, half)
    return np.cos(angles).astype(F32), np.sin(angles).astype(F32)


@pytest.mark.parametrize(("batch", "table_batch", "token_major"), [(1, 1, True), (2, 1, True), (2, 2, False)])
@pytest.mark.parametrize("half", [24, 5])
def test_split_rope_is_bit_exact(device, batch, table_batch, token_major, half):
    """tests/kernels/test_split_rope.py:31-50 shapes (H=4, T=13, half=24) and the ragged
    self-test case (half=5), against the oracle's exact FP32 op order."""
    heads, tokens = 4, 13
    r = _rng(611 + half)
    x = oracle.to_bf16((r.standard_normal((batch, tokens, heads * 2 * half)) * 3).astype(F32))
    cos, sin = _tables(table_batch, heads, tokens, half, token_major)
    cos_d, sin_d = _f32(cos, device), _f32(sin, device)
    value = _bf(x, device)
    assert split_rope.applies(value, cos_d, sin_d)
    got = _np(split_rope.rotate(value, cos_d, sin_d))
    ref = oracle.to_bf16(oracle.split_rope(x, cos, sin))  # tables broadcast over the batch when shared
    assert np.array_equal(got, ref)


def test_pair_rope_is_bit_exact(device):
    r = _rng(5)
    t, heads, dh = 19, 3, 64
    x = oracle.to_bf16((r.standard_normal((t, heads * dh)) * 3).astype(F32))
    ang = np.repeat(r.uniform(-3, 3, (t, dh // 2)), 2, axis=-1).astype(F32)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    out = torch.empty((t, heads * dh), dtype=torch.bfloat16, device=device)
    _lib.launch_rope_pair(_bf(x, device), out, _f32(cos, device), _f32(sin, device), heads=heads, head_dim=dh,
                          table_ld=dh, table_hs=0, tokens=t, table_batched=False)
    ref = oracle.to_bf16(oracle.pair_rope(x.reshape(t, heads, dh), cos[:, None], sin[:, None]).reshape(t, -1))
    assert np.array_equal(_np(out), ref)


# ---- activations ---------------------------------------------------------------------------------


def _gelu64(x):
    """tanh GELU with the clamped inner argument, in float64 (the exact value of the formula)."""
    x = np.asarray(x, dtype=np.float64)
    inner = np.clip(0.7978845608028654 * (x + 0.044715 * x ** 3), -10.0, 10.0)
    return 0.5 * x * (1.0 + np.tanh(inner))


def _silu64(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("op", ["gelu", "silu"])
def test_activations_round_the_exact_value_once(device, op):
    """linspace(-8, 8, 65536) as in tests/kernels/test_fused_ops.py:18-65 against the float64
    value of the same formula rounded once to bf16: every element within one bf16 ulp of the
    float64 value, at least 99.9% bit-equal to its correctly rounded bf16, and the reference's
    own bound (max abs 4e-6 for GELU, 0 for SiLU) met by at least 99.9% of the elements. The
    FP32 restatement of the tanh form cancels in 1 + tanh(u) for negative u, so it is checked
    against float64 too rather than used as the bit pattern to hit."""
    x = oracle.to_bf16(np.linspace(-8, 8, 65536, dtype=F32))
    fn, exact = (fused_ops.gelu_approx, _gelu64) if op == "gelu" else (fused_ops.silu, _silu64)
    got = _np(fn(_bf(x, device)))
    truth = exact(x)
    ref = oracle.to_bf16(truth.astype(F32))
    assert _within_one_ulp(got, truth.astype(F32))
    assert np.mean(got == ref) >= 0.999
    bound = 4e-6 if op == "gelu" else 0.0
    assert np.mean(np.abs(got.astype(np.float64) - ref) <= bound) >= 0.999


def test_gelu_saturates_without_nan(device):
    x = oracle.to_bf16(np.linspace(-128, 128, 65536, dtype=F32))
    got = _np(fused_ops.gelu_approx(_bf(x, device)))
    assert np.all(np.isfinite(got))
    assert np.allclose(got, oracle.gelu_approx(x), rtol=1e-2, atol=1.3e-4)


def test_swiglu_matches_oracle(device):
    r = _rng(9)
    x = oracle.to_bf16((r.standard_normal((33, 2 * 96)) * 3).astype(F32))
    got = _np(fused_ops.swiglu(_bf(x, device)))
    assert _within_one_ulp(got, oracle.swiglu(x))


def test_modulate_gate_and_gated_residual(device):
    r = _rng(10)
    x = oracle.to_bf16(r.standard_normal((2, 7, 96)).astype(F32))
    y = oracle.to_bf16(r.standard_normal((2, 7, 96)).astype(F32))
    g = r.standard_normal((2, 1, 96)).astype(F32)
    s = r.standard_normal(96).astype(F32)
    xd, yd = _bf(x, device), _bf(y, device)
    assert _within_one_ulp(_np(transformer.gated_residual(xd, yd, _f32(g, device))), oracle.gated_residual(x, y, g))
    assert _within_one_ulp(_np(transformer.modulate(xd, _f32(s, device), _f32(g, device))), oracle.modulate(x, s, g))
    assert _within_one_ulp(_np(transformer.gate(yd, _f32(g, device))), oracle.gate(y, g))


# ---- linear ----------------------------------------------------------------------------------------


def _linear_case(m, n, k, seed, device, scale=1.0):
    r = _rng(seed)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5 * scale).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * k ** -0.5).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.5).astype(F32))
    return x, w, b


def _gemm_close(got, ref):
    """FP32 accumulation in another order, then one bf16 rounding: within one ulp of the value
    plus the FP32 sum's own rounding noise."""
    tol = np.abs(ref) * 2.0**-7 + 1e-4 * np.abs(ref).max()
    return np.all(np.abs(got - ref) <= tol)


@pytest.mark.parametrize("tile", ["auto", "0", "1", "2", "3", "4"])
@pytest.mark.parametrize(("m", "n", "k"), [(1056, 1040, 1024), (300, 96, 64), (7, 32, 200), (600, 520, 96)])
def test_linear_matches_oracle_for_every_tile(device, monkeypatch, tile, m, n, k):
    """Ragged against every tile shape (tests/kernels/test_mpp_linear.py:8-43 shape); K = 96 (a
    multiple of 32 but not of the direct-to-LDS kernel's 64-wide stages) takes the register-staged
    kernel on the auto path too."""
    if tile != "auto":
        monkeypatch.setenv("KX355_GEMM_TILE", tile)
    x, w, b = _linear_case(m, n, k, m + n + k, device)
    got = _np(mpp_linear.linear(_bf(x, device), _bf(w, device), _bf(b, device), transposed=True))
    assert _gemm_close(got, oracle.linear(x, w, b))
    got_nb = _np(mpp_linear.linear(_bf(x, device), _bf(w, device), None, transposed=True))
    assert _gemm_close(got_nb, oracle.linear(x, w))


@pytest.mark.parametrize("tile", ["0", "1", "2", "3"])
@pytest.mark.parametrize(("m", "n", "k"), [(1056, 1040, 1024), (512, 512, 256), (300, 96, 64), (513, 520, 192), (9, 8, 64)])
@pytest.mark.parametrize("epilogue", ["bias", "gelu_tanh", "gated_f32", "gated_bf16", "gated_f32_to_bf16", "gated_rows"])
def test_direct_to_lds_linear_every_tile_and_epilogue(device, monkeypatch, tile, m, n, k, epilogue):
    """The K % 32 == 0 direct-to-LDS kernel at each of its tiles (256x256, 192x256, 128x128, 64x128) on
    full tiles (the compile-time epilogue) and ragged M and N (partial tiles, clamped loads,
    masked stores) with each epilogue family: residual fp32 or bf16, output fp32 or bf16, one
    broadcast gate row or one gate row per output row."""
    monkeypatch.setenv("KX355_GEMM_LDS_TILE", tile)
    x, w, b = _linear_case(m, n, k, m + n + k + 1, device)
    lin = oracle.linear(x, w, b)
    if epilogue == "bias":
        got = _np(mpp_linear.linear(_bf(x, device), _bf(w, device), _bf(b, device), transposed=True))
        assert _gemm_close(got, lin)
    elif epilogue == "gelu_tanh":
        got = _np(mpp_linear.fused_linear(_bf(x, device), _bf(w, device), _bf(b, device), activation="gelu_tanh"))
        ref = oracle.gelu_approx(lin)
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 2e-4 * np.abs(ref).max() + 1e-6)
    else:
        r = _rng(m + n)
        resid = r.standard_normal((m, n)).astype(F32)
        gate = r.standard_normal((m, n) if epilogue == "gated_rows" else n).astype(F32)
        if epilogue == "gated_bf16":
            resid = oracle.to_bf16(resid)
            resid_t, out_dtype = _bf(resid, device), torch.float32
        elif epilogue == "gated_f32_to_bf16":
            resid_t, out_dtype = _f32(resid, device), torch.bfloat16
        else:
            resid_t, out_dtype = _f32(resid, device), torch.float32
        out = mpp_linear.fused_linear(_bf(x, device), _bf(w, device), _bf(b, device), residual=resid_t,
                                      gate=_f32(gate, device), out_dtype=out_dtype)
        ref = resid + gate * lin
        tol = 1e-5 * np.abs(ref) + 2e-5 * np.abs(ref).max()
        if out_dtype == torch.bfloat16:
            tol = tol + np.abs(ref) * 2.0**-8
        assert np.all(np.abs(_np(out) - ref) <= tol)


def test_linear_takes_in_out_weights(device):
    x, w, b = _linear_case(64, 48, 32, 3, device)
    got = _np(mpp_linear.linear(_bf(x, device), _bf(w.T, device), _bf(b, device), transposed=False))
    assert _gemm_close(got, oracle.linear(x, w, b))


@pytest.mark.parametrize("act", ["gelu_tanh", "silu", "sigmoid2"])
def test_linear_activation_epilogues(device, act):
    x, w, b = _linear_case(130, 200, 256, 4, device, scale=4.0)
    got = _np(mpp_linear.fused_linear(_bf(x, device), _bf(w, device), _bf(b, device), activation=act))
    lin = oracle.linear(x, w, b)
    ref = {"gelu_tanh": oracle.gelu_approx, "silu": oracle.silu,
           "sigmoid2": lambda v: 2.0 / (1.0 + np.exp(-v))}[act](lin)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 2e-4 * np.abs(ref).max() + 1e-6)


def test_linear_gated_residual_epilogue(device):
    x, w, b = _linear_case(2 * 70, 96, 128, 5, device)
    r = _rng(6)
    resid = oracle.to_bf16(r.standard_normal((2, 70, 96)).astype(F32))
    gate = r.standard_normal((2, 1, 96)).astype(F32)
    got = _np(mpp_linear.fused_linear(_bf(x.reshape(2, 70, 128), device), _bf(w, device), _bf(b, device),
                                      residual=_bf(resid, device), gate=_f32(gate, device)))
    ref = oracle.gated_residual(resid, oracle.linear(x, w, b).reshape(2, 70, 96), gate)
    assert _gemm_close(got, ref)


@pytest.mark.parametrize(("resid_dtype", "out_dtype"), [("f32", "f32"), ("f32", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("bits", [None, 4])
def test_linear_fp32_residual_stream(device, resid_dtype, out_dtype, bits):
    """The residual stream carried in FP32: resid and output each bf16 or fp32. An fp32 output
    is the FP32 epilogue value itself (no rounding): close to the oracle to FP32 accumulation
    noise; a bf16 output is that value rounded once."""
    m, n, k = 2 * 70, 96, 128
    x, w, b = _linear_case(m, n, k, 5, device)
    r = _rng(16)
    resid = r.standard_normal((2, 70, n)).astype(F32)
    if resid_dtype == "bf16":
        resid = oracle.to_bf16(resid)
    gate = r.standard_normal((2, 1, n)).astype(F32)
    resid_d = _f32(resid, device) if resid_dtype == "f32" else _bf(resid, device)
    od = torch.float32 if out_dtype == "f32" else torch.bfloat16
    xd = _bf(x.reshape(2, 70, k), device)
    if bits is None:
        outs = [mpp_linear.fused_linear(xd, _bf(w, device), _bf(b, device), residual=resid_d,
                                        gate=_f32(gate, device), out_dtype=od)]
        weight = w
    else:
        words, scales, biases = oracle.quantize_affine(w, 64, bits)
        layer = quantized.QuantizedLinear(
            torch.from_numpy(words.view(np.int32)).to(device), _bf(scales, device), _bf(biases, device),
            _bf(b, device), group_size=64, bits=bits)
        # the layer (dequantize, dense GEMM) and the in-mainloop kernel
        outs = [layer(xd, residual=resid_d, gate=_f32(gate, device), out_dtype=od),
                quantized.quantized_matmul(xd, layer.weight, layer.scales, layer.biases, group_size=64, bits=bits,
                                           bias=layer.bias, residual=resid_d, gate=_f32(gate, device), out_dtype=od)]
        weight = oracle.dequantize_affine(words, scales, biases, group_size=64, bits=bits)
    ref = oracle.gated_residual(resid, oracle.linear(x, weight, b).reshape(2, 70, n), gate)
    for out in outs:
        assert out.dtype == od
        got = _np(out)
        if out_dtype == "f32":
            assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 2e-5 * np.abs(ref).max())
        else:
            assert _gemm_close(got, ref)


@pytest.mark.parametrize("dim", [1024, 4096, 1000])
def test_modulated_norm_reads_an_fp32_residual_stream(device, dim):
    """AdaLN on an FP32 input (the block's residual stream between branches): bf16 output within
    one bf16 ulp of the FP32 oracle, and not equal to the result on the bf16-rounded input."""
    r = _rng(17)
    x = (r.standard_normal((37, dim)) * 2).astype(F32)
    shift = (r.standard_normal(dim) * 0.3).astype(F32)
    scale = (r.standard_normal(dim) * 0.3).astype(F32)
    out = transformer.adaln(_f32(x, device), _f32(scale, device), _f32(shift, device), 1e-6)
    assert out.dtype == torch.bfloat16
    got = _np(out)
    assert _within_one_ulp(got, oracle.adaln(x, scale, shift))
    rounded_input = oracle.to_bf16(oracle.adaln(oracle.to_bf16(x), scale, shift))
    assert not np.array_equal(got, rounded_input)


@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_linear_non_finite_inputs_stay_non_finite(device, bad):
    """tests/kernels/test_mpp_linear.py:76-85."""
    x, w, b = _linear_case(64, 64, 64, 7, device)
    x[0] = bad
    got = _np(mpp_linear.linear(_bf(x, device), _bf(w, device), _bf(b, device), transposed=True))
    assert not np.any(np.isfinite(got[0]))
    assert np.all(np.isfinite(got[1:]))


def test_linear_rows_adds_the_residual_after_the_product(device):
    x, w, b = _linear_case(70, 96, 64, 8, device)
    resid = oracle.to_bf16(_rng(8).standard_normal((70, 96)).astype(F32))
    got = _np(mpp_linear.linear_rows(_bf(x, device), _bf(w, device), _bf(b, device), residual=_bf(resid, device)))
    ref = resid + oracle.to_bf16(oracle.linear(x, w, b))
    assert _gemm_close(got, ref)


# ---- projection with the per-head Q/K norm and pair RoPE in its epilogue ---------------------------


def _qknorm_case(m, k, q_heads, k_heads, rest, tokens, table_batch, seed):
    r = _rng(seed)
    n = (q_heads + k_heads) * 128 + rest
    x, w, b = _linear_case(m, n, k, seed, None, scale=2.0)
    nq = (r.standard_normal(128) * 0.1 + 1).astype(F32)
    nk = (r.standard_normal(128) * 0.1 + 1).astype(F32)
    ang = np.repeat(r.uniform(-4, 4, (table_batch, tokens, 64)), 2, axis=-1).astype(F32)
    return x, w, b, nq, nk, np.cos(ang).astype(F32), np.sin(ang).astype(F32)


def _qknorm_reference(proj, q_end, k_end, nq, nk, eps, offset, cos_rows, sin_rows):
    """The oracle's norm + rotation of each query / key head of ``proj`` (the bf16 projection)."""
    out = np.array(proj, dtype=F32)
    rows = proj.shape[0]
    for lo, hi, weight in ((0, q_end, nq), (q_end, k_end, nk)):
        if hi > lo:
            heads = (hi - lo) // 128
            normed = oracle.rms_norm(proj[:, lo:hi].reshape(rows, heads, 128), weight, eps, weight_offset=offset)
            out[:, lo:hi] = oracle.pair_rope(normed, cos_rows[:, None], sin_rows[:, None]).reshape(rows, hi - lo)
    return out


def _pair_bound(ref, scale):
    """``scale`` times the magnitude of each element's rotation pair (rotation mixes the pair)."""
    pairs = np.abs(ref).reshape(*ref.shape[:-1], -1, 2).sum(axis=-1, keepdims=True)
    return scale * np.broadcast_to(pairs, pairs.shape[:-1] + (2,)).reshape(ref.shape)


QKNORM_CASES = [
    # m, k, q heads, k heads, other columns, tokens per table row set, table sets, bias, norm dtype, offset, eps
    (300, 512, 4, 4, 512, 300, 1, False, "bf16", 0.0, 1e-6),          # FLUX stream: ragged M, V after
    (2 * 97, 256, 8, 4, 456, 97, 2, True, "f32", 1.0, 1e-5),          # Krea GQA, batched tables, ragged N
    (512, 384, 4, 4, 512 + 2048, 512, 1, False, "bf16", 0.0, 1e-6),   # FLUX single: Q, K, V, then MLP
    (500, 64, 88, 88, 0, 250, 1, True, "bf16", 0.0, 1e-6),            # every column a head, 256-row tiles
    (9, 128, 1, 1, 128, 9, 1, True, "f32", 1.0, 1e-6),                # one partial tile
    (130, 256, 1, 2, 384, 65, 2, True, "bf16", 0.0, 1e-6),            # a tile with a key head and V columns
]


@pytest.mark.parametrize(("m", "k", "q_heads", "k_heads", "rest", "tokens", "table_batch", "bias", "wdtype",
                          "offset", "eps"), QKNORM_CASES,
                         ids=["flux-stream", "krea-gqa-batched", "flux-single", "all-heads-256", "tiny",
                              "mixed-tile"])
def test_qknorm_rope_projection_matches_oracle(device, m, k, q_heads, k_heads, rest, tokens, table_batch, bias,
                                               wdtype, offset, eps):
    """kx_gemm_qknorm_rope_bf16 against the oracle's linear -> bf16 -> per-head RMSNorm -> pair RoPE
    (FLUX.2 transformer.py:25-29, 68-75; Krea model.py:29-46, 69-92). Q/K columns: relative L2 and
    cosine at the standalone norm + RoPE kernel's bar, and every element within 2^-6 of its
    rotation pair's magnitude (one bf16 ulp of the projection, carried through the norm, plus the
    output's rounding); the other columns at the plain GEMM's bar."""
    x, w, b, nq, nk, cos, sin = _qknorm_case(m, k, q_heads, k_heads, rest, tokens, table_batch, m + k + rest)
    n = w.shape[0]
    q_end, k_end = 128 * q_heads, 128 * (q_heads + k_heads)
    wt = torch.bfloat16 if wdtype == "bf16" else torch.float32
    if wdtype == "bf16":
        nq, nk = oracle.to_bf16(nq), oracle.to_bf16(nk)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.launch_gemm_qknorm_rope(
        _bf(x, device), _bf(w, device), out, bias=_bf(b, device) if bias else None, q_end=q_end, k_end=k_end,
        norm_q=torch.from_numpy(nq).to(device, wt), norm_k=torch.from_numpy(nk).to(device, wt), eps=eps,
        weight_offset=offset, cos=_f32(cos, device), sin=_f32(sin, device), table_ld=128, table_hs=0,
        table_rows=tokens, table_bs=tokens * 128 if table_batch > 1 else 0)
    got = _np(out)
    linear = oracle.linear(x, w, b if bias else None)
    rows = np.arange(m)
    tb = rows // tokens if table_batch > 1 else np.zeros(m, dtype=int)
    cos_rows, sin_rows = cos[tb, rows % tokens], sin[tb, rows % tokens]
    ref = _qknorm_reference(oracle.to_bf16(linear), q_end, k_end, nq, nk, eps, offset, cos_rows, sin_rows)
    g, r = got[:, :k_end], ref[:, :k_end]
    assert np.isfinite(got).all()
    assert rel_l2(g, r) < 4e-3 and cosine(g, r) > 0.99999
    assert np.all(np.abs(g - r) <= _pair_bound(r, 2.0**-6) + 1e-5)
    if k_end < n:
        assert _gemm_close(got[:, k_end:], linear[:, k_end:])


@pytest.mark.parametrize("case", [0, 1, 2], ids=["flux-stream", "krea-gqa-batched", "flux-single"])
def test_qknorm_rope_projection_agrees_with_the_two_pass_path(device, monkeypatch, case):
    """Against the plain 256x256 projection then kx_rmsnorm_rope_bf16 on its bf16 output (the path
    the epilogue replaces; Q and K widths that are multiples of 512, that kernel's one-pass
    contract): the other columns bit-identical (same kernel family, same K order), the Q/K columns
    within one bf16 ulp (the norm's sum of squares runs in another order)."""
    m, k, q_heads, k_heads, rest, tokens, table_batch, bias, wdtype, offset, eps = QKNORM_CASES[case]
    x, w, b, nq, nk, cos, sin = _qknorm_case(m, k, q_heads, k_heads, rest, tokens, table_batch, case)
    n = w.shape[0]
    q_end, k_end = 128 * q_heads, 128 * (q_heads + k_heads)
    wt = torch.bfloat16 if wdtype == "bf16" else torch.float32
    xd, wd, bd = _bf(x, device), _bf(w, device), _bf(b, device) if bias else None
    nqd, nkd = torch.from_numpy(nq).to(device, wt), torch.from_numpy(nk).to(device, wt)
    fused = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    _lib.launch_gemm_qknorm_rope(xd, wd, fused, bias=bd, q_end=q_end, k_end=k_end, norm_q=nqd, norm_k=nkd, eps=eps,
                                 weight_offset=offset, cos=_f32(cos, device), sin=_f32(sin, device), table_ld=128,
                                 table_hs=0, table_rows=tokens, table_bs=tokens * 128 if table_batch > 1 else 0)
    monkeypatch.setenv("KX355_GEMM_LDS_TILE", "0")
    proj = mpp_linear.fused_linear(xd, wd, bd)
    rows = torch.arange(m)
    tb = rows // tokens if table_batch > 1 else torch.zeros(m, dtype=torch.long)
    cos_rows = _f32(cos, device)[tb, rows % tokens].contiguous()
    sin_rows = _f32(sin, device)[tb, rows % tokens].contiguous()
    two = proj.clone()
    for lo, hi, weight in ((0, q_end, nqd), (q_end, k_end, nkd)):
        _lib.launch_rmsnorm_rope(proj[:, lo:hi], two[:, lo:hi], weight, eps, offset, norm_width=128,
                                 rope_kind=_lib.KX_ROPE_PAIR, cos=cos_rows, sin=sin_rows, table_ld=128, table_hs=0,
                                 tokens=m, table_batched=True, head_dim=128)
    assert torch.equal(fused[:, k_end:], two[:, k_end:])
    g, r = _np(fused[:, :k_end]), _np(two[:, :k_end])
    assert np.all(np.abs(g - r) <= np.abs(r) * 2.0**-7 + 1e-6)
    assert np.mean(g != r) < 0.01


def test_qknorm_rope_projection_per_head_tables(device):
    """Tables with a row per head (table_hs): query head h and key head h read row block h."""
    m, k, heads = 70, 128, 2
    x, w, b, nq, nk, _, _ = _qknorm_case(m, k, heads, heads, 256, m, 1, 5)
    ang = np.repeat(_rng(6).uniform(-4, 4, (m, heads, 64)), 2, axis=-1).astype(F32)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    out = torch.empty((m, w.shape[0]), dtype=torch.bfloat16, device=device)
    _lib.launch_gemm_qknorm_rope(_bf(x, device), _bf(w, device), out, bias=_bf(b, device), q_end=256, k_end=512,
                                 norm_q=_f32(nq, device), norm_k=_f32(nk, device), eps=1e-6, weight_offset=0.0,
                                 cos=_f32(cos, device), sin=_f32(sin, device), table_ld=heads * 128, table_hs=128,
                                 table_rows=m, table_bs=0)
    proj = oracle.to_bf16(oracle.linear(x, w, b))
    ref = proj.copy()
    for lo, weight in ((0, nq), (256, nk)):
        normed = oracle.rms_norm(proj[:, lo:lo + 256].reshape(m, heads, 128), weight, 1e-6)
        ref[:, lo:lo + 256] = oracle.pair_rope(normed, cos, sin).reshape(m, 256)
    got = _np(out)
    assert rel_l2(got[:, :512], ref[:, :512]) < 4e-3
    assert np.all(np.abs(got[:, :512] - ref[:, :512]) <= _pair_bound(ref[:, :512], 2.0**-6) + 1e-5)


def test_qknorm_rope_projection_layer_helper_matches_the_launch(device):
    """``qknorm_rope_projection`` on a Linear over two sequences with broadcast and per-sequence
    tables reads the same table rows as the explicit launch."""
    m, tokens = 2 * 64, 64
    x, w, b, nq, nk, cos, sin = _qknorm_case(m, 256, 2, 2, 256, tokens, 2, 11)
    layer = ltx_attention.Linear(_bf(w, device), _bf(b, device))
    for table_batch in (1, 2):
        c, s_ = _f32(cos[:table_batch], device), _f32(sin[:table_batch], device)
        out = torch.empty((m, w.shape[0]), dtype=torch.bfloat16, device=device)
        assert ltx_attention.qknorm_rope_projection(layer, _bf(x, device), out, q_width=256, k_width=256,
                                                    norm_q=_f32(nq, device), norm_k=_f32(nk, device), eps=1e-6,
                                                    weight_offset=0.0, cos=c, sin=s_)
        ref = torch.empty_like(out)
        _lib.launch_gemm_qknorm_rope(_bf(x, device), _bf(w, device), ref, bias=_bf(b, device), q_end=256,
                                     k_end=512, norm_q=_f32(nq, device), norm_k=_f32(nk, device), eps=1e-6,
                                     weight_offset=0.0, cos=c, sin=s_, table_ld=128, table_hs=0, table_rows=tokens,
                                     table_bs=tokens * 128 if table_batch > 1 else 0)
        assert torch.equal(out, ref)
        if table_batch == 1:  # the second sequence reads the first table set
            assert torch.equal(out[tokens:, :512], _qk_rows_with_tables(layer, x[tokens:], c, s_, nq, nk, device))
    # outside the kernel's contract (head width 64): nothing written, the caller runs two passes
    out = torch.zeros((m, w.shape[0]), dtype=torch.bfloat16, device=device)
    assert not ltx_attention.qknorm_rope_projection(layer, _bf(x, device), out, q_width=256, k_width=256,
                                                    norm_q=_f32(nq[:64], device), norm_k=_f32(nk[:64], device),
                                                    eps=1e-6, weight_offset=0.0, cos=_f32(cos[0], device)[:, :64],
                                                    sin=_f32(sin[0], device)[:, :64])
    assert not out.any()


def _qk_rows_with_tables(layer, x, cos, sin, nq, nk, device):
    out = torch.empty((x.shape[0], layer.out_features), dtype=torch.bfloat16, device=device)
    assert ltx_attention.qknorm_rope_projection(layer, _bf(x, device), out, q_width=256, k_width=256,
                                                norm_q=_f32(nq, device), norm_k=_f32(nk, device), eps=1e-6,
                                                weight_offset=0.0, cos=cos[0], sin=sin[0])
    return out[:, :512]


# ---- attention -----------------------------------------------------------------------------------


def _attn_inputs(tq, tk, dim, heads, seed):
    r = _rng(seed)
    return tuple(oracle.to_bf16(r.standard_normal((t, heads * dim)).astype(F32)) for t in (tq, tk, tk))


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize(("tq", "tk"), [(7, 7), (16, 16), (33, 33), (517, 517), (300, 1024), (1, 300), (517, 33), (40, 5)])
def test_attention_matches_oracle_across_tile_edges(device, dim, tq, tk):
    """tests/models/ltx2/test_dense_attention.py:49-64: relative L2 < 6e-3 for bf16."""
    q, k, v = _attn_inputs(tq, tk, dim, 2, tq + tk + dim)
    got = dense_attention.dense_attention(_bf(q, device), _bf(k, device), _bf(v, device), heads=2)
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == q.shape
    assert rel_l2(_np(got), oracle.attention(q, k, v, heads=2)) < 6e-3


def test_keys_past_a_partial_tile_take_no_weight(device):
    """tests/models/ltx2/test_dense_attention.py:67-76: a sentinel key one past the end."""
    q, k, v = _attn_inputs(9, 17, 128, 2, 3)
    kp = np.concatenate([k, np.full((1, k.shape[1]), 8.0, F32)])
    vp = np.concatenate([v, np.full((1, v.shape[1]), 1000.0, F32)])
    kd, vd = _bf(kp, device), _bf(vp, device)
    got = dense_attention.dense_attention(_bf(q, device), kd[:17], vd[:17], heads=2)
    assert rel_l2(_np(got), oracle.attention(q, k, v, heads=2)) < 6e-3


def test_attention_large_values_stay_finite(device):
    """bf16 values beyond fp16's range (test_dense_attention.py:79-83) need no saturation here."""
    q, k, v = _attn_inputs(64, 64, 128, 2, 4)
    v[0] = 1e5
    got = _np(dense_attention.dense_attention(_bf(q, device), _bf(k, device), _bf(v, device), heads=2))
    assert np.all(np.isfinite(got))
    assert rel_l2(got, oracle.attention(q, k, oracle.to_bf16(v), heads=2)) < 6e-3


def test_attention_gate_batch_and_strided_inputs(device):
    r = _rng(12)
    b, t, tk, heads, dim = 2, 70, 45, 4, 128
    width = heads * dim
    qkv = oracle.to_bf16(r.standard_normal((b, t, 3 * width)).astype(F32))
    kv = oracle.to_bf16(r.standard_normal((b, tk, 2 * width)).astype(F32))
    gate = oracle.to_bf16(r.uniform(0, 2, (b, t, heads)).astype(F32))
    qkv_d, kv_d = _bf(qkv, device), _bf(kv, device)
    got = dense_attention.batched_attention(qkv_d[..., :width], kv_d[..., :width], kv_d[..., width:], heads=heads,
                                            gate=_bf(gate, device))
    for i in range(b):
        ref = oracle.attention(qkv[i, :, :width], kv[i, :, :width], kv[i, :, width:], heads=heads)
        ref = (ref.reshape(t, heads, dim) * gate[i][:, :, None]).reshape(t, width)
        assert rel_l2(_np(got[i]), ref) < 6e-3


@pytest.mark.parametrize("tk", [256, 250, 64, 1])
def test_attention_resident_keys_over_several_query_tiles(device, tk):
    """At most 256 keys (a text context) stay in LDS while a workgroup runs several query tiles
    of its head: 4000 queries x 32 heads is 11 tiles of 384 per head, two per workgroup (the last
    one alone), with a per-(query, head) gate, against the FP32 oracle."""
    tq, heads, dim = 4000, 32, 128
    q, k, v = _attn_inputs(tq, tk, dim, heads, 40 + tk)
    gate = oracle.to_bf16(_rng(41).uniform(0, 2, (tq, heads)).astype(F32))
    got = dense_attention.batched_attention(_bf(q, device)[None], _bf(k, device)[None], _bf(v, device)[None],
                                            heads=heads, gate=_bf(gate, device)[None])
    ref = (oracle.attention(q, k, v, heads=heads).reshape(tq, heads, dim) * gate[:, :, None]).reshape(tq, -1)
    assert rel_l2(_np(got[0]), ref) < 6e-3 and cosine(_np(got[0]), ref) > 0.9999


def test_attention_resident_keys_grouped_query_batched(device):
    """The resident-key form with grouped-query heads (32 query heads over 8 key/value heads)
    and a batch of two: each workgroup reads its own batch's and group's keys."""
    b, tq, tk, heads, kv_heads, dim = 2, 900, 100, 32, 8, 128
    r = _rng(42)
    q = oracle.to_bf16(r.standard_normal((b, tq, heads * dim)).astype(F32))
    k, v = (oracle.to_bf16(r.standard_normal((b, tk, kv_heads * dim)).astype(F32)) for _ in range(2))
    got = dense_attention.batched_attention(_bf(q, device), _bf(k, device), _bf(v, device), heads=heads,
                                            kv_heads=kv_heads)
    group = heads // kv_heads
    for i in range(b):
        kx, vx = (np.repeat(t[i].reshape(tk, kv_heads, dim), group, axis=1).reshape(tk, heads * dim) for t in (k, v))
        ref = oracle.attention(q[i], kx, vx, heads=heads)
        assert rel_l2(_np(got[i]), ref) < 6e-3


def test_attention_self_attention_at_ltx_width(device):
    q, k, v = _attn_inputs(1100, 1100, 128, 32, 13)
    got = dense_attention.dense_attention(_bf(q, device), _bf(k, device), _bf(v, device), heads=32)
    ref = oracle.attention(q, k, v, heads=32)
    assert rel_l2(_np(got), ref) < 6e-3 and cosine(_np(got), ref) > 0.9999


# ---- affine int4 / int8 ---------------------------------------------------------------------------


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_is_bit_exact(device, bits):
    r = _rng(20 + bits)
    n, k = 96, 512
    codes = r.integers(0, 1 << bits, (n, k))
    words = oracle.pack_affine(codes, bits)
    scales = oracle.to_bf16((np.abs(r.standard_normal((n, k // 64))) * 0.003 + 1e-5).astype(F32))
    biases = oracle.to_bf16((r.standard_normal((n, k // 64)) * 0.05).astype(F32))
    wq = torch.from_numpy(words.view(np.int32)).to(device)
    got = quantized.dequantize(wq, _bf(scales, device), _bf(biases, device), group_size=64, bits=bits)
    ref = oracle.dequantize_affine(words, scales, biases, group_size=64, bits=bits)
    assert np.array_equal(_np(got), ref)


@pytest.mark.parametrize("bits", [4, 8])
def test_gpu_quantizer_is_bit_identical_to_the_oracle(device, bits):
    w = oracle.to_bf16((_rng(30).standard_normal((128, 1024)) * 0.02).astype(F32))
    words, scales, biases = quantized.quantize(_bf(w, device), 64, bits)
    o_words, o_scales, o_biases = oracle.quantize_affine(w, 64, bits)
    assert np.array_equal(words.cpu().numpy().view(np.uint32), o_words)
    assert np.array_equal(_np(scales), o_scales) and np.array_equal(_np(biases), o_biases)


@pytest.mark.parametrize("tile", ["auto", "0", "2", "3"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize(("m", "n", "k"), [(300, 520, 1024), (9, 64, 256)])
def test_quantized_linear_matches_oracle(device, monkeypatch, tile, bits, m, n, k):
    if tile != "auto":
        monkeypatch.setenv("KX355_GEMM_TILE", tile)
    r = _rng(m + n + bits)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * 0.02).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.02).astype(F32))
    words, scales, biases = oracle.quantize_affine(w, 64, bits)
    layer = quantized.QuantizedLinear(torch.from_numpy(words.view(np.int32)).to(device), _bf(scales, device),
                                      _bf(biases, device), _bf(b, device), group_size=64, bits=bits)
    ref = oracle.quantized_linear(x, words, scales, biases, b, group_size=64, bits=bits)
    # the in-mainloop kernels (KX355_GEMM_TILE selects the register-staged kernel's tile)
    got = _np(quantized.quantized_matmul(_bf(x, device), layer.weight, layer.scales, layer.biases, group_size=64,
                                         bits=bits, bias=layer.bias))
    assert _gemm_close(got, ref)
    # the layer: the exactly dequantized weight through the dense kernel
    dense = _np(layer(_bf(x, device)))
    assert _gemm_close(dense, ref)
    assert max_abs(got, dense) <= 2.0**-7 * np.abs(dense).max()


def test_quantized_layers_share_one_dequantization_buffer(device):
    """Consecutive quantized layers on one stream dequantize into one buffer (grown to the largest
    weight, then reused), and each call equals the dense kernel on that layer's own dequantized
    weight, also after a larger layer overwrote the buffer."""
    r = _rng(77)
    layers, xs = [], []
    for n, k in ((256, 512), (640, 1024), (128, 256)):
        w = oracle.to_bf16((r.standard_normal((n, k)) * 0.02).astype(F32))
        words, scales, biases = oracle.quantize_affine(w, 64, 4)
        layers.append(quantized.QuantizedLinear(torch.from_numpy(words.view(np.int32)).to(device), _bf(scales, device),
                                                _bf(biases, device), group_size=64, bits=4))
        xs.append(_bf(oracle.to_bf16(r.standard_normal((96, k)).astype(F32)), device))
    quantized._WORKSPACE.clear()
    outs = [layer(x) for layer, x in zip(layers, xs)]
    torch.cuda.synchronize()
    assert len(quantized._WORKSPACE) == 1
    buf = next(iter(quantized._WORKSPACE.values()))
    assert buf.numel() == 640 * 1024  # grown once, to the largest weight
    ptr = buf.data_ptr()
    again = layers[0](xs[0])
    assert next(iter(quantized._WORKSPACE.values())).data_ptr() == ptr
    for layer, x, got in zip(layers, xs, outs):
        assert torch.equal(got, mpp_linear.fused_linear(x, layer.dequantized(), None))
    assert torch.equal(again, outs[0])


@pytest.mark.parametrize("tile", ["0", "1"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize(("m", "n", "k"), [(512, 512, 512), (300, 520, 1024), (200, 256, 128), (1000, 132, 384)])
@pytest.mark.parametrize("epilogue", ["bias", "gated_f32"])
@pytest.mark.parametrize("layout", ["tiled", "reference"])
def test_quantized_linear_dequantizes_in_lds(device, monkeypatch, tile, bits, m, n, k, epilogue, layout):
    """The direct-to-LDS quantized kernel (packed words and scale / bias words DMA'd per stage,
    each wave dequantizing its own weight fragments in registers) at both of its tiles (256x256,
    192x256), on full and ragged tiles, on the tiled and the reference layout: equal to the oracle
    up to fp32 summation order (the dequantization is bit-exact)."""
    monkeypatch.setenv("KX355_GEMM_LDS_TILE", tile)
    r = _rng(m + n + k + bits)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * 0.02).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.02).astype(F32))
    words, scales, biases = oracle.quantize_affine(w, 64, bits)
    wq, sd, bd, bias = torch.from_numpy(words.view(np.int32)).to(device), _bf(scales, device), _bf(biases, device), _bf(b, device)
    tiled = quantized.tile_weights(wq, sd, bd, bits=bits) if layout == "tiled" else None

    def call(**kw):
        if tiled is None:  # the C ABI on the reference layout (packed rows read in place)
            return quantized.quantized_matmul(_bf(x, device), wq, sd, bd, group_size=64, bits=bits, bias=bias, **kw)
        out = torch.empty((m, n), device=device, dtype=kw.get("out_dtype") or torch.bfloat16)
        flags = _lib.EPI_BIAS | (_lib.EPI_GATED_RESIDUAL if "residual" in kw else 0)  # dtype flags: the launcher
        _lib.launch_qgemm_tiled(_bf(x, device), tiled[0], tiled[1], out, n=n, k=k, bits=bits, bias=bias, flags=flags,
                                resid=kw.get("residual"), gate=kw.get("gate"))
        return out

    ref = oracle.quantized_linear(x, words, scales, biases, b, group_size=64, bits=bits)
    if epilogue == "bias":
        got = _np(call())
        assert _gemm_close(got, ref)
    else:
        resid = r.standard_normal((m, n)).astype(F32)
        gate = r.standard_normal(n).astype(F32)
        got = _np(call(residual=_f32(resid, device), gate=_f32(gate, device), out_dtype=torch.float32))
        full = resid + gate * ref
        assert np.all(np.abs(got - full) <= 1e-5 * np.abs(full) + 2e-5 * np.abs(full).max())


@pytest.mark.parametrize(("m", "n", "k"), [(1000, 32, 1024), (37, 64, 256), (300, 40, 512), (9216, 32, 4096),
                                           (20000, 64, 768), (70000, 32, 256), (500, 32, 640)])
@pytest.mark.parametrize("bits", [None, 4, 8])
@pytest.mark.parametrize("epilogue", ["sigmoid2", "gated_f32"])
def test_skinny_linear_matches_oracle(device, m, n, k, bits, epilogue):
    """N <= 64 (the gate-logit projections) takes the skinny kernels, dense and quantized: the
    LDS-staged one for K % 256 == 0 at every rows-per-workgroup form (16 rows; 36 rows = five 8-row
    DMA groups at the block's 9216 rows; 40 and 55 rows in two and five rounds), the register one
    for K % 256 != 0 (640)."""
    r = _rng(m + n + k)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * k ** -0.5).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.5).astype(F32))
    if bits is None:
        weight = w
        call = lambda **kw: mpp_linear.fused_linear(_bf(x, device), _bf(w, device), _bf(b, device), **kw)  # noqa: E731
    else:
        words, scales, biases = oracle.quantize_affine(w, 64, bits)
        weight = oracle.dequantize_affine(words, scales, biases, group_size=64, bits=bits)
        layer = quantized.QuantizedLinear(torch.from_numpy(words.view(np.int32)).to(device), _bf(scales, device),
                                          _bf(biases, device), _bf(b, device), group_size=64, bits=bits)
        call = lambda **kw: layer(_bf(x, device), **kw)  # noqa: E731
    lin = oracle.linear(x, weight, b)
    if epilogue == "sigmoid2":
        got = _np(call(activation="sigmoid2"))
        ref = 2.0 / (1.0 + np.exp(-lin.astype(np.float64)))
        assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-5)
    else:
        resid = r.standard_normal((m, n)).astype(F32)
        gate = r.standard_normal(n).astype(F32)
        got = _np(call(residual=_f32(resid, device), gate=_f32(gate, device), out_dtype=torch.float32))
        ref = resid + gate * lin
        assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 2e-5 * np.abs(ref).max())


# ---- mxfp8 (OCP MX: E4M3 codes, one E8M0 scale per 32) -------------------------------------------


def _mx_codes(r, rows, cols):
    """Random E4M3 codes holding every one of the 256 codes except the two NaNs."""
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    return finite[r.integers(0, finite.size, (rows, cols))]


def test_mxfp8_dequant_is_exact_for_every_code_and_scale(device):
    """Reference layout: every finite code under every scale byte whose products stay in the
    normal fp32 range (10 .. 240), equal to the oracle's exact decode; NaN codes decode to NaN."""
    scales_all = np.arange(10, 241, dtype=np.uint8)
    n, k = scales_all.size, 256
    codes = np.tile(np.arange(256, dtype=np.uint8), (n, 1))  # row i: all 256 codes, scale byte 10 + i
    words = oracle.pack_bytes(codes)
    scales = np.repeat(scales_all[:, None], k // 32, 1)
    got = quantized.dequantize_mxfp8(torch.from_numpy(words.view(np.int32)).to(device), torch.from_numpy(scales).to(device))
    ref = oracle.dequantize_mxfp8(words, scales)
    g = _np(got)
    assert np.array_equal(np.isnan(g), np.isnan(ref))
    assert np.array_equal(g[~np.isnan(g)], ref[~np.isnan(ref)])


@pytest.mark.parametrize(("out_f", "in_f"), [(352, 200), (64, 8), (96, 512)])
def test_mxfp8_pretransposed_dequant_is_exact(device, out_f, in_f):
    """The pretransposed packing of weight.T, (in, out / 4) words grouped along out: dequantized to
    the (out, in) weight, equal to the oracle's (ragged 64 x 64 tiles on both axes)."""
    r = _rng(out_f + in_f)
    codes = _mx_codes(r, in_f, out_f)
    words = oracle.pack_bytes(codes)
    scales = r.integers(100, 140, (in_f, out_f // 32)).astype(np.uint8)
    got = quantized.dequantize_mxfp8(torch.from_numpy(words.view(np.int32)).to(device),
                                     torch.from_numpy(scales).to(device), transposed=True)
    assert got.shape == (out_f, in_f)
    assert np.array_equal(_np(got), oracle.dequantize_mxfp8(words, scales).T)


@pytest.mark.parametrize("shape", [(128, 1024), (3, 96), (1000, 4096)])
def test_gpu_mxfp8_quantizer_is_bit_identical_to_the_oracle(device, shape):
    r = _rng(shape[0])
    w = (r.standard_normal(shape) * np.exp2(r.integers(-10, 10, (shape[0], 1)))).astype(F32)
    w[0, :32] = 0.0  # a zero group
    w[-1, 5] = 3e30  # the rest of its group underflows
    w[-1, 40] = -1e-39  # a bf16 subnormal
    w = oracle.to_bf16(w)
    words, scales = quantized.quantize_mxfp8(_bf(w, device))
    o_words, o_scales = oracle.quantize_mxfp8(w)
    assert np.array_equal(words.cpu().numpy().view(np.uint32), o_words)
    assert np.array_equal(scales.cpu().numpy(), o_scales)
    h_words, h_scales = quantized.quantize_mxfp8(torch.from_numpy(w).to(torch.bfloat16))  # host packing
    assert torch.equal(words.cpu(), h_words) and torch.equal(scales.cpu(), h_scales)


@pytest.mark.parametrize("tile", ["0", "1"])
@pytest.mark.parametrize(("m", "n", "k"), [(512, 512, 512), (1000, 132, 384), (600, 256, 4096), (300, 520, 1024),
                                           (9, 64, 256), (37, 48, 96), (200, 256, 96)])
@pytest.mark.parametrize("epilogue", ["bias", "gated_f32"])
def test_mxfp8_linear_matches_oracle(device, monkeypatch, tile, m, n, k, epilogue):
    """``kx_qgemm_mxfp8_bf16`` on every kernel it dispatches to: the direct-to-LDS kernel at both of
    its tiles (m >= 512, k % 128 == 0), the register-staged kernel (fewer rows, and k % 64 == 32:
    a half-empty last stage), the skinny kernel (n <= 64); against the oracle's mxfp8 linear (the
    dequantization is exact, so only the fp32 summation order differs) and, for the bias
    epilogue, against the dense kernel on the exactly dequantized weight."""
    monkeypatch.setenv("KX355_GEMM_LDS_TILE", tile)
    r = _rng(m + n + k)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * k ** -0.5).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.02).astype(F32))
    words, scales = oracle.quantize_mxfp8(w)
    layer = quantized.QuantizedLinear(torch.from_numpy(words.view(np.int32)).to(device), torch.from_numpy(scales).to(device),
                                      None, _bf(b, device), mode="mxfp8")
    assert (layer.group_size, layer.bits) == (32, 8)
    ref = oracle.mxfp8_linear(x, words, scales, b)

    def in_loop(**kw):  # the in-mainloop kernels, not the layer's dequantize-then-dense path
        return quantized.quantized_matmul(_bf(x, device), layer.weight, layer.scales, None, group_size=32, bits=8,
                                          mode="mxfp8", bias=layer.bias, **kw)

    if epilogue == "bias":
        got = _np(in_loop())
        assert _gemm_close(got, ref)
        dense = _np(layer(_bf(x, device)))
        assert _gemm_close(dense, ref)
        assert max_abs(got, dense) <= 2.0**-7 * np.abs(dense).max()
    else:
        resid = r.standard_normal((m, n)).astype(F32)
        gate = r.standard_normal(n).astype(F32)
        full = resid + gate * ref
        for fn in (in_loop, layer):
            kw = dict(residual=_f32(resid, device), gate=_f32(gate, device), out_dtype=torch.float32)
            got = _np(fn(**kw) if fn is in_loop else fn(_bf(x, device), **kw))
            assert np.all(np.abs(got - full) <= 1e-5 * np.abs(full) + 2e-5 * np.abs(full).max())


def test_mxfp8_identity_linear_returns_its_input(device):
    """``tests/models/ltx2/weights/test_family.py:262-283``: the mxfp8 identity (eye(32)) bound as
    a quantized linear returns its input; and as the pretransposed layer."""
    eye = torch.eye(32, dtype=torch.bfloat16)
    x = torch.ones((1, 32), dtype=torch.bfloat16, device=device)
    layer = quantized.QuantizedLinear.from_linear(eye.to(device), mode="mxfp8")
    assert torch.equal(layer(x), x)
    in_loop = quantized.quantized_matmul(x, layer.weight, layer.scales, None, group_size=32, bits=8, mode="mxfp8")
    assert torch.equal(in_loop, x)
    pre = quantized.PretransposedQuantizedLinear.from_linear(eye.to(device))
    assert torch.equal(pre(x), x)
    y = torch.randn((5, 32), device=device).to(torch.bfloat16)
    assert torch.equal(layer(y), y) and torch.equal(pre(y), y)


def test_pretransposed_linear_is_the_dense_product_of_its_dequantized_weight(device):
    r = _rng(77)
    w = oracle.to_bf16((r.standard_normal((256, 512)) * 0.05).astype(F32))
    x = oracle.to_bf16(r.standard_normal((300, 512)).astype(F32))
    b = oracle.to_bf16((r.standard_normal(256) * 0.1).astype(F32))
    layer = quantized.PretransposedQuantizedLinear.from_linear(_bf(w, device), _bf(b, device))
    words, scales = oracle.quantize_mxfp8(np.ascontiguousarray(w.T))
    assert np.array_equal(layer.weight.cpu().numpy().view(np.uint32), words)
    ref = oracle.mxfp8_linear(x, words, scales, b, transposed=False)
    assert _gemm_close(_np(layer(_bf(x, device))), ref)
    # the functional form (transpose=False) gives the same product
    got = quantized.quantized_matmul(_bf(x, device), layer.weight, layer.scales, None, transpose=False, group_size=32,
                                     bits=8, mode="mxfp8", bias=_bf(b, device))
    assert torch.equal(got, layer(_bf(x, device)))


def test_env_tile_override_is_restored():
    assert os.environ.get("KX355_GEMM_TILE") in (None, "")
    assert os.environ.get("KX355_GEMM_LDS_TILE") in (None, "")


@pytest.mark.parametrize("table_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ts_dtype", [torch.bfloat16, torch.float32, None])
def test_table_add_is_bit_exact(device, table_dtype, ts_dtype):
    """``kx_table_add_f32``: fp32(table) + fp32(timestep modulation), the block's ``_ada_values``
    (``transformer.py:179-186``), for whole tables and row slices of a strided timestep tensor."""
    g = torch.Generator().manual_seed(11)
    table = torch.randn((9, 640), generator=g).to(table_dtype).to(device)
    if ts_dtype is None:
        got = _lib.table_add(table, None)
        assert got.shape == (1, 1, 9, 640)
        assert torch.equal(got[0, 0], table.float())
        return
    ts = torch.randn((2, 3, 9, 640), generator=g).to(ts_dtype).to(device)
    got = _lib.table_add(table, ts)
    assert torch.equal(got, table[None, None].float() + ts.float())
    part = _lib.table_add(table[3:6], ts[:, :, 3:6, :])
    assert torch.equal(part, table[3:6][None, None].float() + ts[:, :, 3:6, :].float())


@pytest.mark.parametrize("round_to", [torch.bfloat16, torch.float16])
def test_table_add_rounds_and_broadcasts(device, round_to):
    """The output head's ``(shift, scale)`` (``model.py:577-593``): the table plus the embedded
    timestep broadcast over the table's rows by a zero stride, each sum rounded to the hidden
    state's type, bit for bit as torch rounds the FP32 sum."""
    g = torch.Generator().manual_seed(12)
    table = torch.randn((2, 640), generator=g).to(torch.bfloat16).to(device)
    emb = (torch.randn((2, 3, 640), generator=g) * 3.0).to(device)
    got = _lib.table_add(table, emb[:, :, None, :].expand(-1, -1, 2, -1), round_to=round_to)
    want = (table[None, None].float() + emb[:, :, None, :]).to(round_to).float()
    assert got.shape == (2, 3, 2, 640)
    assert torch.equal(got, want)
    assert not torch.equal(got, table[None, None].float() + emb[:, :, None, :])
