"""Parity on the GPU of the steps either side of the block: the timestep / AdaLN producers, the
RoPE table kernel, the output head, the transformer forward (blocks + head), the X0 conversion,
the conditioning composite, the Euler updates, the finite check and one whole denoising step.

Bars: the element-wise passes (X0, composite, Euler, finite check) are one FP32 evaluation with
the reference's roundings, so they are compared bit for bit with the oracle. The transcendental
tables (timestep features, RoPE) are compared within a few FP32 ulps of the angle (the error of
any FP32 sin / cos / exp implementation: |d| <= 1e-6 + 5e-7 |angle|). Outputs of GEMM chains
use the block bar: cosine >= 0.9995 and |got - ref| <= 2e-2 + ulp_bf16(ref) / 2 elementwise
(``assert_block_bar``; the reference's own bf16 graph is printed beside it).
"""

import math

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.ltx2 import denoise as denoise_mod
from kinomlx_amd.ltx2.denoise import LTX2DenoiseError, all_finite, denoise_step
from kinomlx_amd.ltx2.rope import precompute_freqs_cis
from kinomlx_amd.ltx2.state import LatentState, post_process_latent
from kinomlx_amd.ltx2.timestep import get_timestep_embedding
from kinomlx_amd.ltx2.wrappers import Modality, X0Model, _to_denoised
from kinomlx_amd.samplers.steps import euler_step, euler_velocity_step
from oracle.ops import F32, to_bf16
from tests.conftest import assert_block_bar

pytestmark = pytest.mark.gpu

SPEC = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
CHANNELS = 32


def _np(t):
    return t.float().cpu().numpy()


def _angle_tol(angles):
    return 1e-6 + 5e-7 * np.abs(angles)


# ---- tables ---------------------------------------------------------------------------------


@pytest.mark.parametrize("dim", [256, 255])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_timestep_embedding_matches_oracle(device, dim, dtype):
    t = torch.tensor([0.0, 0.05, 0.5, 0.9, 1.0, 0.0371], dtype=torch.float32)
    got = _np(get_timestep_embedding(t.to(device), dim, out_dtype=dtype, time_scale=1000.0))
    ref = oracle.timestep_embedding(t.numpy(), dim, time_scale=1000.0)
    half = dim // 2
    scaled = (t.numpy() * F32(1000.0)).astype(F32)
    angles = scaled[:, None] * np.exp(-math.log(10000) * np.arange(half) / half)[None]
    tol = _angle_tol(np.concatenate([angles, angles], axis=-1))
    if dim % 2:
        tol = np.pad(tol, [(0, 0), (0, 1)], constant_values=1e-6)
        assert np.all(got[:, -1] == 0.0)
    if dtype == torch.bfloat16:
        # one bf16 rounding of values within tol of each other: compare before rounding
        assert np.all(np.abs(got - ref) <= tol + 2.0 ** -8 * np.abs(ref))
    else:
        assert np.all(np.abs(got - ref) <= tol)


def test_rope_tables_match_oracle(device):
    pos = workloads.ltx_positions((3, 4, 5))
    cos, sin = precompute_freqs_cis(pos.to(device), dim=1024, max_pos=(20, 2048, 2048), use_middle_indices_grid=True,
                                    num_attention_heads=8)
    o_cos, o_sin = oracle.precompute_freqs_cis(pos.numpy(), dim=1024, max_pos=(20, 2048, 2048),
                                               use_middle_indices_grid=True, num_attention_heads=8)
    assert cos.shape == (1, 8, 60, 64) and cos.transpose(1, 2).is_contiguous()
    # the angles are the same FP32 values on both sides (same op order, one rounding each);
    # only the sin / cos evaluations differ, by an ulp or two
    assert np.abs(_np(cos) - o_cos).max() <= 1e-6 and np.abs(_np(sin) - o_sin).max() <= 1e-6
    # padding columns (512 - 3 * 170 = 2) hold cos 1, sin 0 exactly
    flat_cos = _np(cos.transpose(1, 2).reshape(1, 60, 512))
    assert np.all(flat_cos[..., :2] == 1.0)


def test_rope_tables_first_bound_and_ragged(device):
    pos = workloads.ltx_positions((2, 3, 7))[..., 0].contiguous()  # (B, axes, T)
    cos, sin = precompute_freqs_cis(pos.to(device), dim=768, max_pos=(20, 2048, 2048), num_attention_heads=6)
    o_cos, o_sin = oracle.precompute_freqs_cis(pos.numpy(), dim=768, max_pos=(20, 2048, 2048), num_attention_heads=6)
    assert cos.shape == (1, 6, 42, 64)
    assert np.abs(_np(cos) - o_cos).max() <= 1e-6 and np.abs(_np(sin) - o_sin).max() <= 1e-6


# ---- model pieces -----------------------------------------------------------------------------


def _model_case(num_blocks=2, seed=0):
    p = workloads.ltx_model_params(SPEC, num_blocks, in_channels=CHANNELS, out_channels=CHANNELS, seed=seed)
    op = {}
    for name, value in p.items():
        if name == "blocks":
            op["blocks"] = [{k: v.float().numpy() for k, v in b.items()} for b in value]
        else:
            op[name] = value.float().numpy()
    inputs = workloads.ltx_model_inputs(SPEC, in_channels=CHANNELS, seed=seed)
    return p, op, inputs


def _check(got, ref, graph):
    assert_block_bar(got, ref, "", context=graph)


def test_adaln_single_matches_oracle(device):
    p, op, _ = _model_case(num_blocks=1)
    model = workloads.build_ltx_model(SPEC, p, device, in_channels=CHANNELS, out_channels=CHANNELS)
    t = torch.tensor([0.25, 0.9], dtype=torch.float32)
    modulation, embedded = model.adaln_single(t.to(device), torch.bfloat16, time_scale=1000.0)
    assert modulation.shape == (2, 9 * SPEC.dim) and embedded.shape == (2, SPEC.dim)
    ref_m, ref_e = oracle.adaln_single(op, "adaln_single", t.numpy(), time_scale=1000.0)
    g_m, g_e = oracle.adaln_single(op, "adaln_single", t.numpy(), time_scale=1000.0, bf16_graph=True)
    _check(_np(embedded), ref_e, g_e)
    _check(_np(modulation), ref_m, g_m)


def test_output_head_matches_oracle(device):
    p, op, _ = _model_case(num_blocks=1)
    model = workloads.build_ltx_model(SPEC, p, device, in_channels=CHANNELS, out_channels=CHANNELS)
    x = workloads.bf16(workloads.normal(5, "head.x", (1, SPEC.tokens, SPEC.dim)))
    emb = workloads.bf16(workloads.normal(5, "head.emb", (1, 1, SPEC.dim), 0.5))
    got = _np(model._output(x.to(device), emb.to(device), model.scale_shift_table, model.proj_out))
    xn, en = x.float().numpy(), emb.float().numpy()
    _check(got, oracle.output_head(op, xn, en), oracle.output_head(op, xn, en, bf16_graph=True))


def _oracle_forward(op, inputs, sigma, num_blocks, bf16_graph=False):
    pe = oracle.precompute_freqs_cis(inputs["positions"].numpy(), dim=SPEC.dim, use_middle_indices_grid=True,
                                     num_attention_heads=SPEC.heads)
    return oracle.ltx_forward(op, inputs["latent"][0].float().numpy(), inputs["context"][0].float().numpy(),
                              np.array([sigma], F32), np.array([sigma], F32), pe, heads=SPEC.heads,
                              num_blocks=num_blocks, bf16_graph=bf16_graph)


def _modality(inputs, sigma, device):
    return Modality(latent=inputs["latent"].to(device), context=inputs["context"].to(device),
                    timesteps=torch.full((1,), sigma, device=device), sigma=torch.full((1,), sigma, device=device),
                    positions=inputs["positions"].to(device))


def test_transformer_forward_matches_oracle(device):
    p, op, inputs = _model_case(num_blocks=2)
    model = workloads.build_ltx_model(SPEC, p, device, in_channels=CHANNELS, out_channels=CHANNELS)
    velocity, audio = model(_modality(inputs, 0.7, device))
    assert audio is None and velocity.shape == (1, SPEC.tokens, CHANNELS) and velocity.dtype == torch.bfloat16
    _check(_np(velocity[0]), _oracle_forward(op, inputs, 0.7, 2), _oracle_forward(op, inputs, 0.7, 2, True))


def test_denoise_step_matches_oracle(device):
    p, op, inputs = _model_case(num_blocks=2)
    model = X0Model(workloads.build_ltx_model(SPEC, p, device, in_channels=CHANNELS, out_channels=CHANNELS))
    latent = inputs["latent"].to(device)
    state = LatentState(latent=latent, denoise_mask=torch.ones((1, SPEC.tokens, 1), device=device),
                        positions=inputs["positions"].to(device), clean_latent=latent)
    sigma, sigma_next = 0.7, 0.45
    new_state, _ = denoise_step(state, None, sigma=sigma, sigma_next=sigma_next, transformer=model,
                                video_context=inputs["context"].to(device))
    lat = inputs["latent"][0].float().numpy()

    def step(bf16_graph):
        velocity = to_bf16(_oracle_forward(op, inputs, sigma, 2, bf16_graph))
        denoised = to_bf16(oracle.to_denoised(lat[None], velocity[None], np.array([sigma], F32)))
        return to_bf16(oracle.euler_step(lat[None], denoised, sigma, sigma_next))[0]

    _check(_np(new_state.latent[0]), step(False), step(True))


# ---- element-wise passes: bit-exact --------------------------------------------------------------


def _rand(seed, shape, dtype, scale=1.0):
    return (workloads.normal(seed, "elem", shape) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("per_token", [False, True])
def test_to_denoised_is_bit_exact(device, dtype, per_token):
    latent, velocity = _rand(1, (2, 37, 24), dtype), _rand(2, (2, 37, 24), dtype)
    ts = torch.rand((2, 37) if per_token else (2,), generator=torch.Generator().manual_seed(3))
    mod = Modality(latent=latent.to(device), context=torch.empty(0), timesteps=ts.to(device),
                   sigma=torch.ones(2), positions=torch.empty(0))
    got = _to_denoised(mod, velocity.to(device))
    assert got.dtype == dtype
    ref = oracle.to_denoised(latent.float().numpy(), velocity.float().numpy(), ts.numpy())
    ref = to_bf16(ref) if dtype == torch.bfloat16 else ref
    assert np.array_equal(_np(got), ref)


def test_to_denoised_known_answer(device):
    mod = Modality(latent=torch.full((1, 2, 128), -1.640625, dtype=torch.bfloat16, device=device),
                   context=torch.empty(0), timesteps=torch.full((1, 2), 0.090820007, device=device),
                   sigma=torch.ones(1), positions=torch.empty(0))
    got = _to_denoised(mod, torch.full((1, 2, 128), -2.453125, dtype=torch.bfloat16, device=device))
    assert torch.all(got == -1.4140625).item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_euler_velocity_step_is_bit_exact(device, dtype):
    s, v = _rand(4, (3, 1000), dtype), _rand(5, (3, 1000), dtype)
    got = euler_velocity_step(s.to(device), v.to(device), 0.9, 0.8123)
    ref = oracle.euler_velocity_step(s.float().numpy(), v.float().numpy(), 0.9, 0.8123,
                                     bf16=dtype == torch.bfloat16)
    assert got.dtype == dtype and np.array_equal(_np(got), ref)
    # the reference's known answer: narrowing before the add
    one = torch.tensor([0.01], dtype=torch.bfloat16, device=device)
    got = euler_velocity_step(one, one, 1.0, 0.1234567)
    assert _np(got)[0] == oracle.euler_velocity_step(_np(one), _np(one), 1.0, 0.1234567, bf16=True)[0]
    with pytest.raises(ValueError, match="finite"):
        euler_velocity_step(one, one, 1.0, float("inf"))


@pytest.mark.parametrize("sdtype,ddtype", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                           (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
def test_euler_step_is_bit_exact(device, sdtype, ddtype):
    s, d = _rand(6, (2, 333, 7), sdtype), _rand(7, (2, 333, 7), ddtype)
    got = euler_step(s.to(device), d.to(device), 0.75, 0.3)
    ref = oracle.euler_step(s.float().numpy(), d.float().numpy(), 0.75, 0.3)
    ref = to_bf16(ref) if sdtype == torch.bfloat16 else ref
    assert got.dtype == sdtype and np.array_equal(_np(got), ref)
    # sigma_next = 0 lands on the prediction (rounded to the sample dtype)
    assert torch.equal(euler_step(s.to(device), d.to(device), 0.75, 0.0).cpu(), d.to(sdtype))
    with pytest.raises(ValueError, match="current sigma must be positive"):
        euler_step(s.to(device), d.to(device), 0.0, -1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mask_value", [0.0, 0.05, 0.5, 0.95, 1.0])
def test_composite_is_bit_exact(device, dtype, mask_value):
    denoised = torch.full((1, 2, 3), -8.0, dtype=dtype, device=device)
    clean = torch.full((1, 2, 3), 4.6875, dtype=dtype, device=device)
    state = LatentState(latent=denoised, denoise_mask=torch.full((1, 2, 1), mask_value, device=device),
                        positions=torch.zeros((1, 1, 2, 2)), clean_latent=clean, uniform_mask=False)
    got = post_process_latent(denoised, state)
    ref = oracle.post_process_latent(np.full((1, 2, 3), -8.0, F32), np.full((1, 2, 3), 4.6875, F32),
                                     np.full((1, 2), mask_value, F32))
    ref = to_bf16(ref) if dtype == torch.bfloat16 else ref
    assert got.dtype == dtype and np.array_equal(_np(got), ref)


def test_composite_random_mask_is_bit_exact(device):
    d, c = _rand(8, (2, 50, 16), torch.bfloat16), _rand(9, (2, 50, 16), torch.float32)
    mask = torch.rand((2, 50), generator=torch.Generator().manual_seed(4))
    state = LatentState(latent=d.to(device), denoise_mask=mask.to(device), positions=torch.zeros(1),
                        clean_latent=c.to(device), uniform_mask=False)
    got = post_process_latent(d.to(device), state)
    ref = to_bf16(oracle.post_process_latent(d.float().numpy(), c.numpy(), mask.numpy()))
    assert np.array_equal(_np(got), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_finite_check(device, dtype):
    n = 3_000_001  # several grid-stride passes of the capped grid
    x = torch.zeros(n, dtype=dtype, device=device)
    assert all_finite(x) == [True]
    for index in (0, 777_777, n - 1):
        for bad in (float("nan"), float("inf"), float("-inf")):
            y = x.clone()
            y[index] = bad
            assert all_finite(y) == [False], (index, bad)
            assert all_finite(x, y, x) == [True, False, True]
    assert all_finite(torch.zeros(0, dtype=dtype, device=device)) == [True]
    assert all_finite(torch.full((5,), 3.0e38, dtype=torch.float32, device=device)) == [True]


# ---- the denoise step's control flow (reference test_denoise.py:13-67) -----------------------------


class _ConstantX0:
    def __init__(self, value=0.0):
        self.value = value
        self.calls = []

    def __call__(self, video, audio=None):
        self.calls.append(video)
        return torch.full_like(video.latent, self.value), None


def _state(device, mixed=False, dtype=torch.float32):
    mask = torch.tensor([[[0.5], [1.0]]], device=device) if mixed else torch.ones((1, 2, 1), device=device)
    return LatentState(latent=torch.ones((1, 2, 3), dtype=dtype, device=device), denoise_mask=mask,
                       positions=torch.zeros((1, 3, 2, 2), device=device),
                       clean_latent=torch.full((1, 2, 3), 4.0, dtype=dtype, device=device), uniform_mask=not mixed)


def test_uniform_state_uses_batch_scalar_timestep(device):
    model = _ConstantX0()
    result, audio = denoise_step(_state(device), sigma=1.0, sigma_next=0.0, transformer=model,
                                 video_context=torch.zeros((1, 1, 4), device=device))
    assert audio is None and model.calls[0].timesteps.shape == (1,)
    assert torch.equal(result.latent, torch.zeros_like(result.latent))


def test_mixed_mask_uses_per_token_timestep_and_preserves_clean_fraction(device):
    model = _ConstantX0()
    result, _ = denoise_step(_state(device, mixed=True), sigma=1.0, sigma_next=0.0, transformer=model,
                             video_context=torch.zeros((1, 1, 4), device=device))
    assert torch.equal(model.calls[0].timesteps.cpu(), torch.tensor([[0.5, 1.0]]))
    assert torch.equal(result.latent[:, 0].cpu(), torch.full((1, 3), 2.0))
    assert torch.equal(result.latent[:, 1].cpu(), torch.zeros((1, 3)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nonfinite_step_raises(device, dtype):
    with pytest.raises(LTX2DenoiseError, match="nonfinite video latent"):
        denoise_step(_state(device, dtype=dtype), sigma=1.0, sigma_next=0.5, transformer=_ConstantX0(float("nan")),
                     video_context=torch.zeros((1, 1, 4), device=device))


def test_disabled_video_is_not_advanced_or_checked(device):
    state = _state(device)
    result, _ = denoise_step(state, sigma=1.0, sigma_next=0.5, transformer=_ConstantX0(float("nan")),
                             video_context=torch.zeros((1, 1, 4), device=device), video_enabled=False)
    assert result is state


def test_step_rejects_ancestral_and_noise(device):
    with pytest.raises(ValueError, match="must not receive transition noise"):
        denoise_step(_state(device), sigma=1.0, sigma_next=0.5, transformer=_ConstantX0(),
                     video_context=torch.zeros((1, 1, 4), device=device), video_noise=torch.zeros(1))
    assert denoise_mod.modality_from_state(_state(device), torch.zeros(1), 0.5).timesteps.dtype == torch.float32
