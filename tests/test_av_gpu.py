"""The joint audio/video LTX-2 block on the GPU against the oracle (block bar, both streams:
cosine >= 0.9995 and |got - ref| <= 2e-2 + ulp_bf16(ref) / 2 elementwise, ``assert_block_bar``;
the reference's own bf16 graph is printed beside it)."""

import numpy as np
import pytest
import torch

from kinomlx_amd import workloads
from kinomlx_amd.ltx2.rope import precompute_freqs_cis
from kinomlx_amd.ltx2.transformer import TransformerArgs
from tests._av import AUDIO, SPEC, oracle_av_params, oracle_run, tables
from tests.conftest import assert_block_bar

pytestmark = pytest.mark.gpu


def _check(got, ref, graph):
    assert_block_bar(got, ref, "a/v", context=graph)


def _args(p, inputs, device):
    inner = AUDIO.heads * AUDIO.head_dim
    vpos, apos = inputs["positions"].to(device), inputs["audio_positions"].to(device)
    pe = precompute_freqs_cis(vpos, dim=SPEC.dim, use_middle_indices_grid=True, num_attention_heads=SPEC.heads)
    audio_pe = precompute_freqs_cis(apos, dim=AUDIO.dim, max_pos=(20,), use_middle_indices_grid=True,
                                    num_attention_heads=AUDIO.heads)
    cross = precompute_freqs_cis(vpos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                 num_attention_heads=AUDIO.heads)
    audio_cross = precompute_freqs_cis(apos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                       num_attention_heads=AUDIO.heads)
    d = lambda k: p[k].to(device)  # noqa: E731
    video = TransformerArgs(x=inputs["x"].to(device), context=inputs["context"].to(device), timesteps=d("timesteps"),
                            positional_embeddings=pe, cross_positional_embeddings=cross,
                            cross_scale_shift_timestep=d("cross_ss"), cross_gate_timestep=d("cross_gate"))
    audio = TransformerArgs(x=inputs["audio_x"].to(device), context=inputs["audio_context"].to(device),
                            timesteps=d("audio_timesteps"), positional_embeddings=audio_pe,
                            cross_positional_embeddings=audio_cross, cross_scale_shift_timestep=d("audio_cross_ss"),
                            cross_gate_timestep=d("audio_cross_gate"))
    return video, audio


@pytest.mark.parametrize("fuse", [True, False])
def test_av_block_matches_oracle(device, fuse):
    p = workloads.ltx_av_params(SPEC, AUDIO)
    inputs = workloads.ltx_av_inputs(SPEC, AUDIO)
    block = workloads.build_ltx_av_block(SPEC, AUDIO, p, device, fuse=fuse)
    video, audio = _args(p, inputs, device)
    out_v, out_a = block(video, audio)
    torch.cuda.synchronize()
    op = oracle_av_params(p)
    pes = tables(inputs)
    ref_v, ref_a = oracle_run(op, inputs, pes)
    graph_v, graph_a = oracle_run(op, inputs, pes, bf16_graph=True)
    _check(out_v.x[0].float().cpu().numpy(), ref_v, graph_v)
    _check(out_a.x[0].float().cpu().numpy(), ref_a, graph_a)


def _quantized(p, bits):
    """Every 2-D linear weight of ``p`` in the packed affine form (group 64)."""
    from kinomlx_amd.kernels.quantized import quantize

    q = dict(p)
    for key in [k for k, v in p.items() if k.endswith(".weight") and v.dim() == 2 and v.shape[1] % 64 == 0]:
        name = key[: -len(".weight")]
        q[f"{name}.wq"], q[f"{name}.scales"], q[f"{name}.biases"] = quantize(q.pop(key), 64, bits)
        q[f"{name}.group_size"], q[f"{name}.bits"] = torch.tensor(64), torch.tensor(bits)
    return q


@pytest.mark.parametrize("bits", [None, 4], ids=["bf16", "int4"])
def test_av_block_side_stream_matches_one_stream(device, bits):
    """With both streams present the block runs the audio stream on a second HIP stream beside
    the video stream's; three chained blocks give the one-stream schedule's outputs bit for bit
    (with int4 layers each stream dequantizes into its own workspace)."""
    from kinomlx_amd import streams

    p = workloads.ltx_av_params(SPEC, AUDIO)
    if bits:
        p = _quantized(p, bits)
    inputs = workloads.ltx_av_inputs(SPEC, AUDIO)
    block = workloads.build_ltx_av_block(SPEC, AUDIO, p, device)
    outs = {}
    for two in (True, False):
        block.audio_side_stream = two
        video, audio = _args(p, inputs, device)
        seq = []
        for _ in range(3):
            video, audio = block(video, audio)
            seq.append((video.x.clone(), audio.x.clone()))
        torch.cuda.synchronize()
        outs[two] = seq
    assert streams._SIDE_STREAMS
    for (v2, a2), (v1, a1) in zip(outs[True], outs[False]):
        assert torch.equal(v2, v1) and torch.equal(a2, a1)


def test_disabled_audio_still_feeds_video(device):
    """A present but disabled audio stream is left as it is and still supplies the audio ->
    video K/V; the video output then differs from a block run without audio."""
    p = workloads.ltx_av_params(SPEC, AUDIO)
    inputs = workloads.ltx_av_inputs(SPEC, AUDIO)
    block = workloads.build_ltx_av_block(SPEC, AUDIO, p, device)
    video, audio = _args(p, inputs, device)
    from dataclasses import replace

    off = replace(audio, enabled=False)
    out_v, out_a = block(video, off)
    assert out_a is off
    alone, _ = block(video, None)
    assert not torch.equal(out_v.x, alone.x)


# ---- the joint transformer forward and denoising step ------------------------------------------

CHANNELS = 32


def _model_case():
    import oracle

    p = workloads.ltx_av_model_params(SPEC, AUDIO, 2, in_channels=CHANNELS, out_channels=CHANNELS)
    op = {}
    for name, value in p.items():
        op[name] = [{k: v.float().numpy() for k, v in b.items()} for b in value] if name == "blocks" \
            else value.float().numpy()
    inputs = workloads.ltx_av_model_inputs(SPEC, AUDIO, in_channels=CHANNELS)
    vpos, apos = inputs["positions"].numpy(), inputs["audio_positions"].numpy()
    inner = AUDIO.heads * AUDIO.head_dim
    pes = (oracle.precompute_freqs_cis(vpos, dim=SPEC.dim, use_middle_indices_grid=True, num_attention_heads=SPEC.heads),
           oracle.precompute_freqs_cis(apos, dim=AUDIO.dim, max_pos=(20,), use_middle_indices_grid=True,
                                       num_attention_heads=AUDIO.heads),
           oracle.precompute_freqs_cis(vpos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                       num_attention_heads=AUDIO.heads),
           oracle.precompute_freqs_cis(apos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                       num_attention_heads=AUDIO.heads))
    return p, op, inputs, pes


def _oracle_velocities(op, inputs, pes, sigma, bf16_graph=False):
    import oracle

    s = np.array([sigma], np.float32)
    return oracle.ltx_av_forward(op, inputs["latent"][0].float().numpy(), inputs["audio_latent"][0].float().numpy(),
                                 inputs["context"][0].float().numpy(), inputs["audio_context"][0].float().numpy(),
                                 s, s, s, s, pes, heads=SPEC.heads, audio_heads=AUDIO.heads, num_blocks=2,
                                 bf16_graph=bf16_graph)


def test_av_transformer_forward_matches_oracle(device):
    from kinomlx_amd.ltx2.wrappers import Modality

    p, op, inputs, pes = _model_case()
    model = workloads.build_ltx_av_model(SPEC, AUDIO, p, device, in_channels=CHANNELS, out_channels=CHANNELS)
    sig = torch.full((1,), 0.7, device=device)
    video = Modality(latent=inputs["latent"].to(device), context=inputs["context"].to(device), timesteps=sig,
                     sigma=sig, positions=inputs["positions"].to(device))
    audio = Modality(latent=inputs["audio_latent"].to(device), context=inputs["audio_context"].to(device),
                     timesteps=sig, sigma=sig, positions=inputs["audio_positions"].to(device))
    vel_v, vel_a = model(video, audio)
    ref_v, ref_a = _oracle_velocities(op, inputs, pes, 0.7)
    graph_v, graph_a = _oracle_velocities(op, inputs, pes, 0.7, bf16_graph=True)
    _check(vel_v[0].float().cpu().numpy(), ref_v, graph_v)
    _check(vel_a[0].float().cpu().numpy(), ref_a, graph_a)


def test_av_denoise_step_matches_oracle(device):
    import oracle
    from kinomlx_amd.ltx2.denoise import denoise_step
    from kinomlx_amd.ltx2.state import LatentState
    from kinomlx_amd.ltx2.wrappers import X0Model
    from oracle.ops import to_bf16

    p, op, inputs, pes = _model_case()
    model = X0Model(workloads.build_ltx_av_model(SPEC, AUDIO, p, device, in_channels=CHANNELS,
                                                 out_channels=CHANNELS))

    def state(latent, positions):
        latent = latent.to(device)
        return LatentState(latent=latent, denoise_mask=torch.ones((1, latent.shape[1], 1), device=device),
                           positions=positions.to(device), clean_latent=latent)

    sigma, nxt = 0.7, 0.45
    vs, aus = denoise_step(state(inputs["latent"], inputs["positions"]),
                           state(inputs["audio_latent"], inputs["audio_positions"]), sigma=sigma, sigma_next=nxt,
                           transformer=model, video_context=inputs["context"].to(device),
                           audio_context=inputs["audio_context"].to(device))

    def step(graph):
        out = []
        for lat, vel in zip((inputs["latent"], inputs["audio_latent"]), _oracle_velocities(op, inputs, pes, sigma, graph)):
            x = lat.float().numpy()
            d = to_bf16(oracle.to_denoised(x, to_bf16(vel)[None], np.array([sigma], np.float32)))
            out.append(to_bf16(oracle.euler_step(x, d, sigma, nxt))[0])
        return out

    (ref_v, ref_a), (g_v, g_a) = step(False), step(True)
    _check(vs.latent[0].float().cpu().numpy(), ref_v, g_v)
    _check(aus.latent[0].float().cpu().numpy(), ref_a, g_a)
