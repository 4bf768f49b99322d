"""Shared joint audio/video block case for the oracle pins and the GPU parity tests."""

import numpy as np

import oracle
from kinomlx_amd import workloads

SPEC = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
AUDIO = workloads.LTXAudioSpec(tokens=20, text_tokens=8, dim=512, heads=8, head_dim=64)


def oracle_av_params(p: dict) -> dict:
    """Workload joint-block parameters -> the oracle's dict (tables folded with the step rows)."""
    skip = {"timesteps", "audio_timesteps", "cross_ss", "cross_gate", "audio_cross_ss", "audio_cross_gate"}
    out = {k: v.float().numpy() for k, v in p.items() if k not in skip and "scale_shift_table" not in k}
    for pre in ("", "audio_"):
        out[f"{pre}ada"] = (p[f"{pre}scale_shift_table"].float() + p[f"{pre}timesteps"].float()[0, 0]).numpy()
        out[f"{pre}prompt"] = p[f"{pre}prompt_scale_shift_table"].float().numpy()
    for stream, pre in (("video", ""), ("audio", "audio_")):
        table = p[f"scale_shift_table_a2v_ca_{stream}"].float()
        rows = np.concatenate([(table[:4] + p[f"{pre}cross_ss"].float()[0, 0]).numpy(),
                               (table[4:5] + p[f"{pre}cross_gate"].float()[0, 0]).numpy()])
        out[f"av_{stream}"] = rows
    return out


def tables(inputs):
    """Oracle RoPE tables: video (3D) and audio (1D) self-attention, and both cross tables (the
    temporal axis at the audio stream's width)."""
    vpos, apos = inputs["positions"].numpy(), inputs["audio_positions"].numpy()
    pe = oracle.precompute_freqs_cis(vpos, dim=SPEC.dim, use_middle_indices_grid=True, num_attention_heads=SPEC.heads)
    audio_pe = oracle.precompute_freqs_cis(apos, dim=AUDIO.dim, max_pos=(20,), use_middle_indices_grid=True,
                                          num_attention_heads=AUDIO.heads)
    inner = AUDIO.heads * AUDIO.head_dim
    cross = oracle.precompute_freqs_cis(vpos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                       num_attention_heads=AUDIO.heads)
    audio_cross = oracle.precompute_freqs_cis(apos[:, 0:1], dim=inner, max_pos=(20,), use_middle_indices_grid=True,
                                             num_attention_heads=AUDIO.heads)
    return pe, audio_pe, cross, audio_cross


def oracle_run(op, inputs, pes, bf16_graph=False):
    pe, audio_pe, cross, audio_cross = pes
    return oracle.ltx_av_block(
        op, inputs["x"][0].float().numpy(), inputs["audio_x"][0].float().numpy(),
        inputs["context"][0].float().numpy(), inputs["audio_context"][0].float().numpy(),
        pe, audio_pe, cross, audio_cross, heads=SPEC.heads, audio_heads=AUDIO.heads, bf16_graph=bf16_graph)
