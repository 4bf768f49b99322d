"""Pins of the oracle's joint audio/video block (``oracle.ltx_av_block``) on the CPU."""

import numpy as np

import oracle
from kinomlx_amd import workloads
from tests._av import AUDIO, SPEC, oracle_av_params, oracle_run, tables


def _case():
    p = workloads.ltx_av_params(SPEC, AUDIO)
    return p, oracle_av_params(p), workloads.ltx_av_inputs(SPEC, AUDIO)


def test_zero_av_gates_reduce_to_the_two_single_stream_blocks():
    """With both A/V gates zero the A/V attention adds nothing: each stream equals its own
    single-stream block (attention, text cross-attention, feed-forward in the reference order)."""
    p, op, inputs = _case()
    op["av_video"][4] = 0.0
    op["av_audio"][4] = 0.0
    pes = tables(inputs)
    v, a = oracle_run(op, inputs, pes)
    ref_v = oracle.ltx_video_block(op, inputs["x"][0].float().numpy(), inputs["context"][0].float().numpy(), pes[0],
                                   heads=SPEC.heads)
    audio_params = {k[len("audio_"):]: val for k, val in op.items() if k.startswith("audio_")}
    ref_a = oracle.ltx_video_block(audio_params, inputs["audio_x"][0].float().numpy(),
                                   inputs["audio_context"][0].float().numpy(), pes[1], heads=AUDIO.heads)
    assert np.allclose(v, ref_v, atol=1e-5) and np.allclose(a, ref_a, atol=1e-5)


def test_each_stream_sees_the_other_only_through_its_gate():
    """Perturbing the audio input moves the video output only when the audio -> video gate is
    open, and the reverse; the cross-attention is therefore wired both ways."""
    p, op, inputs = _case()
    pes = tables(inputs)
    moved = dict(inputs, audio_x=inputs["audio_x"] * 1.5)
    v0, a0 = oracle_run(op, inputs, pes)
    v1, a1 = oracle_run(op, moved, pes)
    assert np.abs(v1 - v0).max() > 1e-3  # audio reaches video
    closed = dict(op, av_video=op["av_video"].copy())
    closed["av_video"][4] = 0.0
    v2, _ = oracle_run(closed, inputs, pes)
    v3, _ = oracle_run(closed, moved, pes)
    assert np.array_equal(v2, v3)
    moved_v = dict(inputs, x=inputs["x"] * 1.5)
    _, a4 = oracle_run(op, moved_v, pes)
    assert np.abs(a4 - a0).max() > 1e-3  # video reaches audio
