"""The committed golden vectors (``tests/golden/*.npz``, written by ``tests/golden/make_golden.py``).

CPU: the oracle reproduces the reference's own RoPE known-answer case and every stored vector
(any drift of the oracle or of the seeded workload generators fails here). GPU: every kernel on
the path and every block composition is held to the same stored vectors, with the bars of the
kernel and block parity tests (bit-exact for RoPE and dequantisation).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from tests._blocks import build_krea_block, device_tables, flux_case, krea_case, ltx_case
from tests.conftest import cosine, max_abs, rel_l2
from tests.golden import make_golden as mg

GOLDEN = Path(__file__).resolve().parent / "golden"
F32 = np.float32


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


OPS = _load("ops_small.npz")
BLOCKS = _load("blocks_small.npz")


# ---- CPU: the oracle against the stored vectors ----------------------------------------------


def test_oracle_reproduces_the_reference_rope_known_answer():
    g = _load("rope_grid_known_answer.npz")
    cos, sin = oracle.precompute_freqs_cis(g["positions"], dim=8, theta=10000.0, max_pos=(20,),
                                           use_middle_indices_grid=True, num_attention_heads=2)
    assert np.allclose(cos, g["cos"], atol=1e-6) and np.allclose(sin, g["sin"], atol=1e-6)


def test_oracle_reproduces_the_operator_vectors():
    fresh = mg.ops_small()
    assert sorted(fresh) == sorted(OPS)
    for key, value in OPS.items():
        if value.dtype == np.uint32 or key.endswith(("rope", "dequant")):
            assert np.array_equal(fresh[key], value), key
        else:
            assert max_abs(fresh[key], value) <= 1e-5 * (1 + np.abs(value).max()), key


def test_workload_generators_and_oracle_blocks_reproduce_the_block_vectors():
    fresh = mg.blocks_small()
    for key, value in BLOCKS.items():
        if key.endswith("_digest"):
            assert np.array_equal(fresh[key], value), f"{key}: the seeded workload generator drifted"
        else:
            assert max_abs(fresh[key], value) < 1e-4, key


def test_product_quantizer_packs_the_stored_words():
    from kinomlx_amd.kernels import quantized

    for bits in (4, 8):
        words, scales, biases = quantized.quantize(torch.from_numpy(OPS[f"q{bits}_w"]), 64, bits)
        assert np.array_equal(words.numpy().view(np.uint32), OPS[f"q{bits}_words"])
        assert np.array_equal(scales.float().numpy(), OPS[f"q{bits}_scales"])
        assert np.array_equal(biases.float().numpy(), OPS[f"q{bits}_biases"])


# ---- GPU: kernels and blocks against the stored vectors --------------------------------------


def _bf(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32)).to(device).to(torch.bfloat16)


def _f32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32)).to(device)


def _np(t):
    return t.float().cpu().numpy()


def _one_ulp(got, ref):
    return np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-6)


@pytest.mark.gpu
def test_kernels_match_the_operator_vectors(device):
    from kinomlx_amd.flux2 import transformer as flux
    from kinomlx_amd.kernels import fused_ops, mpp_linear, quantized, split_rope
    from kinomlx_amd.ltx2 import dense_attention, transformer

    g = OPS
    x = _bf(g["x"], device)
    assert _one_ulp(_np(fused_ops.rms_norm(x, _bf(g["w"], device))), g["rms_norm"])
    assert _one_ulp(_np(transformer.adaln(x, _f32(g["scale"], device), _f32(g["shift"], device), 1e-6)), g["adaln"])
    assert _one_ulp(_np(flux.normalized(x, _f32(g["shift"], device), _f32(g["scale"], device))), g["normalized"])
    for name, fn in (("gelu", fused_ops.gelu_approx), ("silu", fused_ops.silu), ("swiglu", fused_ops.swiglu)):
        assert _one_ulp(_np(fn(x)), oracle.to_bf16(g[name])), name

    cos = torch.from_numpy(np.ascontiguousarray(g["split_cos"].transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    sin = torch.from_numpy(np.ascontiguousarray(g["split_sin"].transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    assert np.array_equal(_np(split_rope.rotate(x[None], cos, sin)[0]), g["split_rope"])
    pair = flux.rotate(x.view(1, 9, 4, 128), (_f32(g["pair_cos"], device)[None, :, None],
                                              _f32(g["pair_sin"], device)[None, :, None]))
    assert np.array_equal(_np(pair).reshape(9, 512), g["pair_rope"])

    att = dense_attention.dense_attention(_bf(g["att_q"], device), _bf(g["att_k"], device),
                                          _bf(g["att_v"], device), heads=2)
    assert rel_l2(_np(att), g["attention"]) < 8e-3

    lin = mpp_linear.linear(x, _bf(g["lin_w"], device), _bf(g["lin_b"], device), transposed=True)
    assert rel_l2(_np(lin), g["linear"]) < 4e-3
    xq = _bf(g["x"][:, :256], device)
    for bits in (4, 8):
        words = torch.from_numpy(g[f"q{bits}_words"].view(np.int32)).to(device)
        scales, biases = _bf(g[f"q{bits}_scales"], device), _bf(g[f"q{bits}_biases"], device)
        deq = quantized.dequantize(words, scales, biases, group_size=64, bits=bits)
        assert np.array_equal(_np(deq), g[f"q{bits}_dequant"]), bits
        got = quantized.quantized_matmul(xq, words, scales, biases, group_size=64, bits=bits,
                                         bias=_bf(g["lin_b"][:64], device))
        assert rel_l2(_np(got), g[f"q{bits}_linear"]) < 4e-3, bits


def _block_ok(got, ref, what):
    c, m = cosine(got, ref), max_abs(got, ref)
    print(f"{what}: cosine {c:.7f} max_abs {m:.4g}")
    assert c >= 0.9995 and m <= 2e-2, (what, c, m)


@pytest.mark.gpu
def test_blocks_match_the_block_vectors(device):
    from kinomlx_amd.krea2 import transformer as krea
    from kinomlx_amd.ltx2.transformer import TransformerArgs

    p, _, inputs, pe = ltx_case(mg.LTX_SPEC)
    block = workloads.build_ltx_block(mg.LTX_SPEC, p, device)
    out, _ = block(TransformerArgs(x=inputs["x"].to(device), context=inputs["context"].to(device),
                                   timesteps=p["timesteps"].to(device), positional_embeddings=device_tables(pe, device)))
    _block_ok(_np(out.x[0]), BLOCKS["ltx"], "ltx")

    for name, spec in (("flux", mg.FLUX_SPEC), ("gelu", mg.GELU_SPEC)):
        fp, _, _, finputs, _ = flux_case(spec)
        fblock = workloads.build_flux_double_block(spec, fp, device)
        i_out, t_out = fblock(finputs["image"].to(device), finputs["text"].to(device),
                              fp["image_mod"].reshape(1, -1).to(device), fp["text_mod"].reshape(1, -1).to(device),
                              workloads.flux_tables(spec, device))
        _block_ok(_np(i_out[0]), BLOCKS[f"{name}_image"], f"{name} image")
        _block_ok(_np(t_out[0]), BLOCKS[f"{name}_text"], f"{name} text")

    shape = mg.KREA_SHAPE
    kp, _, kx, tmod, ids = krea_case(**shape)
    dh = shape["hidden"] // shape["heads"]
    tables = krea.Krea2RotaryEmbedding(theta=1000.0, axes_dims=(dh // 4, dh // 4, dh // 2))(ids.to(device))
    kblock = build_krea_block(kp, shape["hidden"], shape["heads"], shape["kv_heads"], device)
    got = kblock(kx.to(device), time_modulation=tmod.to(device), rotary=tables, attention_mask=None)
    _block_ok(_np(got[0]), BLOCKS["krea"], "krea")
