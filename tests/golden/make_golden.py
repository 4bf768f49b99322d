"""Writes the committed golden vectors under ``tests/golden/`` (run: ``python -m
tests.golden.make_golden``). Test data, not product code.

* ``rope_grid_known_answer.npz`` — the reference's own known-answer case for the LTX RoPE
  frequency grid (``tests/models/ltx2/transformer/test_primitives.py:115-132``: positions
  ``[0, 1]`` with ``max_pos (20,)``, dim 8, 2 heads, expected angles
  ``float32(10000 ** linspace(0, 1, 4) * pi / 2) * float32(2 * 0.5 / 20 - 1)``), computed in float64
  exactly as that test computes its expectation.
* ``ops_small.npz`` — seeded inputs and FP32-oracle outputs of every operator on the path at
  tiny shapes (norms, activations, RoPE, attention, linear, affine int4/int8 packing and
  dequantisation), so that kernel tests and the oracle are both held to fixed vectors.
* ``blocks_small.npz`` — FP32-oracle outputs of one small LTX-2 block, one FLUX.2 double block,
  one config-1-style GELU double block and one Krea 2 block, on the seeded synthetic workloads
  of ``kinomlx_amd.workloads`` / ``tests._blocks`` (parameters are regenerated from their seeds;
  a digest of the inputs is stored to detect generator drift).

The reference itself cannot run in this container (MLX is absent, Python 3.10 cannot parse
it), so apart from the known-answer case these vectors are the oracle's: they pin the oracle
and the kernels against drift, and the oracle is pinned to the reference by
``tests/test_oracle.py``.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

import oracle
from kinomlx_amd import workloads
from tests._blocks import flux_case, krea_case, ltx_case

HERE = Path(__file__).resolve().parent
F32 = np.float32

LTX_SPEC = workloads.LTXSpec(grid=(1, 2, 8), text_tokens=4, dim=512, heads=4, head_dim=128)
FLUX_SPEC = workloads.FluxSpec(grid=(2, 4), text_tokens=4, dim=512, heads=4, head_dim=128, ff_hidden=512, ff="swiglu")
GELU_SPEC = workloads.FluxSpec(grid=(2, 4), text_tokens=4, dim=512, heads=8, head_dim=64, ff_hidden=1024, ff="gelu")
KREA_SHAPE = dict(hidden=512, heads=4, kv_heads=2, tokens=12, ff_hidden=512)


def digest(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(np.asarray(a, dtype=F32)).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8).copy()


def rope_grid_known_answer() -> dict:
    positions = np.array([[[[0.0, 1.0]]]], dtype=F32)
    grid = np.power(10000.0, np.linspace(0.0, 1.0, 4, dtype=np.float64))
    angles = (grid * np.pi / 2).astype(F32) * F32(2 * 0.5 / 20 - 1)
    return {
        "positions": positions,
        "cos": np.cos(angles).astype(F32).reshape(1, 2, 1, 2),
        "sin": np.sin(angles).astype(F32).reshape(1, 2, 1, 2),
    }


def ops_small() -> dict:
    r = np.random.default_rng(20261202)
    bf = oracle.to_bf16
    out: dict[str, np.ndarray] = {}
    x = bf((r.standard_normal((9, 512)) * 2).astype(F32))
    w = bf((1 + 0.1 * r.standard_normal(512)).astype(F32))
    shift, scale = (r.standard_normal(512).astype(F32) * 0.5 for _ in range(2))
    out.update(x=x, w=w, shift=shift, scale=scale)
    out["rms_norm"] = oracle.rms_norm(x, w, 1e-6)
    out["adaln"] = oracle.adaln(x, scale, shift)
    out["normalized"] = oracle.normalized(x, shift, scale)
    out["gelu"] = oracle.gelu_approx(x)
    out["silu"] = oracle.silu(x)
    out["swiglu"] = oracle.swiglu(x)
    # split RoPE: (B=1, T=9, H=4, half=64) head-major tables
    ang = r.uniform(-3, 3, (1, 4, 9, 64)).astype(F32)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    out.update(split_cos=cos, split_sin=sin, split_rope=bf(oracle.split_rope(x[None], cos, sin)[0]))
    pang = np.repeat(r.uniform(-3, 3, (9, 64)).astype(F32), 2, -1)
    pcos, psin = np.cos(pang).astype(F32), np.sin(pang).astype(F32)
    out.update(pair_cos=pcos, pair_sin=psin,
               pair_rope=bf(oracle.pair_rope(x.reshape(9, 4, 128), pcos[:, None], psin[:, None]).reshape(9, 512)))
    q = bf(r.standard_normal((37, 128)).astype(F32))
    k = bf(r.standard_normal((45, 128)).astype(F32))
    v = bf(r.standard_normal((45, 128)).astype(F32))
    out.update(att_q=q, att_k=k, att_v=v, attention=oracle.attention(q, k, v, heads=2))
    lw = bf((r.standard_normal((96, 512)) * 0.05).astype(F32))
    lb = bf((r.standard_normal(96) * 0.1).astype(F32))
    out.update(lin_w=lw, lin_b=lb, linear=oracle.linear(x, lw, lb))
    xq = x[:, :256]
    qb = lb[:64]
    for bits in (4, 8):
        qw = (r.standard_normal((64, 256)) * 0.02).astype(F32)
        words, scales, biases = oracle.quantize_affine(qw, 64, bits)
        out[f"q{bits}_w"] = qw
        out[f"q{bits}_words"] = words
        out[f"q{bits}_scales"] = scales
        out[f"q{bits}_biases"] = biases
        out[f"q{bits}_dequant"] = oracle.dequantize_affine(words, scales, biases, group_size=64, bits=bits)
        out[f"q{bits}_linear"] = oracle.quantized_linear(xq, words, scales, biases, qb, group_size=64, bits=bits)
    return out


def blocks_small() -> dict:
    out: dict[str, np.ndarray] = {}
    _, op, inputs, pe = ltx_case(LTX_SPEC)
    x, ctx = inputs["x"][0].float().numpy(), inputs["context"][0].float().numpy()
    out["ltx_digest"] = digest(x, ctx, op["attn1.to_q.weight"], op["ff.proj_out.weight"], op["ada"])
    out["ltx"] = oracle.ltx_video_block(op, x, ctx, pe, heads=LTX_SPEC.heads)
    for name, spec in (("flux", FLUX_SPEC), ("gelu", GELU_SPEC)):
        _, fop, _, finputs, rope = flux_case(spec)
        image, text = finputs["image"][0].float().numpy(), finputs["text"][0].float().numpy()
        out[f"{name}_digest"] = digest(image, text, fop["attn.to_q.weight"], fop["image_mod"])
        i_out, t_out = oracle.flux_double_block(fop, image, text, fop["image_mod"], fop["text_mod"], rope,
                                                heads=spec.heads, ff=spec.ff)
        out[f"{name}_image"], out[f"{name}_text"] = i_out, t_out
    _, kop, kx, tmod, ids = krea_case(**KREA_SHAPE)
    dh = KREA_SHAPE["hidden"] // KREA_SHAPE["heads"]
    cos, sin = oracle.krea_rotary(ids.numpy(), theta=1000.0, axes_dims=(dh // 4, dh // 4, dh // 2))
    mod = tmod[0].float().numpy().reshape(6, -1) + kop["scale_shift_table"]
    xk = kx[0].float().numpy()
    out["krea_digest"] = digest(xk, mod, kop["attn.to_q.weight"], ids.numpy())
    out["krea"] = oracle.krea_block(kop, xk, mod, (cos[0], sin[0]), heads=KREA_SHAPE["heads"],
                                    kv_heads=KREA_SHAPE["kv_heads"])
    return out


def main() -> None:
    np.savez_compressed(HERE / "rope_grid_known_answer.npz", **rope_grid_known_answer())
    np.savez_compressed(HERE / "ops_small.npz", **ops_small())
    np.savez_compressed(HERE / "blocks_small.npz", **blocks_small())
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
