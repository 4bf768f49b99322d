"""FLUX.2 and config-1 block parity on the GPU, through the MI355X operator surface
(``kinomlx_amd.flux2``), against the FP32 oracle on the same seeded inputs.

Bars (``tests.conftest.assert_block_parity``) against the FP32 evaluation: at D <= 1024 the north
star (cosine similarity >= 0.9995 and every element within 2e-2 beyond the bf16 output's own
rounding; the literal max abs error <= 2e-2 for blocks run with an FP32 residual stream, FP32 in
and out); at D = 4096 (config 2) cosine >= 0.9995, relative L2 <= 6e-3 and an RMS error within
1.25x the rounding noise of the FP32 evaluation rounded where this build stores bf16. Config 2's
double block hands its output to the single block in FP32. The standalone adjacent-pair
``rotate`` is bit-exact.
"""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.flux2 import kv as flux_kv
from kinomlx_amd.flux2 import transformer as flux
from tests import _torch_ref
from tests._blocks import flux_case
from tests.conftest import assert_block_parity, max_abs, rel_l2

pytestmark = pytest.mark.gpu
F32 = np.float32


def _np(t):
    return t.float().cpu().numpy()


def _check(got, ref, kx, graph, what, fp32_out=False, fp32_bar=True):
    assert_block_parity(got, ref, what, ref_kx=kx, graph=graph, fp32_out=fp32_out, small=fp32_bar)


def _run_double(spec, p, inputs, device, *, fuse=True, batch=1, fp32=False, out_dtype=None):
    block = workloads.build_flux_double_block(spec, p, device, fuse=fuse)
    image = inputs["image"].to(device).expand(batch, -1, -1).contiguous()
    text = inputs["text"].to(device).expand(batch, -1, -1).contiguous()
    if fp32:
        image, text = image.float(), text.float()
    im = p["image_mod"].reshape(1, -1).to(device).expand(batch, -1)
    tm = p["text_mod"].reshape(1, -1).to(device).expand(batch, -1)
    i_out, t_out = block(image, text, im, tm, workloads.flux_tables(spec, device), out_dtype=out_dtype)
    torch.cuda.synchronize()
    return i_out, t_out


DOUBLE_SPECS = [
    workloads.FluxSpec(grid=(4, 8), text_tokens=8, dim=512, heads=4, head_dim=128, ff_hidden=1024, ff="swiglu"),
    workloads.FluxSpec(grid=(5, 7), text_tokens=3, dim=1024, heads=16, head_dim=64, ff_hidden=4096, ff="gelu"),
    workloads.FluxSpec(grid=(8, 16), text_tokens=32, dim=4096, heads=32, head_dim=128, ff_hidden=12288,
                       ff="swiglu"),
]


@pytest.mark.parametrize("spec", DOUBLE_SPECS, ids=["swiglu-d512", "gelu-h64-ragged", "swiglu-d4096"])
def test_double_block_matches_oracle(device, spec):
    p, op, _, inputs, rope = flux_case(spec)
    i_out, t_out = _run_double(spec, p, inputs, device)
    image, text = inputs["image"][0].float().numpy(), inputs["text"][0].float().numpy()
    args = (op, image, text, op["image_mod"], op["text_mod"], rope)
    ri, rt = oracle.flux_double_block(*args, heads=spec.heads, ff=spec.ff)
    gi, gt = oracle.flux_double_block(*args, heads=spec.heads, ff=spec.ff, bf16_graph=True)
    ki, kt = oracle.flux_double_block(*args, heads=spec.heads, ff=spec.ff, rounding_mode="kx")
    small = spec.dim <= 1024
    _check(_np(i_out[0]), ri, ki, gi, "image", fp32_bar=small)
    _check(_np(t_out[0]), rt, kt, gt, "text", fp32_bar=small)
    i32, t32 = _run_double(spec, p, inputs, device, fp32=True)
    assert i32.dtype == torch.float32
    _check(_np(i32[0]), ri, ki, gi, "  image fp32 out", fp32_out=True, fp32_bar=small)
    _check(_np(t32[0]), rt, kt, gt, "  text fp32 out", fp32_out=True, fp32_bar=small)


def test_config1_block_full_size_matches_oracle(device):
    """Config 1 at its full size: 1024 image (32 x 32) + 128 text tokens, D = 1024, 16 x 64,
    GELU MLP x 4, 2D per-axis RoPE (theta 1e4)."""
    spec = workloads.CONFIGS[1]
    p, op, _, inputs, rope = flux_case(spec)
    i_out, t_out = _run_double(spec, p, inputs, device)
    image, text = inputs["image"][0].float().numpy(), inputs["text"][0].float().numpy()
    args = (op, image, text, op["image_mod"], op["text_mod"], rope)
    ri, rt = oracle.config1_double_block(*args, heads=spec.heads)
    gi, gt = oracle.config1_double_block(*args, heads=spec.heads, bf16_graph=True)
    ki, kt = oracle.config1_double_block(*args, heads=spec.heads, rounding_mode="kx")
    _check(_np(i_out[0]), ri, ki, gi, "config1 image")
    _check(_np(t_out[0]), rt, kt, gt, "config1 text")
    i32, t32 = _run_double(spec, p, inputs, device, fp32=True)
    _check(_np(i32[0]), ri, ki, None, "config1 image fp32 out", fp32_out=True)
    _check(_np(t32[0]), rt, kt, None, "config1 text fp32 out", fp32_out=True)


def test_double_block_unfused_and_batched_agree_with_fused(device):
    spec = DOUBLE_SPECS[0]
    p, _, _, inputs, _ = flux_case(spec)
    fi, ft = _run_double(spec, p, inputs, device)
    ui, ut = _run_double(spec, p, inputs, device, fuse=False)
    bi, bt = _run_double(spec, p, inputs, device, batch=2)
    # the fused projections norm and rotate Q/K in their epilogue (the norm's sum of squares in
    # another order than the standalone pass: a bf16 ulp in a few Q/K elements)
    for f, u in ((fi, ui), (ft, ut)):
        assert rel_l2(_np(f), _np(u)) < 1e-3 and max_abs(_np(f), _np(u)) < 2e-2
    assert torch.equal(bi[0], fi[0]) and torch.equal(bi[1], fi[0])
    assert torch.equal(bt[0], ft[0]) and torch.equal(bt[1], ft[0])


@pytest.mark.parametrize("dim,heads,hidden", [(512, 4, 1024), (4096, 32, 12288)], ids=["d512", "d4096"])
def test_single_block_matches_oracle(device, dim, heads, hidden):
    spec = workloads.FluxSpec(grid=(4, 8), text_tokens=8, dim=dim, heads=heads, head_dim=128,
                              ff_hidden=hidden, ff="swiglu", single=True)
    p, op, single, inputs, rope = flux_case(spec)
    x = torch.cat([inputs["text"], inputs["image"]], dim=1)
    block = workloads.build_flux_single_block(spec, p, device)
    mod, tables = p["single_mod"].reshape(1, -1).to(device), workloads.flux_tables(spec, device)
    got = block(x.to(device), mod, tables)
    xn = x[0].float().numpy()
    ref = oracle.flux_single_block(single, xn, op["single_mod"], rope, heads=heads, width=dim)
    graph = oracle.flux_single_block(single, xn, op["single_mod"], rope, heads=heads, width=dim, bf16_graph=True)
    kx = oracle.flux_single_block(single, xn, op["single_mod"], rope, heads=heads, width=dim, rounding_mode="kx")
    small = dim <= 1024
    _check(_np(got[0]), ref, kx, graph, "single", fp32_bar=small)
    got32 = block(x.to(device).float(), mod, tables)
    assert got32.dtype == torch.float32
    _check(_np(got32[0]), ref, kx, graph, "  single fp32 out", fp32_out=True, fp32_bar=small)


def test_config2_double_then_single_full_size_matches_fp32_evaluation(device):
    """Config 2 at full size: 4096 image (64 x 64) + 512 text tokens, D = 4096, 32 x 128,
    SwiGLU 12288; one double-stream block, then one single-stream block over [text, image],
    with the residual stream handed between the blocks in FP32."""
    spec = workloads.CONFIGS[2]
    p, op, single, inputs, rope = flux_case(spec)
    i_out, t_out = _run_double(spec, p, inputs, device, out_dtype=torch.float32)
    assert i_out.dtype == torch.float32
    sblock = workloads.build_flux_single_block(spec, p, device)
    tables = workloads.flux_tables(spec, device)
    mod = p["single_mod"].reshape(1, -1).to(device)
    joined = torch.cat([t_out, i_out], dim=1)
    got = _np(sblock(joined, mod, tables, out_dtype=torch.bfloat16)[0])
    got32 = _np(sblock(joined, mod, tables)[0])
    del sblock, joined

    tp = {k: torch.from_numpy(np.asarray(v)).to(device) for k, v in op.items()}
    sp = {k: torch.from_numpy(np.asarray(v)).to(device) for k, v in single.items()}
    rope_d = tuple(torch.from_numpy(t).to(device) for t in rope)
    image, text = inputs["image"][0].float().to(device), inputs["text"][0].float().to(device)
    torch.backends.cuda.matmul.allow_tf32 = False
    outs = {}
    with torch.no_grad():
        for mode in (None, "kx", "graph"):
            ri, rt = _torch_ref.flux_double_block(tp, image, text, tp["image_mod"], tp["text_mod"], rope_d,
                                                  spec.heads, rounding_mode=mode)
            if mode == "graph":  # the reference hands the hidden state between blocks in bf16
                ri, rt = _torch_ref.bf16_store(ri), _torch_ref.bf16_store(rt)
            outs[mode] = _torch_ref.flux_single_block(sp, torch.cat([rt, ri]), tp["single_mod"], rope_d, spec.heads,
                                                      spec.dim, rounding_mode=mode).cpu().numpy()
    _check(got, outs[None], outs["kx"], outs["graph"], "config2 double+single", fp32_bar=False)
    _check(got32, outs[None], outs["kx"], outs["graph"], "config2 double+single fp32 out", fp32_out=True, fp32_bar=False)


# ---- the standalone operator surface ---------------------------------------------------------


@pytest.mark.parametrize("table_batch", [1, 2])
def test_rotate_is_bit_exact(device, table_batch):
    """``flux2.transformer.rotate`` (``transformer.py:25-29``): adjacent pairs, FP32 products
    each rounded, then the sum, one cast; tables from ``rotary_positions`` of 4-axis ids."""
    r = np.random.default_rng(71)
    batch, tokens, heads, dh = 2, 19, 3, 128
    x = oracle.to_bf16((r.standard_normal((batch, tokens, heads, dh)) * 3).astype(F32))
    ids = torch.from_numpy(r.integers(0, 64, (table_batch, tokens, 4)).astype(np.float32)).to(device)
    cos, sin = flux.rotary_positions(ids)
    assert cos.shape == (table_batch, tokens, 1, dh)
    got = _np(flux.rotate(torch.from_numpy(x).to(device).to(torch.bfloat16), (cos, sin)))
    c, s = _np(cos), _np(sin)
    ref = oracle.to_bf16(oracle.pair_rope(x, np.broadcast_to(c, (batch, tokens, 1, dh)),
                                          np.broadcast_to(s, (batch, tokens, 1, dh))))
    assert np.array_equal(got, ref)


def test_rotary_positions_follow_the_2000_power_law(device):
    ids = torch.tensor([[[1.0, 2.0, 3.0, 4.0]]], device=device)
    cos, _ = flux.rotary_positions(ids)
    ref_cos, _ = oracle.flux_rotary_positions(ids.cpu().numpy())
    assert np.allclose(_np(cos).reshape(-1), np.asarray(ref_cos).reshape(-1), atol=2e-6)


def test_attend_and_joint_attention_match_oracle(device):
    r = np.random.default_rng(72)
    tokens, heads, dh = 77, 4, 128
    q, k, v = (oracle.to_bf16(r.standard_normal((1, tokens, heads, dh)).astype(F32)) for _ in range(3))
    qd, kd, vd = (torch.from_numpy(a).to(device).to(torch.bfloat16) for a in (q, k, v))
    got = _np(flux_kv.attend(qd, kd, vd))
    ref = oracle.attention(q[0].reshape(tokens, -1), k[0].reshape(tokens, -1), v[0].reshape(tokens, -1), heads=heads)
    assert got.shape == (1, tokens, heads, dh)
    assert rel_l2(got[0].reshape(tokens, -1), ref) < 8e-3
    ids = torch.from_numpy(r.integers(0, 32, (1, tokens, 4)).astype(np.float32)).to(device)
    tables = flux.rotary_positions(ids)
    joint = _np(flux.joint_attention(qd, kd, vd, tables))
    c, s = (_np(t)[0, :, 0] for t in tables)
    qr = oracle.to_bf16(oracle.pair_rope(q[0], c[:, None], s[:, None])).reshape(tokens, -1)
    kr = oracle.to_bf16(oracle.pair_rope(k[0], c[:, None], s[:, None])).reshape(tokens, -1)
    ref = oracle.attention(qr, kr, v[0].reshape(tokens, -1), heads=heads)
    assert joint.shape == (1, tokens, heads * dh)
    assert rel_l2(joint[0], ref) < 8e-3


def test_normalized_qknorm_swiglu_and_modulation(device):
    r = np.random.default_rng(73)
    x = oracle.to_bf16(r.standard_normal((9, 1024)).astype(F32))
    shift, scale = (r.standard_normal(1024).astype(F32) * 0.5 for _ in range(2))
    xd = torch.from_numpy(x).to(device).to(torch.bfloat16)
    got = _np(flux.normalized(xd, torch.from_numpy(shift).to(device), torch.from_numpy(scale).to(device)))
    assert max_abs(got, oracle.normalized(x, shift, scale)) < 2.0**-7 * (1 + np.abs(got).max())

    norm = flux.QKNorm()
    w = oracle.to_bf16((1 + 0.1 * r.standard_normal(128)).astype(F32))
    norm.weight = torch.from_numpy(w).to(device).to(torch.bfloat16)
    heads = oracle.to_bf16(r.standard_normal((9, 8, 128)).astype(F32))
    got = _np(norm(torch.from_numpy(heads).to(device).to(torch.bfloat16)))
    assert rel_l2(got, oracle.rms_norm(heads, w, 1e-6)) < 4e-3

    got = _np(flux.swiglu(xd))
    assert rel_l2(got, oracle.swiglu(x)) < 4e-3

    mod = flux.Modulation()
    wm = oracle.to_bf16((r.standard_normal((3 * 512, 1024)) * 0.02).astype(F32))
    mod.linear = flux.Linear(torch.from_numpy(wm).to(device).to(torch.bfloat16))
    got = _np(mod(xd))
    ref = oracle.linear(oracle.to_bf16(oracle.silu(x)), wm)
    assert rel_l2(got, ref) < 4e-3
