"""FP16 activations on the GPU: the reference's default LTX-2 transformer dtype
(``docs/PERFORMANCE.md:228-230``) through every hot-path operator and the block, against the FP32
oracle (``_f16`` entry points of ``include/kx355.h``: the bf16 kernels with fp16 MFMA products and
fp16 roundings).

Bars, written per test:
* norms, activations: within one fp16 ulp of the oracle's FP32 value (one rounding);
* split and pair RoPE: bit-exact against the oracle rounded to fp16 (``split_rope.py:35-56``);
* attention: the reference's own fp16 bar, relative L2 < 1e-3 against FP32 attention over its
  tile-edge shape list (``tests/models/ltx2/test_dense_attention.py:15,49-76``);
* linear: within one fp16 ulp (plus the FP32 accumulation-order slack) of the float64 product;
* the LTX-2 block: the block bar of ``tests.conftest`` with fp16 output roundings; at D = 4096 its
  elementwise anchor is the reference's own fp16 graph.
"""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import _lib, workloads
from kinomlx_amd.kernels import fused_ops, mpp_linear, split_rope
from kinomlx_amd.ltx2 import dense_attention
from kinomlx_amd.ltx2.transformer import TransformerArgs, adaln
from tests import _torch_ref
from tests._blocks import dense_params, device_tables, oracle_params
from tests.conftest import assert_block_parity, half_ulp_fp16, rel_l2

pytestmark = pytest.mark.gpu

F32 = np.float32
H = torch.float16


def _rng(seed):
    return np.random.default_rng(seed)


def _f16(a):
    return np.asarray(a, dtype=F32).astype(np.float16).astype(F32)


def _dev(a, device, dtype=H):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32)).to(device).to(dtype)


def _np(t):
    return t.float().cpu().numpy()


def _within_ulps(got, ref, ulps=1.0, atol=0.0):
    """|got - ref| <= ulps fp16 spacings (2 x half-ulp) at the larger of |got| and |ref| (an FP32
    value just below a power of two may round up across it), plus ``atol``."""
    got, ref = got.astype(np.float64), ref.astype(np.float64)
    bound = 2 * ulps * half_ulp_fp16(np.maximum(np.abs(got), np.abs(ref))) + atol
    err = np.abs(got - ref)
    worst = float(np.max(err - bound))
    assert worst <= 0, (worst, float(err.max()))


@pytest.mark.parametrize("dim", [1024, 4096, 96])
def test_rms_norm_fp16(device, dim):
    r = _rng(dim)
    x = _f16(r.standard_normal((37, dim)) * 3)
    w = _f16(1 + 0.1 * r.standard_normal(dim))
    got = fused_ops.rms_norm(_dev(x, device), _dev(w, device))
    assert got.dtype == H
    _within_ulps(_np(got), oracle.rms_norm(x, w))
    got = fused_ops.rms_norm(_dev(x, device))  # unweighted: the AdaLN kernel
    assert got.dtype == H
    _within_ulps(_np(got), oracle.rms_norm(x))
    got = fused_ops.rms_norm(_dev(x, device), _dev(w, device, torch.float32))  # fp32 weight
    _within_ulps(_np(got), oracle.rms_norm(x, w))


@pytest.mark.parametrize("xdtype", [H, torch.float32])
def test_adaln_fp16(device, xdtype):
    r = _rng(5)
    x = _f16(r.standard_normal((2, 70, 2048)) * 2)
    shift = (r.standard_normal((2, 1, 2048)) * 0.5).astype(F32)
    scale = (r.standard_normal((2, 1, 2048)) * 0.5).astype(F32)
    got = adaln(_dev(x, device, xdtype), _dev(scale, device, torch.float32), _dev(shift, device, torch.float32), 1e-6,
                out_dtype=H)
    assert got.dtype == H
    # y * (1 + scale) + shift cancels to near zero for some elements: there the two FP32
    # evaluations (FMA in the kernel, separate roundings in the oracle) differ by an FP32 ulp of
    # the operands (up to ~8), 1e-6 absolute, as the bf16 test allows
    _within_ulps(_np(got), oracle.adaln(x, scale, shift), atol=1e-6)


def test_activations_fp16(device):
    """GELU-tanh and SiLU over ``linspace(-8, 8, 65536)`` (``tests/kernels/test_fused_ops.py:18-36``),
    against float64 rounded to fp16: at most one fp16 ulp."""
    x = _f16(np.linspace(-8, 8, 65536))
    xd = _dev(x, device)
    x64 = x.astype(np.float64)
    inner = np.clip(np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64 ** 3), -10, 10)
    _within_ulps(_np(fused_ops.gelu_approx(xd)), 0.5 * x64 * (1 + np.tanh(inner)))
    _within_ulps(_np(fused_ops.silu(xd)), x64 / (1 + np.exp(-x64)))
    big = _dev(np.array([-128.0, 128.0] * 4), device)
    assert torch.isfinite(fused_ops.gelu_approx(big)).all() and torch.isfinite(fused_ops.silu(big)).all()


@pytest.mark.parametrize("batch,table_batch", [(1, 1), (2, 1), (2, 2)])
def test_split_rope_fp16_bit_exact(device, batch, table_batch):
    """``split_rope.rotate`` on fp16 (``split_rope.py:32``, the kernel-vs-graph shapes of
    ``tests/kernels/test_split_rope.py:31-50``): each product rounded in fp32, then the sum, one cast."""
    r = _rng(batch * 10 + table_batch)
    heads, tokens, half = 4, 13, 24
    x = _f16(r.standard_normal((batch, tokens, heads * 2 * half)) * 4)
    ang = r.uniform(-40, 40, (table_batch, heads, tokens, half)).astype(F32)
    cos, sin = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    assert split_rope.applies(_dev(x, device), _dev(cos, device, torch.float32), _dev(sin, device, torch.float32))
    got = split_rope.rotate(_dev(x, device), _dev(cos, device, torch.float32), _dev(sin, device, torch.float32))
    assert got.dtype == H
    ref = _f16(oracle.split_rope(x, cos, sin))
    assert np.array_equal(_np(got), ref)


def test_pair_rope_fp16_bit_exact(device):
    r = _rng(77)
    rows, heads, dh = 19, 3, 128
    x = _f16(r.standard_normal((rows, heads * dh)) * 3)
    ang = r.uniform(-30, 30, (rows, dh // 2)).astype(F32)
    cos = np.repeat(np.cos(ang), 2, axis=-1).astype(F32)
    sin = np.repeat(np.sin(ang), 2, axis=-1).astype(F32)
    out = torch.empty((rows, heads * dh), dtype=H, device=device)
    _lib.launch_rope_pair(_dev(x, device), out, _dev(cos, device, torch.float32), _dev(sin, device, torch.float32),
                          heads=heads, head_dim=dh, table_ld=dh, table_hs=0, tokens=rows, table_batched=False)
    ref = _f16(oracle.pair_rope(x.reshape(rows, heads, dh), cos[:, None], sin[:, None]).reshape(rows, -1))
    assert np.array_equal(_np(out), ref)


TILE_EDGES = [(7, 7), (16, 16), (33, 33), (517, 517), (300, 1024), (1, 300), (517, 33), (40, 5)]


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("tq,tk", TILE_EDGES)
def test_dense_attention_fp16_across_tile_edges(device, dim, tq, tk):
    """The reference's tile-edge list at its fp16 tolerance (relative L2 < 1e-3,
    ``tests/models/ltx2/test_dense_attention.py:15,49-64``)."""
    heads = 2
    g = torch.Generator().manual_seed(tq + tk + dim)
    q, k, v = (torch.randn((n, heads * dim), generator=g).to(H) for n in (tq, tk, tk))
    got = dense_attention.dense_attention(q.to(device), k.to(device), v.to(device), heads=heads)
    assert got.dtype == H and got.shape == q.shape
    ref = oracle.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), heads=heads)
    assert rel_l2(_np(got), ref) < 1e-3


def test_keys_past_a_partial_tile_take_no_weight_fp16(device):
    """``tests/models/ltx2/test_dense_attention.py:67-76``: a key one past the real keys, in the
    same buffer, that would dominate every row if the kernel read it."""
    heads, dim = 2, 128
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((n, heads * dim), generator=g).to(H) for n in (9, 17, 17))
    kp = torch.cat([k, torch.full((1, heads * dim), 8.0, dtype=H)]).to(device)
    vp = torch.cat([v, torch.full((1, heads * dim), 1000.0, dtype=H)]).to(device)
    got = dense_attention.dense_attention(q.to(device), kp[:17], vp[:17], heads=heads)
    ref = oracle.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), heads=heads)
    assert rel_l2(_np(got), ref) < 1e-3


def test_attention_fp16_gate_mask_and_split(device):
    """The gated, masked (score bias) and key-split forms in fp16 against the oracle."""
    heads, dim = 4, 128
    g = torch.Generator().manual_seed(11)
    q = torch.randn((1, 127, heads * dim), generator=g).to(H)
    k = torch.randn((1, 5376, heads * dim), generator=g).to(H)
    v = torch.randn((1, 5376, heads * dim), generator=g).to(H)
    gate = (torch.rand((1, 127, heads), generator=g) * 2).to(H)
    assert _lib.attention_splits(1, 127, 5376, heads) > 1
    got = dense_attention.batched_attention(q.to(device), k.to(device), v.to(device), heads=heads, gate=gate.to(device))
    ref = oracle.attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(), heads=heads)
    ref = (ref.reshape(127, heads, dim) * gate[0].float().numpy()[:, :, None]).reshape(127, -1)
    assert rel_l2(_np(got[0]), ref) < 1e-3
    mask = torch.rand((1, 127, 5376), generator=g) > 0.3
    got = dense_attention.batched_attention(q.to(device), k.to(device), v.to(device), heads=heads,
                                            mask=mask.to(device))
    bias = np.where(mask[0].numpy(), 0.0, -np.inf).astype(F32)
    ref = oracle.attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(), heads=heads, bias=bias)
    assert rel_l2(_np(got[0]), ref) < 1e-3


@pytest.mark.parametrize("m,n,k", [(70, 96, 64), (1000, 640, 512), (9216, 32, 4096), (127, 2048, 2048),
                                   (4864, 4096, 8192)])
@pytest.mark.parametrize("epi", ["bias", "gelu", "gated_f32", "gated_f16"])
def test_linear_fp16(device, m, n, k, epi):
    """``mpp_linear.linear`` / ``fused_linear`` on fp16 (``mpp_linear.py:145-294``): the tiled,
    skinny (n <= 64), split-K (127 rows) and tail-split (long K) forms, each epilogue."""
    r = _rng(m + n + k)
    x = _f16(r.standard_normal((m, k)) * 0.5)
    w = _f16(r.standard_normal((n, k)) * k ** -0.5)
    b = _f16(r.standard_normal(n) * 0.02)
    xd, wd, bd = _dev(x, device), _dev(w, device), _dev(b, device)
    # rows checked: all of a small product; of a large one every 13th and the last 300 (the tail
    # split's slices)
    rows = np.arange(m) if m <= 2048 else np.unique(np.r_[0:m:13, m - 300:m])
    x64, w64 = x[rows].astype(np.float64), w.astype(np.float64)
    ref = x64 @ w64.T + b
    # FP32 accumulation over k terms in another order: 16 fp32 ulps of the sum of |products|
    slack = 2.0 ** -20 * (np.abs(x64) @ np.abs(w64).T)
    kwargs = {}
    if epi == "gelu":
        kwargs = dict(activation="gelu_tanh")
        inner = np.clip(np.sqrt(2 / np.pi) * (ref + 0.044715 * ref ** 3), -10, 10)
        ref = 0.5 * ref * (1 + np.tanh(inner))
        slack = slack * 1.2 + 1e-6
    if epi.startswith("gated"):
        resid = r.standard_normal((m, n)).astype(F32)
        if epi == "gated_f16":
            resid = _f16(resid)
        gate = (r.standard_normal(n) * 0.5).astype(F32)
        rd = _dev(resid, device, torch.float32 if epi == "gated_f32" else H)
        kwargs = dict(residual=rd, gate=_dev(gate, device, torch.float32),
                      out_dtype=torch.float32 if epi == "gated_f32" else None)
        ref = resid[rows] + gate * ref
        slack = slack * np.abs(gate) + 1e-6
    got = mpp_linear.fused_linear(xd, wd, bd, **kwargs)
    if epi == "bias":
        assert mpp_linear.applies(xd, wd, bd, transposed=True)
        assert torch.equal(mpp_linear.linear(xd, wd, bd, transposed=True), got)
    assert got.dtype == (torch.float32 if epi == "gated_f32" else H)
    out = _np(got)[rows]
    # one fp16 rounding of the output (none for an fp32 output) plus the accumulation slack
    bound = slack + (2 * half_ulp_fp16(ref) if got.dtype == H else 0.0)
    assert np.all(np.abs(out - ref) <= bound), float(np.max(np.abs(out - ref) - bound))


def test_fp16_refuses_mixed_operands(device):
    x = torch.zeros((4, 64), dtype=H, device=device)
    w = torch.zeros((8, 64), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        mpp_linear.fused_linear(x, w)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        dense_attention.dense_attention(x, x.to(torch.bfloat16), x, heads=1)
    assert not dense_attention.applies(x[None], x.to(torch.bfloat16)[None], heads=1)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        fused_ops.rms_norm(x.float())


def _fp16_case(spec):
    p = workloads.ltx_params(spec, 0, dtype=H)
    inputs = workloads.ltx_inputs(spec, 0, dtype=H)
    pe = oracle.precompute_freqs_cis(inputs["positions"].numpy(), dim=spec.dim, theta=10000.0,
                                     max_pos=(20, 2048, 2048), use_middle_indices_grid=True,
                                     num_attention_heads=spec.heads)
    return p, oracle_params(p), inputs, pe


def _fp16_block(spec, p, inputs, pe, device, *, fp32=False):
    block = workloads.build_ltx_block(spec, p, device)
    x = inputs["x"].to(device)
    args = TransformerArgs(x=x.float() if fp32 else x, context=inputs["context"].to(device),
                           timesteps=p["timesteps"].to(device), positional_embeddings=device_tables(pe, device))
    out, _ = block(args)
    torch.cuda.synchronize()
    assert out.x.dtype == (torch.float32 if fp32 else H)
    return out.x[0].float().cpu().numpy()


def test_ltx_block_fp16_matches_oracle(device):
    """A D = 1024 LTX-2 block in fp16 (weights, activations, context, modulation rows) against
    the FP32 oracle: the literal north-star bar beyond the fp16 output rounding."""
    spec = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
    p, op, inputs, pe = _fp16_case(spec)
    got = _fp16_block(spec, p, inputs, pe, device)
    x, ctx = inputs["x"][0].float().numpy(), inputs["context"][0].float().numpy()
    ref = oracle.ltx_video_block(op, x, ctx, pe, heads=spec.heads)
    assert_block_parity(got, ref, "ltx fp16 d1024", half="fp16")
    got32 = _fp16_block(spec, p, inputs, pe, device, fp32=True)
    assert_block_parity(got32, ref, "  fp32 out", fp32_out=True, half="fp16")


def test_ltx_block_fp16_full_9216_tokens(device):
    """The config-3 shape (9216 + 256 tokens, D = 4096, 32 x 128) in fp16 against the FP32 torch
    evaluation: the D = 4096 block bar with fp16 roundings, anchored to the reference's fp16 graph."""
    spec = workloads.CONFIGS[3]
    p, op, inputs, pe = _fp16_case(spec)
    got = _fp16_block(spec, p, inputs, pe, device)
    tp = {k: torch.from_numpy(np.asarray(v)).to(device) for k, v in dense_params(op).items()}
    pe_d = tuple(torch.from_numpy(t).to(device) for t in pe)
    x, ctx = inputs["x"][0].float().to(device), inputs["context"][0].float().to(device)
    torch.backends.cuda.matmul.allow_tf32 = False
    evals = {}
    with torch.no_grad():
        for mode in (None, "kx", "graph"):
            evals[mode] = _torch_ref.ltx_video_block(tp, x, ctx, pe_d, heads=spec.heads, rounding_mode=mode,
                                                     half=H).cpu().numpy()
    del tp
    torch.cuda.empty_cache()
    assert_block_parity(got, evals[None], "config3 fp16 full block", ref_kx=evals["kx"], graph=evals["graph"],
                        small=False, half="fp16")
