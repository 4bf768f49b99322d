"""Stage-by-stage parity of the full-size LTX-2 block (benchmark configs 3 and 4, int4 and int8).

The block is run one kernel stage at a time, through the same calls the block makes, and the
chained stages are first checked bit-identical to the block's own output. Each stage's output is
then compared with its FP32 evaluation from the GPU's own inputs to that stage (the bf16 or FP32
tensors the previous kernel wrote), so every kernel is held to an elementwise bar at the full
9216-token shape without the upstream rounding noise that a whole-block comparison carries:

* a bf16 output: ``|got - ref| <= 2e-2 + ulp_bf16(ref) / 2`` (the north-star 2e-2 beyond the
  output's own rounding);
* an FP32 output (the residual stream the out-projection epilogues write): ``|got - ref| <= 2e-2``.

The FP32 evaluation follows the reference's arithmetic for each stage: the AdaLN
(``kinomlx/models/ltx2/transformer/transformer.py:16-23``), the projections as ``addmm``
(``kinomlx/kernels/mpp_linear.py:1-6``), ``2 * sigmoid`` gates and the full-width Q/K RMSNorm then
split RoPE (``kinomlx/models/ltx2/transformer/attention.py:291-371``, ``rope.py:18-61``), softmax
attention (``kinomlx/models/ltx2/kernels/dense_attention.py:87-153``), the gated residuals
(``transformer.py:26-30``), GELU-tanh (``kinomlx/kernels/fused_ops.py:27-35``). Quantized layers
are evaluated on the oracle's bit-exact dequantized weights (the operand the GPU multiplies).
"""

import dataclasses

import pytest
import torch

from kinomlx_amd import _lib, workloads
from kinomlx_amd.ltx2 import dense_attention
from kinomlx_amd.ltx2.attention import norm_rope, norm_rope_qk
from kinomlx_amd.ltx2.transformer import TransformerArgs, adaln, modulate
from tests import _torch_ref
from tests._blocks import dense_params, device_tables, ltx_case

pytestmark = pytest.mark.gpu

STAGE_ABS = 2e-2

CASES = {
    "config3": workloads.CONFIGS[3],
    "config4-int4": workloads.CONFIGS[4],
    "config4-int8": dataclasses.replace(workloads.CONFIGS[4], bits=8),
}


def _half_ulp_bf16(ref: torch.Tensor) -> torch.Tensor:
    """Half the bf16 spacing at |ref| (float64): 2^(floor(log2 |ref|) - 8)."""
    a = ref.abs().clamp_min(2.0 ** -126)
    _, e = torch.frexp(a)  # a = m * 2^e, m in [0.5, 1): floor(log2 a) = e - 1
    return torch.ldexp(torch.ones_like(a), (e - 9).to(torch.int32))


def _stage(report: list, name: str, got: torch.Tensor, ref: torch.Tensor) -> None:
    g = got.double().reshape(ref.shape)
    r = ref.double()
    d = (g - r).abs()
    bf16 = got.dtype == torch.bfloat16
    excess = d - _half_ulp_bf16(r) if bf16 else d
    row = {"stage": name, "dtype": "bf16" if bf16 else "fp32", "max_ref": float(r.abs().max()),
           "max_abs": float(d.max()), "excess": float(excess.max()),
           "rel_rms": float(d.square().mean().sqrt() / r.square().mean().sqrt().clamp_min(1e-300))}
    report.append(row)
    print(f"  {name:10s} {row['dtype']}  max|ref| {row['max_ref']:8.4g}  max|d| {row['max_abs']:.4g}  "
          f"excess {row['excess']:.4g}  rel-rms {row['rel_rms']:.3g}")


def _lin(w: dict, name: str, x: torch.Tensor) -> torch.Tensor:
    return _torch_ref._lin(w, name, x.float())


def _gated_heads(o: torch.Tensor, gate: torch.Tensor, heads: int) -> torch.Tensor:
    t, width = o.shape
    return (o.reshape(t, heads, width // heads) * gate.float()[:, :, None]).reshape(t, width)


@pytest.mark.parametrize("case", list(CASES))
def test_full_block_stages_meet_the_elementwise_bar(device, case):
    spec = CASES[case]
    print(f"\n{case}: building inputs", flush=True)
    p, op, inputs, pe = ltx_case(spec)
    block = workloads.build_ltx_block(spec, p, device)
    heads, dim, eps = spec.heads, spec.dim, block.norm_eps
    x = inputs["x"].to(device)
    context = inputs["context"].to(device)
    pe_d = device_tables(pe, device)
    a1, a2 = block.attn1, block.attn2
    assert a1._qkv is not None and a2._kv is not None

    # ---- the block, one kernel stage at a time (the calls BasicAVTransformerBlock makes) ----
    s = {}
    ada = _lib.table_add(block.scale_shift_table, p["timesteps"].to(device))
    s["n1"] = adaln(x, ada[:, :, 1], ada[:, :, 0], eps)
    s["g1"] = a1.to_gate_logits(s["n1"], activation="sigmoid2")
    s["qkv1"] = a1._qkv(s["n1"])
    s["q1"], s["k1"] = norm_rope_qk(s["qkv1"][..., :dim], s["qkv1"][..., dim:2 * dim], a1.q_norm, a1.k_norm,
                                    pe_d, heads)
    v1 = s["qkv1"][..., 2 * dim:]
    s["o1"] = dense_attention.batched_attention(s["q1"], s["k1"], v1, heads=heads, gate=s["g1"])
    s["x1"] = a1.to_out(s["o1"], residual=x, gate=ada[:, :, 2], out_dtype=torch.float32)
    prompt = _lib.table_add(block.prompt_scale_shift_table, None)
    s["qn"] = adaln(s["x1"], ada[:, :, 7], ada[:, :, 6], eps)
    s["ctx"] = modulate(context, prompt[:, :, 1], prompt[:, :, 0])
    s["g2"] = a2.to_gate_logits(s["qn"], activation="sigmoid2")
    s["q2raw"] = a2.to_q(s["qn"])
    s["kv2"] = a2._kv(s["ctx"])
    s["q2"] = norm_rope(s["q2raw"], a2.q_norm, None, heads)
    s["k2"] = norm_rope(s["kv2"][..., :dim], a2.k_norm, None, heads)
    s["o2"] = dense_attention.batched_attention(s["q2"], s["k2"], s["kv2"][..., dim:], heads=heads, gate=s["g2"])
    s["x2"] = a2.to_out(s["o2"], residual=s["x1"], gate=ada[:, :, 8], out_dtype=torch.float32)
    s["n3"] = adaln(s["x2"], ada[:, :, 4], ada[:, :, 3], eps)
    s["h"] = block.ff.project_in(s["n3"])
    s["y"] = block.ff.project_out(s["h"], residual=s["x2"], gate=ada[:, :, 5], out_dtype=x.dtype)

    out, _ = block(TransformerArgs(x=x, context=context, timesteps=p["timesteps"].to(device),
                                   positional_embeddings=pe_d))
    torch.cuda.synchronize()
    assert torch.equal(out.x, s["y"]), "the stage chain is not the block's own computation"
    del block, out
    s = {k: v[0] for k, v in s.items()}  # batch 1: (T, width)

    # ---- each stage in FP32 from the GPU's own inputs to it ----
    print(f"{case}: stages chained and equal to the block; FP32 evaluation", flush=True)
    w = {k: torch.from_numpy(v).to(device) for k, v in dense_params(op).items()}
    cos, sin = (t.float() for t in pe_d)
    ad = ada[0, 0].float()
    torch.backends.cuda.matmul.allow_tf32 = False
    report = []
    print(f"{case}: {spec.tokens} + {spec.text_tokens} tokens, D {dim}, bits {spec.bits}", flush=True)
    with torch.no_grad():
        xf = x[0].float()
        _stage(report, "n1", s["n1"], _torch_ref._rms(xf) * (1 + ad[1]) + ad[0])
        _stage(report, "g1", s["g1"], 2 * torch.sigmoid(_lin(w, "attn1.to_gate_logits", s["n1"])))
        qkv_ref = torch.cat([_lin(w, f"attn1.to_{n}", s["n1"]) for n in "qkv"], -1)
        _stage(report, "qkv1", s["qkv1"], qkv_ref)
        del qkv_ref
        qkv = s["qkv1"].float()
        for name, cols, nw in (("q1", slice(0, dim), "attn1.q_norm.weight"),
                               ("k1", slice(dim, 2 * dim), "attn1.k_norm.weight")):
            ref = _torch_ref._split_rope(_torch_ref._rms(qkv[:, cols], w[nw]), cos, sin)
            _stage(report, name, s[name], ref)
        ref = _gated_heads(_torch_ref._attention(s["q1"].float(), s["k1"].float(), qkv[:, 2 * dim:], heads),
                           s["g1"], heads)
        _stage(report, "o1", s["o1"], ref)
        del qkv
        _stage(report, "x1", s["x1"], xf + ad[2] * _lin(w, "attn1.to_out", s["o1"]))
        _stage(report, "qn", s["qn"], _torch_ref._rms(s["x1"].float()) * (1 + ad[7]) + ad[6])
        pr = prompt[0, 0].float()
        _stage(report, "ctx", s["ctx"], context[0].float() * (1 + pr[1]) + pr[0])
        _stage(report, "g2", s["g2"], 2 * torch.sigmoid(_lin(w, "attn2.to_gate_logits", s["qn"])))
        _stage(report, "q2raw", s["q2raw"], _lin(w, "attn2.to_q", s["qn"]))
        _stage(report, "kv2", s["kv2"], torch.cat([_lin(w, "attn2.to_k", s["ctx"]), _lin(w, "attn2.to_v", s["ctx"])], -1))
        _stage(report, "q2", s["q2"], _torch_ref._rms(s["q2raw"].float(), w["attn2.q_norm.weight"]))
        kv2 = s["kv2"].float()
        _stage(report, "k2", s["k2"], _torch_ref._rms(kv2[:, :dim], w["attn2.k_norm.weight"]))
        ref = _gated_heads(_torch_ref._attention(s["q2"].float(), s["k2"].float(), kv2[:, dim:], heads), s["g2"], heads)
        _stage(report, "o2", s["o2"], ref)
        _stage(report, "x2", s["x2"], s["x1"].float() + ad[8] * _lin(w, "attn2.to_out", s["o2"]))
        _stage(report, "n3", s["n3"], _torch_ref._rms(s["x2"].float()) * (1 + ad[4]) + ad[3])
        ref = torch.nn.functional.gelu(_lin(w, "ff.proj_in", s["n3"]), approximate="tanh")
        _stage(report, "h", s["h"], ref)
        del ref
        _stage(report, "y", s["y"], s["x2"].float() + ad[5] * _lin(w, "ff.proj_out", s["h"]))
    worst = max(report, key=lambda r: r["excess"])
    assert worst["excess"] <= STAGE_ABS, worst
    assert all(torch.isfinite(v).all() for v in s.values())
