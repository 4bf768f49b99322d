"""Shared helpers for block-level tests: workload parameters as oracle / torch-reference dicts."""

import numpy as np
import torch

import oracle
from kinomlx_amd import workloads


def oracle_params(p: dict) -> dict:
    """Workload parameter dict (CPU torch) -> the oracle's float32 numpy dict."""
    out = {}
    for name, value in p.items():
        if name in ("timesteps", "scale_shift_table", "prompt_scale_shift_table"):
            continue
        if name.endswith(".wq"):
            out[name] = value.numpy().view(np.uint32)
        elif name.endswith((".group_size", ".bits")):
            out[name] = int(value)
        else:
            out[name] = value.float().numpy()
    if "scale_shift_table" in p:
        out["ada"] = (p["scale_shift_table"].float() + p["timesteps"].float()[0, 0]).numpy()
        out["prompt"] = p["prompt_scale_shift_table"].float().numpy()
    return out


def ltx_case(spec, seed=0):
    """(params, oracle params, inputs, oracle RoPE tables (numpy, head-major))."""
    p = workloads.ltx_params(spec, seed)
    if spec.bits:
        p = workloads.quantize_ltx_params(p, spec.bits, spec.group_size)
    inputs = workloads.ltx_inputs(spec, seed)
    pe = oracle.precompute_freqs_cis(inputs["positions"].numpy(), dim=spec.dim, theta=10000.0,
                                     max_pos=(20, 2048, 2048), use_middle_indices_grid=True,
                                     num_attention_heads=spec.heads)
    return p, oracle_params(p), inputs, pe


def device_tables(pe, device):
    """Oracle head-major tables -> token-major device storage viewed head-major."""
    cos, sin = pe
    cos_d = torch.from_numpy(np.ascontiguousarray(cos.transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    sin_d = torch.from_numpy(np.ascontiguousarray(sin.transpose(0, 2, 1, 3))).to(device).transpose(1, 2)
    return cos_d, sin_d


def flux_case(spec, seed=0):
    """(params, oracle double-block params, oracle single-block params, inputs, (cos, sin) numpy
    ``(T, Dh)`` tables) for a FLUX.2 / config-1 spec."""
    p = workloads.flux_params(spec, seed)
    inputs = workloads.flux_inputs(spec, seed)
    cos, sin = workloads.flux_rope(spec)
    op = {k: v.float().numpy() for k, v in p.items()}
    single = {k[len("single."):]: v for k, v in op.items() if k.startswith("single.")}
    return p, op, single, inputs, (cos.numpy(), sin.numpy())


def krea_case(hidden, heads, kv_heads, tokens, ff_hidden, seed=0, batch=1):
    """Seeded Krea 2 block: (device-agnostic CPU params, oracle params, x (B, T, D) bf16,
    time_modulation (B, 6D) bf16, position ids (B, T, 3))."""
    dh = hidden // heads
    p = {}
    for name, rows in (("to_q", hidden), ("to_k", kv_heads * dh), ("to_v", kv_heads * dh), ("to_gate", hidden),
                       ("to_out", hidden)):
        p[f"attn.{name}.weight"] = workloads.bf16(workloads.normal(seed, f"krea.attn.{name}", (rows, hidden), 0.02))
    for name in ("norm_q", "norm_k"):
        p[f"attn.{name}.weight"] = workloads.normal(seed, f"krea.attn.{name}", (dh,), 0.1)
    for name in ("norm1", "norm2"):
        p[f"{name}.weight"] = workloads.normal(seed, f"krea.{name}", (hidden,), 0.1)
    p["ff.gate.weight"] = workloads.bf16(workloads.normal(seed, "krea.ff.gate", (ff_hidden, hidden), 0.02))
    p["ff.up.weight"] = workloads.bf16(workloads.normal(seed, "krea.ff.up", (ff_hidden, hidden), 0.02))
    p["ff.down.weight"] = workloads.bf16(workloads.normal(seed, "krea.ff.down", (hidden, ff_hidden), 0.02))
    p["scale_shift_table"] = workloads.normal(seed, "krea.table", (6, hidden), 0.1)
    x = workloads.bf16(workloads.normal(seed, "krea.x", (batch, tokens, hidden)))
    tmod = workloads.bf16(workloads.normal(seed, "krea.tmod", (batch, 6 * hidden), 0.3))
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, 40, (batch, tokens, 3), generator=g).float()
    op = {k: v.float().numpy() for k, v in p.items()}
    return p, op, x, tmod, ids


def build_krea_block(p, hidden, heads, kv_heads, device, *, fuse=True):
    from kinomlx_amd.krea2.transformer import Krea2BlockConfig, Krea2TransformerBlock
    from kinomlx_amd.ltx2.attention import Linear

    cfg = Krea2BlockConfig(attention_head_dim=hidden // heads, num_attention_heads=heads,
                           num_key_value_heads=kv_heads)
    block = Krea2TransformerBlock(cfg)
    for name in ("to_q", "to_k", "to_v", "to_gate", "to_out"):
        setattr(block.attn, name, Linear(p[f"attn.{name}.weight"].to(device)))
    block.attn.norm_q.weight = p["attn.norm_q.weight"].to(device)
    block.attn.norm_k.weight = p["attn.norm_k.weight"].to(device)
    block.norm1.weight = p["norm1.weight"].to(device)
    block.norm2.weight = p["norm2.weight"].to(device)
    for name in ("gate", "up", "down"):
        setattr(block.ff, name, Linear(p[f"ff.{name}.weight"].to(device)))
    block.scale_shift_table = p["scale_shift_table"].to(device)
    if fuse:
        block.fuse_projections()
    return block


def dense_params(op: dict) -> dict:
    """Oracle parameters with every affine-quantized layer replaced by its dequantized weight
    (``name.weight`` = the oracle's bit-exact ``bf16(scale * q + bias)`` as float32), the operand
    the quantized GEMM multiplies; for the FP32 torch evaluation of quantized blocks."""
    out = {}
    for name, value in op.items():
        if name.endswith((".scales", ".biases", ".group_size", ".bits")):
            continue
        if name.endswith(".wq"):
            base = name[:-len(".wq")]
            out[f"{base}.weight"] = oracle.dequantize_affine(
                value, op[f"{base}.scales"], op[f"{base}.biases"], group_size=int(op[f"{base}.group_size"]),
                bits=int(op[f"{base}.bits"]))
        else:
            out[name] = value
    return out
