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
