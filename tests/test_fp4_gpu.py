"""mxfp4 / nvfp4 quantized linears on the GPU (the reference's feed-forward modes,
``video_ff_quantize_specs``, ``kinomlx/models/ltx2/settings.py:39``; defaults
``kinomlx/models/ltx2/weights/tensors.py:190-195``): the dequantization kernel bit-exact against the
oracle's E2M1 x scale closed form for every code under every scale byte, the quantize-on-load kernel
bit-identical to the oracle's quantizer and to the host packing, the layer against the oracle's
linear on the exactly dequantized weight, and an LTX-2 transformer loaded with FP4 feed-forward
layers."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.kernels import mpp_linear, quantized
from kinomlx_amd.ltx2.weights import load_transformer
from kinomlx_amd.ltx2.wrappers import Modality
from tests.conftest import cosine, rel_l2

pytestmark = pytest.mark.gpu

F32 = np.float32
MODES = {"mxfp4": 32, "nvfp4": 16}


def _np(t):
    return t.float().cpu().numpy()


def _words(w, device):
    return torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).to(device)


@pytest.mark.parametrize("mode", list(MODES))
def test_fp4_dequant_is_exact_for_every_code_and_scale(device, mode):
    """Row i holds all 16 codes (twice per 32) under scale byte i: E8M0 bytes 100..154 (mxfp4), every
    finite positive E4M3 byte 0..126 (nvfp4), against the oracle's exact decode."""
    group = MODES[mode]
    sbytes = np.arange(100, 155, dtype=np.uint8) if mode == "mxfp4" else np.arange(0, 127, dtype=np.uint8)
    n, k = sbytes.size, 64
    codes = np.tile(np.arange(16, dtype=np.int64), (n, k // 16))
    words = oracle.pack_nibbles(codes)
    scales = np.repeat(sbytes[:, None], k // group, 1)
    got = quantized.dequantize_fp4(_words(words, device), torch.from_numpy(scales).to(device), mode)
    assert got.dtype == torch.bfloat16 and got.shape == (n, k)
    assert np.array_equal(_np(got), oracle.dequantize_fp4(words, scales, mode=mode))


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("shape", [(128, 1024), (3, 96), (1000, 4096)])
def test_gpu_fp4_quantizer_is_bit_identical_to_the_oracle(device, mode, shape):
    r = np.random.default_rng(shape[0] + len(mode))
    w = (r.standard_normal(shape) * np.exp2(r.integers(-10, 8, (shape[0], 1)))).astype(F32)
    w[0, :32] = 0.0  # zero groups
    w[-1, :16] = 0.75  # a constant group
    w[-1, 40] = 3e4  # the rest of its group flushes to zero codes
    w[-1, 70] = -1e-39  # a bf16 subnormal
    w = oracle.to_bf16(w)
    words, scales = quantized.quantize_fp4(torch.from_numpy(w).to(torch.bfloat16).to(device), mode)
    o_words, o_scales = (oracle.quantize_mxfp4 if mode == "mxfp4" else oracle.quantize_nvfp4)(w)
    assert np.array_equal(words.cpu().numpy().view(np.uint32), o_words)
    assert np.array_equal(scales.cpu().numpy(), o_scales)
    h_words, h_scales = quantized.quantize_fp4(torch.from_numpy(w).to(torch.bfloat16), mode)  # host packing
    assert torch.equal(words.cpu(), h_words) and torch.equal(scales.cpu(), h_scales)


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize(("m", "n", "k"), [(512, 512, 512), (1000, 132, 384), (9, 64, 256), (2048, 4096, 1024)])
@pytest.mark.parametrize("epilogue", ["bias", "gated_f32"])
def test_fp4_linear_matches_oracle(device, mode, m, n, k, epilogue):
    """``QuantizedLinear(mode=...)`` (exact dequantization, then the dense GEMM) and the functional
    ``quantized_matmul`` against the oracle's FP4 linear: the dense kernel's own bar on the exactly
    dequantized weight, and bit-identical to the dense kernel on that weight."""
    r = np.random.default_rng(m + n + k)
    x = oracle.to_bf16((r.standard_normal((m, k)) * 0.5).astype(F32))
    w = oracle.to_bf16((r.standard_normal((n, k)) * k ** -0.5).astype(F32))
    b = oracle.to_bf16((r.standard_normal(n) * 0.02).astype(F32))
    words, scales = (oracle.quantize_mxfp4 if mode == "mxfp4" else oracle.quantize_nvfp4)(w)
    xd = torch.from_numpy(x).to(device).to(torch.bfloat16)
    bd = torch.from_numpy(b).to(device).to(torch.bfloat16)
    layer = quantized.QuantizedLinear(_words(words, device), torch.from_numpy(scales).to(device), None, bd, mode=mode)
    assert (layer.group_size, layer.bits) == (MODES[mode], 4) and layer.in_features == k
    ref = oracle.fp4_linear(x, words, scales, b, mode=mode)
    kw = {}
    if epilogue == "gated_f32":
        resid = r.standard_normal((m, n)).astype(F32)
        gate = (r.standard_normal(n) * 0.5).astype(F32)
        kw = dict(residual=torch.from_numpy(resid).to(device), gate=torch.from_numpy(gate).to(device),
                  out_dtype=torch.float32)
        ref = resid + gate * ref
    got = layer(xd, **kw)
    functional = quantized.quantized_matmul(xd, layer.weight, layer.scales, None, group_size=MODES[mode], bits=4,
                                            mode=mode, bias=bd, **kw)
    dense = mpp_linear.fused_linear(xd, torch.from_numpy(oracle.dequantize_fp4(words, scales, mode=mode)).to(device)
                                    .to(torch.bfloat16), bd, **kw)
    assert torch.equal(got, dense) and torch.equal(functional, dense)
    out = _np(got)
    assert cosine(out, ref) > 0.99999 and rel_l2(out, ref) < 4e-3


SPEC = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
CHANNELS = 32


def _source_name(key: str) -> str:
    key = key.replace(".to_out.", ".to_out.0.").replace("ff.proj_in.", "ff.net.0.proj.")
    return "model.diffusion_model." + key.replace("ff.proj_out.", "ff.net.2.")


def _checkpoint(p, path):
    tensors = {}
    for index, block in enumerate(p["blocks"]):
        for name, value in block.items():
            tensors[_source_name(f"transformer_blocks.{index}.{name}")] = value.contiguous()
    for name, value in p.items():
        if name != "blocks":
            tensors[_source_name(name)] = value.contiguous()
    save_file(tensors, str(path))


def _velocity(model, inputs, device):
    sigma = torch.full((1,), 0.6, device=device)
    mod = Modality(latent=inputs["latent"].to(device), context=inputs["context"].to(device), timesteps=sigma,
                   sigma=sigma, positions=inputs["positions"].to(device))
    out, _ = model(mod)
    torch.cuda.synchronize()
    return out.cpu()


def test_transformer_with_fp4_feed_forward_layers(device, tmp_path):
    """``video_ff_quantize_specs`` routing FF layers to nvfp4 (project_out) and mxfp4 (project_in),
    quantized on load: the loaded layers are FP4 ``QuantizedLinear``s, and the model's velocity equals,
    bit for bit, the dense model on the oracle's exact dequantization of the same packed weights."""
    p = workloads.ltx_model_params(SPEC, 2, in_channels=CHANNELS, out_channels=CHANNELS)
    path = tmp_path / "ltx.safetensors"
    _checkpoint(p, path)
    specs = (("project_out", "nvfp4"), ("project_in", "mxfp4"))
    model = load_transformer(path, device, heads=SPEC.heads, head_dim=SPEC.head_dim, video_ff_quantize_specs=specs)
    up, down = model.transformer_blocks[1].ff.project_in.proj, model.transformer_blocks[1].ff.project_out
    assert isinstance(up, quantized.QuantizedLinear) and up.mode == "mxfp4"
    assert isinstance(down, quantized.QuantizedLinear) and down.mode == "nvfp4"
    blocks = []
    for block in p["blocks"]:
        q = dict(block)
        for name, mode in (("ff.proj_in", "mxfp4"), ("ff.proj_out", "nvfp4")):
            w = q[f"{name}.weight"].float().numpy()
            packed = (oracle.quantize_mxfp4 if mode == "mxfp4" else oracle.quantize_nvfp4)(oracle.to_bf16(w))
            q[f"{name}.weight"] = torch.from_numpy(oracle.dequantize_fp4(*packed, mode=mode)).to(torch.bfloat16)
        blocks.append(q)
    dense = workloads.build_ltx_model(SPEC, dict(p, blocks=blocks), device, in_channels=CHANNELS,
                                      out_channels=CHANNELS)
    inputs = workloads.ltx_model_inputs(SPEC, in_channels=CHANNELS)
    a, b = _velocity(model, inputs, device), _velocity(dense, inputs, device)
    assert torch.isfinite(a.float()).all() and torch.equal(a, b)
