"""Checkpoints into HBM on the GPU: the staged safetensors loader, the quantize-on-load kernel and
a whole LTX-2 video transformer built from a reference-named checkpoint.

Bars: every loaded tensor is bit-identical to what was written; the quantize kernel is
bit-identical to the oracle's quantizer and to the host packing; a model loaded from the file
(bf16, or quantized on load) gives bit-identical velocities to the same model assembled from
the in-memory parameters; a prepared (``__quant__.``) mxfp8 checkpoint gives bit-identical
velocities to quantize-on-load.
"""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.io import load_to_device
from kinomlx_amd.io import safetensors as st
from kinomlx_amd.kernels import quantized
from kinomlx_amd.ltx2.weights import QUANTIZED_LINEARS, load_transformer
from kinomlx_amd.ltx2.wrappers import Modality
from tests.conftest import cosine, rel_l2

pytestmark = pytest.mark.gpu

SPEC = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=1024, heads=8, head_dim=128)
CHANNELS = 32


def test_load_to_device_round_trips_every_dtype(device, tmp_path, monkeypatch):
    monkeypatch.setattr(st, "STAGING_BYTES", 1 << 20)  # many chunks through both staging buffers
    g = torch.Generator().manual_seed(0)
    tensors = {
        "big_bf16": torch.randn((1536, 1100), generator=g).to(torch.bfloat16),  # 3.2 MiB
        "f32": torch.randn((7, 3), generator=g),
        "f16": torch.randn(5, generator=g).half(),
        "i32": torch.randint(-9, 9, (4, 4), generator=g, dtype=torch.int32),
        "i64": torch.arange(5, dtype=torch.int64),
        "u8": torch.arange(250, dtype=torch.uint8),
        "b": torch.tensor([True, False, True]),
        "empty": torch.zeros((0, 3)),
        "f8": torch.randn(16, generator=g).to(torch.float8_e4m3fn),
    }
    path = tmp_path / "all.safetensors"
    save_file(tensors, str(path))
    got = load_to_device(path, device)
    assert set(got) == set(tensors)
    for name, ref in tensors.items():
        out = got[name]
        assert out.device.type == "cuda" and out.dtype == ref.dtype and out.shape == ref.shape, name
        assert torch.equal(out.cpu().view(torch.uint8) if ref.numel() else out.cpu(),
                           ref.view(torch.uint8) if ref.numel() else ref), name
    subset = load_to_device(path, device, names=["u8"])
    assert list(subset) == ["u8"]
    with pytest.raises(KeyError):
        load_to_device(path, device, names=["nope"])


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("shape", [(96, 256), (1000, 4096), (3, 64)])
def test_quantize_kernel_is_bit_exact(device, bits, shape):
    w = workloads.bf16(workloads.normal(7, "qk", shape, 0.02))
    w[0, :64] = 0.5  # a constant group: scale 1, every code 0
    words, scales, biases = quantized.quantize(w.to(device), 64, bits)
    o_words, o_scales, o_biases = oracle.quantize_affine(w.float().numpy(), 64, bits)
    assert np.array_equal(words.cpu().numpy().view(np.uint32), o_words)
    assert np.array_equal(scales.float().cpu().numpy(), o_scales)
    assert np.array_equal(biases.float().cpu().numpy(), o_biases)
    h_words, h_scales, h_biases = quantized.quantize(w, 64, bits)  # host packing
    assert torch.equal(words.cpu(), h_words) and torch.equal(scales.cpu(), h_scales)
    assert torch.equal(biases.cpu(), h_biases)


def test_quantize_kernel_strided_rows(device):
    w = workloads.bf16(workloads.normal(8, "qs", (64, 512), 0.02)).to(device)
    view = w[:, :256]  # rows 512 apart
    words, scales, biases = quantized.quantize(view, 64, 4)
    ref = quantized.quantize(view.contiguous(), 64, 4)
    assert all(torch.equal(a, b) for a, b in zip((words, scales, biases), ref))


def _source_name(key: str) -> str:
    key = key.replace(".to_out.", ".to_out.0.").replace("ff.proj_in.", "ff.net.0.proj.")
    return "model.diffusion_model." + key.replace("ff.proj_out.", "ff.net.2.")


def _write_checkpoint(p, path):
    tensors = {}
    for index, block in enumerate(p["blocks"]):
        for name, value in block.items():
            tensors[_source_name(f"transformer_blocks.{index}.{name}")] = value.contiguous()
    for name, value in p.items():
        if name != "blocks":
            tensors[_source_name(name)] = value.contiguous()
    # keys the video transformer must skip
    tensors["model.diffusion_model.transformer_blocks.0.audio_attn1.to_q.weight"] = torch.zeros(4, 4)
    tensors["model.diffusion_model.audio_scale_shift_table"] = torch.zeros(9, 4)
    tensors["vae.decoder.conv_in.weight"] = torch.zeros(3)
    save_file(tensors, str(path))


def _velocity(model, inputs, device):
    sigma = torch.full((1,), 0.6, device=device)
    mod = Modality(latent=inputs["latent"].to(device), context=inputs["context"].to(device), timesteps=sigma,
                   sigma=sigma, positions=inputs["positions"].to(device))
    out, _ = model(mod)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("bits", [None, 4])
def test_model_from_checkpoint_matches_the_in_memory_model(device, tmp_path, bits):
    p = workloads.ltx_model_params(SPEC, 2, in_channels=CHANNELS, out_channels=CHANNELS)
    path = tmp_path / "ltx.safetensors"
    _write_checkpoint(p, path)
    loaded = load_transformer(path, device, heads=SPEC.heads, head_dim=SPEC.head_dim, quantize_bits=bits)
    assert loaded.num_blocks == 2 and loaded.in_channels == CHANNELS and loaded.out_channels == CHANNELS
    if bits:
        p = dict(p, blocks=[workloads.quantize_ltx_params(b, bits) for b in p["blocks"]])
    built = workloads.build_ltx_model(SPEC, p, device, in_channels=CHANNELS, out_channels=CHANNELS)
    inputs = workloads.ltx_model_inputs(SPEC, in_channels=CHANNELS)
    a, b = _velocity(loaded, inputs, device), _velocity(built, inputs, device)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


def test_pretransposed_adaln_linears_bind_like_plain_ones(device, tmp_path):
    """The reference's preparation may store every top-level AdaLN linear pretransposed, as
    ``__layout__.<name>.weight_t`` only (``kinomlx/models/ltx2/weights/layout.py:11-20``): the
    model must still be built with its prompt AdaLN, every tensor placed (strict), and give the
    plain checkpoint's velocities bit for bit."""
    p = workloads.ltx_model_params(SPEC, 1, in_channels=CHANNELS, out_channels=CHANNELS)
    plain_path, layout_path = tmp_path / "plain.safetensors", tmp_path / "layout.safetensors"
    _write_checkpoint(p, plain_path)
    tensors = {}
    for index, block in enumerate(p["blocks"]):
        for name, value in block.items():
            tensors[_source_name(f"transformer_blocks.{index}.{name}")] = value.contiguous()
    for name, value in p.items():
        if name == "blocks":
            continue
        if name in ("adaln_single.linear.weight", "prompt_adaln_single.linear.weight"):
            tensors[f"__layout__.{name}_t"] = value.t().contiguous()
        else:
            tensors[_source_name(name)] = value.contiguous()
    assert "__layout__.prompt_adaln_single.linear.weight_t" in tensors
    save_file(tensors, str(layout_path))
    plain = load_transformer(plain_path, device, heads=SPEC.heads, head_dim=SPEC.head_dim)
    layout = load_transformer(layout_path, device, heads=SPEC.heads, head_dim=SPEC.head_dim, strict=True)
    assert layout.prompt_adaln_single is not None and plain.prompt_adaln_single is not None
    inputs = workloads.ltx_model_inputs(SPEC, in_channels=CHANNELS)
    assert torch.equal(_velocity(layout, inputs, device), _velocity(plain, inputs, device))


def test_strict_loading_rejects_unplaced_tensors(device, tmp_path):
    p = workloads.ltx_model_params(SPEC, 1, in_channels=CHANNELS, out_channels=CHANNELS)
    path = tmp_path / "extra.safetensors"
    p["blocks"][0]["attn1.to_q.lora"] = torch.zeros(2)
    _write_checkpoint(p, path)
    with pytest.raises(ValueError, match="no place in the video model"):
        load_transformer(path, device, heads=SPEC.heads, head_dim=SPEC.head_dim)
    assert load_transformer(path, device, heads=SPEC.heads, head_dim=SPEC.head_dim, strict=False).num_blocks == 1


def _mlx_key(key: str) -> str:
    return key.replace("ff.proj_in.", "ff.project_in.proj.").replace("ff.proj_out.", "ff.project_out.")


def _write_prepared(p, path, *, pretransposed: bool):
    """A prepared checkpoint as ``preparation.py:139-157`` writes one: MLX keys, and every block
    linear's weight packed by mx.quantize(w or w.T, 32, 8, "mxfp8") under ``__quant__.``
    (uint32 words, uint8 scales; the bias stays a normal tensor)."""
    tensors = {}
    for index, block in enumerate(p["blocks"]):
        for name, value in block.items():
            key = _mlx_key(f"transformer_blocks.{index}.{name}")
            base = key[: -len(".weight")].split(".", 2)[2] if key.endswith(".weight") else None
            if base in QUANTIZED_LINEARS:
                words, scales = quantized.quantize_mxfp8(value.t().contiguous() if pretransposed else value)
                tensors[f"__quant__.{key[: -len('.weight')]}.weight"] = words.view(torch.uint32)
                tensors[f"__quant__.{key[: -len('.weight')]}.scales"] = scales
            else:
                tensors[key] = value.contiguous()
    for name, value in p.items():
        if name != "blocks":
            tensors[name] = value.contiguous()
    save_file(tensors, str(path))


# 32 heads, as the reference model has: the pretransposed packing groups the gate-logit projection's
# output axis (heads wide) by 32
MX_SPEC = workloads.LTXSpec(grid=(2, 4, 8), text_tokens=16, dim=2048, heads=32, head_dim=64)


@pytest.mark.parametrize("mode", ["mxfp8-blocks", "mxfp8-blocks-pretranspose"])
def test_prepared_mxfp8_checkpoint_matches_quantize_on_load(device, tmp_path, mode):
    """``transformer_quantize`` on a dense checkpoint (quantized on the device) and on a prepared
    one (``__quant__.`` tensors bound straight into the quantized layers) give bit-identical
    velocities; the pretransposed layers equal the dense model on their exactly dequantized
    weights, the in-mainloop mxfp8 GEMM differs from it only in fp32 summation order."""
    pre = mode.endswith("pretranspose")
    p = workloads.ltx_model_params(MX_SPEC, 2, in_channels=CHANNELS, out_channels=CHANNELS)
    dense_path, prepared_path = tmp_path / "dense.safetensors", tmp_path / "prepared.safetensors"
    _write_checkpoint(p, dense_path)
    _write_prepared(p, prepared_path, pretransposed=pre)
    kw = dict(heads=MX_SPEC.heads, head_dim=MX_SPEC.head_dim, transformer_quantize=mode)
    on_load = load_transformer(dense_path, device, **kw)
    prepared = load_transformer(prepared_path, device, **kw)
    layer = prepared.transformer_blocks[1].ff.project_out
    assert isinstance(layer, quantized.PretransposedQuantizedLinear if pre else quantized.QuantizedLinear)
    assert layer.mode == "mxfp8" and (layer.group_size, layer.bits) == (32, 8)
    inputs = workloads.ltx_model_inputs(MX_SPEC, in_channels=CHANNELS)
    a, b = _velocity(on_load, inputs, device), _velocity(prepared, inputs, device)
    assert torch.isfinite(a.float()).all() and torch.equal(a, b)

    # the model on the exact dequantization of every packed weight (oracle)
    blocks = []
    for block in p["blocks"]:
        q = dict(block)
        for name in workloads.QUANTIZED_LTX_LINEARS:
            w = q[f"{name}.weight"].float().numpy()
            if pre:
                deq = oracle.dequantize_mxfp8(*oracle.quantize_mxfp8(np.ascontiguousarray(w.T))).T
            else:
                deq = oracle.dequantize_mxfp8(*oracle.quantize_mxfp8(w))
            q[f"{name}.weight"] = torch.from_numpy(np.ascontiguousarray(deq)).to(torch.bfloat16)
        blocks.append(q)
    dense = workloads.build_ltx_model(MX_SPEC, dict(p, blocks=blocks), device, in_channels=CHANNELS, out_channels=CHANNELS)
    c = _velocity(dense, inputs, device)
    if pre:
        assert torch.equal(a, c)
    else:
        a32, c32 = a.float().numpy(), c.float().numpy()
        assert cosine(a32, c32) > 0.9999 and rel_l2(a32, c32) < 5e-3


def test_prepared_quant_tensors_need_a_mode(device, tmp_path):
    p = workloads.ltx_model_params(SPEC, 1, in_channels=CHANNELS, out_channels=CHANNELS)
    path = tmp_path / "prepared.safetensors"
    _write_prepared(p, path, pretransposed=False)
    with pytest.raises(ValueError, match="Missing quantization mode"):
        load_transformer(path, device, heads=SPEC.heads, head_dim=SPEC.head_dim)
