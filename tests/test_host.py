"""Host-side logic of the operator surface: contracts, error messages and routing predicates
that hold before any kernel runs, plus the product's CPU-side helpers (quantizer, RoPE tables,
workload FLOP counts) against the oracle. CPU only."""

import numpy as np
import pytest
import torch

import oracle
from kinomlx_amd import workloads
from kinomlx_amd.kernels import mpp_linear, quantized, split_rope
from kinomlx_amd.ltx2 import dense_attention, rope


def _zeros(tokens, width, dtype=torch.bfloat16):
    return torch.zeros((1, tokens, width), dtype=dtype)


def test_dense_attention_refuses_inputs_outside_the_contract():
    """Messages of kinomlx/models/ltx2/kernels/dense_attention.py:112-130 (test_dense_attention.py:86-99)."""
    q = torch.zeros(32, 256, dtype=torch.bfloat16)
    k = torch.zeros(20, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        dense_attention.dense_attention(q.float(), k.float(), k.float(), heads=2)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        dense_attention.dense_attention(q, k, k.float(), heads=2)
    with pytest.raises(ValueError, match="64 or 128"):
        dense_attention.dense_attention(q, k, k, heads=3)
    with pytest.raises(ValueError, match="64 or 128"):
        dense_attention.dense_attention(q, k, k, heads=8)
    with pytest.raises(ValueError, match="64 or 128"):
        dense_attention.dense_attention(q, k[:, :128], k[:, :128], heads=2)
    with pytest.raises(ValueError, match="64 or 128"):
        dense_attention.dense_attention(q, k, k[:-1], heads=2)


def test_dense_attention_applies_only_to_gpu_bf16_64_or_128_wide_heads():
    # CPU tensors never take the kernel
    assert not dense_attention.applies(_zeros(5, 256), _zeros(9, 256), heads=2)
    assert not dense_attention.applies(_zeros(5, 256, torch.float32), _zeros(5, 256, torch.float32), heads=2)
    assert not dense_attention.applies(_zeros(5, 96), _zeros(5, 96), heads=2)
    assert not dense_attention.applies(_zeros(0, 256), _zeros(5, 256), heads=2)
    assert dense_attention.HEAD_DIMS == (64, 128)


def test_split_rope_contract_on_the_host():
    value = torch.zeros(1, 13, 4 * 48, dtype=torch.bfloat16)
    cos = torch.zeros(1, 4, 13, 24)
    assert not split_rope.applies(value, cos, cos)  # CPU tensors
    assert not split_rope.applies(value, cos[:, :3], cos[:, :3])
    with pytest.raises(ValueError, match="does not apply"):
        split_rope.rotate(value, cos, cos)
    split_rope.set_enabled(False)
    try:
        assert not split_rope.enabled()
    finally:
        split_rope.set_enabled(True)
    with pytest.raises(ValueError, match="matching shapes"):
        rope.apply_split_rotary_emb(value, cos, cos[:, :, :5])


def test_linear_supports_and_applies():
    assert mpp_linear.supports(1056, 1024, 1040, transposed=True, dtype=torch.bfloat16)
    assert not mpp_linear.supports(10, 12, 16, transposed=True, dtype=torch.bfloat16)
    assert not mpp_linear.supports(10, 16, 16, transposed=True, dtype=torch.float32)
    w = torch.zeros(16, 32, dtype=torch.bfloat16)
    assert mpp_linear.prepare(w).peak is None
    assert mpp_linear.prepare(w.t(), transposed=False).values.shape == (16, 32)
    assert mpp_linear.restore(mpp_linear.prepare(w)) is not None
    assert not mpp_linear.applies(torch.zeros(4, 32, dtype=torch.bfloat16), w, None, transposed=True) or torch.cuda.is_available()


def test_quant_defaults_follow_the_reference():
    """``tests/models/ltx2/weights/test_storage_weights.py:207-213`` and the table of
    ``kinomlx/models/ltx2/weights/tensors.py:185-203``."""
    assert quantized.quant_defaults("mxfp8", None, None) == (32, 8)
    assert quantized.quant_defaults("affine", 128, 6) == (128, 6)
    assert quantized.quant_defaults("affine", None, None) == (64, 4)
    assert quantized.quant_defaults("mxfp4", None, None) == (32, 4)
    assert quantized.quant_defaults("nvfp4", None, None) == (16, 4)
    with pytest.raises(ValueError, match="must be positive"):
        quantized.quant_defaults("affine", 0, 4)
    with pytest.raises(ValueError, match="must be positive"):
        quantized.quant_defaults("affine", 64, 0)
    with pytest.raises(ValueError, match="Unsupported FF quantization mode"):
        quantized.quant_defaults("int3", None, None)
    # the FP4 modes take their own group size and width only
    quantized.QuantizedLinear(torch.zeros((32, 8), dtype=torch.int32), torch.zeros((32, 4), dtype=torch.uint8),
                              None, mode="nvfp4")
    with pytest.raises(ValueError, match="nvfp4 takes group size 16 and 4 bits"):
        quantized.QuantizedLinear(torch.zeros((32, 8), dtype=torch.int32), torch.zeros((32, 2), dtype=torch.uint8),
                                  None, group_size=32, mode="nvfp4")


def test_quant_routing_covers_whole_block_and_targeted_ff_modes():
    """``tests/models/ltx2/weights/test_storage_weights.py:175-206`` on the base-level routing
    (``kinomlx/models/ltx2/weights/quantization.py:199-218``)."""
    from kinomlx_amd.ltx2 import weights

    assert weights.quant_mode_for_base("attn1.to_q", transformer_quantize="mxfp8-blocks") == "mxfp8"
    assert weights.quant_mode_for_base("attn2.to_gate_logits", transformer_quantize="mxfp8-blocks-pretranspose") == "mxfp8"
    assert weights.quant_mode_for_base("ff.project_out", video_ff_quantize_specs=(("project_out", "nvfp4"),)) == "nvfp4"
    assert weights.quant_mode_for_base("ff.project_in.proj", video_ff_quantize_specs=(("project_out", "nvfp4"),)) is None
    assert weights.quant_mode_for_base("attn1.to_q") is None
    assert weights.quant_pretransposed("mxfp8-blocks-pretranspose") and not weights.quant_pretransposed("mxfp8-blocks")
    with pytest.raises(ValueError, match="Unsupported transformer weight quantization mode"):
        weights.quant_mode_for_base("attn1.to_q", transformer_quantize="fp8-blocks")


def test_host_mxfp8_quantizer_is_bit_identical_to_the_oracle():
    g = torch.Generator().manual_seed(4)
    w = (torch.randn((64, 256), generator=g) * torch.exp2(torch.randint(-9, 9, (64, 1), generator=g).float()))
    w = w.to(torch.bfloat16)
    w[3, :32] = 0  # a zero group: scale byte 0
    w[5, 7] = 1e30  # a group whose other elements underflow
    w[6, 1] = -3e-39  # a bf16 subnormal
    words, scales = quantized.quantize_mxfp8(w)
    o_words, o_scales = oracle.quantize_mxfp8(w.float().numpy())
    assert words.dtype == torch.int32 and scales.dtype == torch.uint8
    assert np.array_equal(words.numpy().view(np.uint32), o_words) and np.array_equal(scales.numpy(), o_scales)


@pytest.mark.parametrize("bits", [4, 8])
def test_product_quantizer_is_bit_identical_to_the_oracle(bits):
    w = workloads.normal(3, "q", (96, 256), 0.02).to(torch.bfloat16)
    words, scales, biases = quantized.quantize(w, 64, bits)
    o_words, o_scales, o_biases = oracle.quantize_affine(w.float().numpy(), 64, bits)
    assert np.array_equal(words.numpy().view(np.uint32), o_words)
    assert np.array_equal(scales.float().numpy(), o_scales)
    assert np.array_equal(biases.float().numpy(), o_biases)
    assert np.array_equal(quantized.unpack(words, bits).numpy(), oracle.unpack_affine(o_words, bits).astype(np.int64))


def test_product_rope_tables_take_gpu_tensors_only():
    """The tables come from a HIP kernel: CPU positions are refused, not computed on the host."""
    pos = workloads.ltx_positions((3, 4, 5))
    with pytest.raises(ValueError, match="GPU tensors"):
        rope.precompute_freqs_cis(pos, dim=1024, max_pos=(20, 2048, 2048), use_middle_indices_grid=True,
                                  num_attention_heads=8)


def test_workload_flops_match_baseline():
    f3 = workloads.flop_count(workloads.CONFIGS[3])
    assert f3["gemm"] / 1e9 == pytest.approx(4351.4, abs=0.2)
    assert f3["attention"] / 1e9 == pytest.approx(1430.2, abs=0.1)
    assert workloads.flop_count(workloads.CONFIGS[1])["total"] / 1e9 == pytest.approx(34.4, abs=0.1)
    assert workloads.flop_count(workloads.CONFIGS[2])["total"] / 1e9 == pytest.approx(4715.9, abs=0.2)
    f5 = workloads.flop_count(workloads.CONFIGS[5])
    assert f5["gemm"] / 1e9 == pytest.approx(12846.6, abs=0.2)
    assert workloads.CONFIGS[3].tokens == 9216 and workloads.CONFIGS[5].tokens == 27280


def test_tail_split_rule():
    from kinomlx_amd import _lib

    # 9216 x 4096: 576 tiles of 256x256, 2.25 rounds on 256 CUs -> two whole rounds over 8192 rows,
    # the 1024-row tail (64 tiles) as 4 K slices
    assert _lib.tail_split(9216, 4096, 16384) == (8192, 4)
    assert _lib.tail_split(4864, 4096, 8192) == (4096, 4)
    assert _lib.tail_split(4352, 4096, 8192) == (4096, 8)
    assert _lib.tail_split(9216, 4096, 4096) is None   # short K keeps the plain tiling
    assert _lib.tail_split(8192, 4096, 16384) is None  # already whole rounds
    assert _lib.tail_split(1024, 4096, 16384) is None  # under one round
    assert _lib.tail_split(9216, 4000, 16384) is None  # N not a whole number of 256-wide tiles
    # 27 280 rows: a 176-tile tail; 4 slices take 3 rounds of quarter tiles (0.75 of a round)
    assert _lib.tail_split(27280, 4096, 16384) == (24576, 4)
    for m, n, k in [(9216, 4096, 16384), (4864, 4096, 8192), (27280, 4096, 16384), (5376, 4096, 16384)]:
        rows, splits = _lib.tail_split(m, n, k)
        tail_tiles = -(-(m - rows) // 256) * (n // 256)
        assert rows % 256 == 0 and (rows // 256) * (n // 256) % 256 == 0
        assert k % (64 * splits) == 0 and k // splits >= 512
        assert tail_tiles * splits <= 256 or -(-tail_tiles * splits // 256) / splits < 1.0


def test_quantized_layers_refuse_scales_the_kernels_would_misread():
    """The kernels reinterpret the scale bits: affine layers take bf16 scales and biases, mxfp8
    layers uint8 E8M0 exponents; any other dtype is refused instead of read as the wrong bits."""
    words = torch.zeros((32, 8), dtype=torch.int32)
    good = torch.zeros((32, 1), dtype=torch.bfloat16)
    quantized.QuantizedLinear(words, good, good, group_size=64, bits=4)
    for scales, biases in ((good.half(), good), (good.float(), good), (good, good.half())):
        with pytest.raises(ValueError, match="bfloat16"):
            quantized.QuantizedLinear(words, scales, biases, group_size=64, bits=4)
    with pytest.raises(ValueError, match="uint8"):
        quantized.QuantizedLinear(words, torch.zeros((32, 1), dtype=torch.bfloat16), None, mode="mxfp8")


@pytest.mark.parametrize("mode", ["mxfp4", "nvfp4"])
def test_host_fp4_quantizer_is_bit_identical_to_the_oracle(mode):
    """The torch host packing of ``quantize_fp4`` (used for weights still in host memory) against
    the oracle's quantizer, on bf16 weights over a range of magnitudes with zero and constant groups."""
    import oracle

    r = np.random.default_rng(9)
    w = (r.standard_normal((48, 256)) * np.exp2(r.integers(-12, 6, (48, 1)))).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] = 0.75
    w[2, 7] = 1e4
    w = oracle.to_bf16(w)
    words, scales = quantized.quantize_fp4(torch.from_numpy(w).to(torch.bfloat16), mode)
    o_words, o_scales = (oracle.quantize_mxfp4 if mode == "mxfp4" else oracle.quantize_nvfp4)(w)
    assert np.array_equal(words.numpy().view(np.uint32), o_words)
    assert np.array_equal(scales.numpy(), o_scales)
