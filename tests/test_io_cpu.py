"""Checkpoint I/O on the CPU: the safetensors header contract and the LTX-2 source-key mapping.

Known answers from the reference's tests (``tests/models/ltx2/weights/test_schema_keys_layout.py:
17-54``); header checks against files written by the independent ``safetensors`` package and
against hand-made broken files.
"""

import json
import struct

import pytest
import torch
from safetensors.torch import save_file

from kinomlx_amd.io import inspect_safetensors, read_dtypes, read_header, read_metadata
from kinomlx_amd.ltx2.weights import checkpoint_bindings, convert_checkpoint_key


def _key(k, **kw):
    c = convert_checkpoint_key(k, **kw)
    return None if c is None else c.target_key


def test_key_conversion_known_answers():
    assert _key("transformer_blocks.0.attn1.to_out.0.weight") == "transformer_blocks.0.attn1.to_out.weight"
    assert _key("transformer_blocks.1.ff.net.0.proj.weight") == "transformer_blocks.1.ff.project_in.proj.weight"
    assert _key("transformer_blocks.1.ff.net.2.bias") == "transformer_blocks.1.ff.project_out.bias"
    audio = "transformer_blocks.2.audio_ff.net.2.weight"
    assert _key(audio) is None
    assert _key(audio, include_audio=True) == "transformer_blocks.2.audio_ff.project_out.weight"
    assert _key("model.diffusion_model.transformer_blocks.0.ff.net.2.weight") == "transformer_blocks.0.ff.project_out.weight"
    assert _key("vae.decoder.weight") is None
    generic = "embeddings_connector.transformer_1d_blocks.0.attn1.to_q.weight"
    assert _key(f"model.diffusion_model.{generic}", include_audio=True) is None
    assert _key("video_embeddings_connector.transformer_1d_blocks.0.attn1.to_q.weight", include_audio=True) is None


def test_key_priorities():
    assert convert_checkpoint_key("model.diffusion_model.proj_out.weight").priority == 0
    assert convert_checkpoint_key("diffusion_model.proj_out.weight").priority == 1
    assert convert_checkpoint_key("proj_out.weight").priority == 2
    assert convert_checkpoint_key("wrapper.model.diffusion_model.proj_out.weight").priority == 3
    assert convert_checkpoint_key("wrapper.diffusion_model.proj_out.weight").priority == 4
    c = convert_checkpoint_key("net.proj_out.weight")
    assert (c.target_key, c.priority) == ("proj_out.weight", 6)
    assert convert_checkpoint_key("av_ca_a2v_gate_adaln_single.linear.weight") is None


def test_header_inventory_of_an_independently_written_file(tmp_path):
    path = tmp_path / "w.safetensors"
    tensors = {
        "b": torch.arange(6, dtype=torch.float32).reshape(2, 3),
        "a": torch.ones(4, dtype=torch.bfloat16),
        "c": torch.zeros((0, 5), dtype=torch.int32),
        "d": torch.tensor([True, False]),
        "e": torch.arange(3, dtype=torch.uint8),
    }
    save_file(tensors, str(path), metadata={"format": "pt", "note": "x"})
    inv = inspect_safetensors(path)
    assert inv.tensor_names == ("a", "b", "c", "d", "e")
    by = {t.name: t for t in inv.tensors}
    assert by["b"].shape == (2, 3) and by["b"].dtype == "F32" and by["b"].byte_count == 24
    assert by["c"].element_count == 0 and by["c"].byte_count == 0
    assert read_dtypes(path) == {"a": "BF16", "b": "F32", "c": "I32", "d": "BOOL", "e": "U8"}
    assert read_metadata(path) == {"format": "pt", "note": "x"}
    assert inv.payload_bytes == sum(t.byte_count for t in inv.tensors)


def _write(path, header, payload=b"", length=None):
    raw = json.dumps(header).encode() if not isinstance(header, bytes) else header
    n = len(raw) if length is None else length
    path.write_bytes(struct.pack("<Q", n) + raw + payload)
    return path


@pytest.mark.parametrize("case,message", [
    ("prefix", "truncated safetensors length prefix"),
    ("limit", "safety limit"),
    ("declared", "declared length exceeds file size"),
    ("json", "invalid safetensors header"),
    ("array", "must be an object"),
])
def test_header_errors(tmp_path, case, message):
    path = tmp_path / "bad.safetensors"
    if case == "prefix":
        path.write_bytes(b"\x01\x02\x03")
    elif case == "limit":
        _write(path, {}, length=200_000_000)
    elif case == "declared":
        _write(path, {}, length=50)
    elif case == "json":
        _write(path, b"{not json")
    else:
        _write(path, [1, 2])
    with pytest.raises(ValueError, match=message):
        read_header(path)


@pytest.mark.parametrize("entry,payload,message", [
    ({"x": {"dtype": "Q7", "shape": [1], "data_offsets": [0, 1]}}, b"\0", "unsupported dtype"),
    ({"x": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}, b"\0", "invalid shape"),
    ({"x": {"dtype": "U8", "shape": [True], "data_offsets": [0, 1]}}, b"\0", "invalid shape"),
    ({"x": {"dtype": "U8", "shape": [1], "data_offsets": [0]}}, b"\0", "invalid data offsets"),
    ({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 2]}}, b"\0\0", "invalid payload span"),
    ({"x": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]},
      "y": {"dtype": "U8", "shape": [2], "data_offsets": [1, 3]}}, b"\0\0\0", "overlaps"),
    ({"x": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}, b"\0\0", "leaves a gap"),
    ({"x": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}, b"\0\0", "unclaimed trailing bytes"),
    ({"__metadata__": {"a": 1}}, b"", "only strings"),
    ({"x": [1]}, b"", "invalid safetensors tensor entry"),
])
def test_inventory_errors(tmp_path, entry, payload, message):
    path = _write(tmp_path / "bad.safetensors", entry, payload)
    with pytest.raises(ValueError, match=message):
        inspect_safetensors(path)


def test_bindings_prefer_the_diffusion_prefix_and_skip_foreign_keys(tmp_path):
    path = tmp_path / "ckpt.safetensors"
    save_file({
        "model.diffusion_model.proj_out.weight": torch.ones(2, 2),
        "proj_out.weight": torch.zeros(2, 2),
        "model.diffusion_model.transformer_blocks.0.attn1.to_out.0.weight": torch.ones(2, 2),
        "model.diffusion_model.transformer_blocks.0.audio_attn1.to_q.weight": torch.ones(2, 2),
        "vae.decoder.conv.weight": torch.ones(1),
    }, str(path))
    assert checkpoint_bindings(path) == {
        "proj_out.weight": "model.diffusion_model.proj_out.weight",
        "transformer_blocks.0.attn1.to_out.weight": "model.diffusion_model.transformer_blocks.0.attn1.to_out.0.weight",
    }
    tie = tmp_path / "tie.safetensors"
    save_file({"a.proj_out.weight": torch.ones(1), "b.proj_out.weight": torch.ones(1)}, str(tie))
    with pytest.raises(ValueError, match="both map to"):
        checkpoint_bindings(tie)
