"""Safetensors checkpoints straight into HBM.

Mirror of the reading side of ``kinomlx/io/safetensors.py`` (``read_header`` ``:92-119``,
``read_dtypes`` ``:122-129``, ``inspect_safetensors`` ``:132-204``, ``SafetensorsTensor``,
``SafetensorsInventory``): the same header contract and validation (length prefix, 100 MB
header cap, JSON object, string-only metadata, known dtypes, shapes, exact and gap-free payload
spans). Loading is MI355X-side: the payload is memory-mapped and streamed through two pinned
host buffers whose copies into device memory run asynchronously on a side stream, so reading
the file overlaps the PCIe transfers; tensors land in HBM in their stored dtype.
"""

from __future__ import annotations

import json
import math
import struct
from collections.abc import Iterable
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

DTYPES: dict[str, tuple[torch.dtype, int]] = {
    "BOOL": (torch.bool, 1),
    "F8_E4M3": (torch.float8_e4m3fn, 1),
    "F8_E5M2": (torch.float8_e5m2, 1),
    "I8": (torch.int8, 1),
    "U8": (torch.uint8, 1),
    "BF16": (torch.bfloat16, 2),
    "F16": (torch.float16, 2),
    "I16": (torch.int16, 2),
    "U16": (torch.uint16, 2),
    "F32": (torch.float32, 4),
    "I32": (torch.int32, 4),
    "U32": (torch.uint32, 4),
    "F64": (torch.float64, 8),
    "I64": (torch.int64, 8),
    "U64": (torch.uint64, 8),
}
MAX_HEADER_BYTES = 100_000_000
STAGING_BYTES = 64 << 20


@dataclass(frozen=True)
class SafetensorsTensor:
    """One validated tensor descriptor: payload-relative byte span ``data_offsets``."""

    name: str
    dtype: str
    shape: tuple[int, ...]
    data_offsets: tuple[int, int]

    @property
    def element_count(self) -> int:
        return math.prod(self.shape)

    @property
    def byte_count(self) -> int:
        return self.data_offsets[1] - self.data_offsets[0]


@dataclass(frozen=True)
class SafetensorsInventory:
    """Header-only inventory; ``tensors`` sorted by name."""

    path: Path
    tensors: tuple[SafetensorsTensor, ...]
    metadata: tuple[tuple[str, str], ...]
    header_bytes: int
    payload_bytes: int

    @property
    def tensor_names(self) -> tuple[str, ...]:
        return tuple(t.name for t in self.tensors)


def _header_length(path: Path, stream, file_size: int) -> int:
    prefix = stream.read(8)
    if len(prefix) != 8:
        raise ValueError(f"{path}: truncated safetensors length prefix")
    length = struct.unpack("<Q", prefix)[0]
    if length > MAX_HEADER_BYTES:
        raise ValueError(f"{path}: safetensors header exceeds the {MAX_HEADER_BYTES}-byte safety limit")
    if length > file_size - 8:
        raise ValueError(f"{path}: truncated safetensors header (declared length exceeds file size)")
    return length


def read_header(path: Path | str) -> dict:
    """The JSON header as a dict, without reading tensor data."""
    path = Path(path)
    with path.open("rb") as stream:
        stream.seek(0, 2)
        file_size = stream.tell()
        stream.seek(0)
        length = _header_length(path, stream, file_size)
        raw = stream.read(length)
    if len(raw) != length:
        raise ValueError(f"{path}: truncated safetensors header")
    try:
        header = json.loads(raw.decode("utf-8"))
    except (UnicodeDecodeError, ValueError, RecursionError) as exc:
        raise ValueError(f"{path}: invalid safetensors header") from exc
    if not isinstance(header, dict):
        raise ValueError(f"{path}: safetensors header must be an object")
    return header


def read_dtypes(path: Path | str) -> dict[str, str]:
    """Tensor name -> stored dtype name."""
    return {name: str(entry["dtype"]) for name, entry in read_header(path).items()
            if name != "__metadata__" and isinstance(entry, dict) and "dtype" in entry}


def _int_list(value, length: int | None = None) -> bool:
    return (isinstance(value, list) and (length is None or len(value) == length)
            and all(isinstance(v, int) and not isinstance(v, bool) for v in value))


def inspect_safetensors(path: Path | str) -> SafetensorsInventory:
    """Validate every descriptor and the payload layout (spans exact, ordered, gap-free)."""
    source = Path(path).expanduser().resolve()
    header = read_header(source)
    file_size = source.stat().st_size
    with source.open("rb") as stream:
        header_bytes = _header_length(source, stream, file_size)
    payload_bytes = file_size - 8 - header_bytes

    meta = header.get("__metadata__")
    if meta is None:
        metadata: tuple[tuple[str, str], ...] = ()
    elif isinstance(meta, dict) and all(isinstance(k, str) and isinstance(v, str) for k, v in meta.items()):
        metadata = tuple(sorted(meta.items()))
    else:
        raise ValueError(f"{source}: safetensors metadata must contain only strings")

    tensors = []
    for name, entry in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(entry, dict):
            raise ValueError(f"{source}: invalid safetensors tensor entry {name!r}")
        dtype, shape, offsets = entry.get("dtype"), entry.get("shape"), entry.get("data_offsets")
        if not isinstance(dtype, str) or dtype not in DTYPES:
            raise ValueError(f"{source}: tensor {name!r} has unsupported dtype {dtype!r}")
        if not _int_list(shape) or any(v < 0 for v in shape):
            raise ValueError(f"{source}: tensor {name!r} has an invalid shape")
        if not _int_list(offsets, 2):
            raise ValueError(f"{source}: tensor {name!r} has invalid data offsets")
        start, end = offsets
        if start < 0 or end < start or end > payload_bytes or end - start != math.prod(shape) * DTYPES[dtype][1]:
            raise ValueError(f"{source}: tensor {name!r} has an invalid payload span")
        tensors.append(SafetensorsTensor(name, dtype, tuple(shape), (start, end)))
    cursor = 0
    for t in sorted(tensors, key=lambda t: (t.data_offsets, t.name)):
        start, end = t.data_offsets
        if start != cursor:
            relation = "overlaps" if start < cursor else "leaves a gap before"
            raise ValueError(f"{source}: tensor payload {t.name!r} {relation} byte {cursor}")
        cursor = end
    if cursor != payload_bytes:
        raise ValueError(f"{source}: safetensors payload has unclaimed trailing bytes")
    return SafetensorsInventory(source, tuple(sorted(tensors, key=lambda t: t.name)), metadata,
                                header_bytes, payload_bytes)


def read_metadata(path: Path | str) -> dict[str, str]:
    """The string-to-string ``__metadata__`` map."""
    return dict(inspect_safetensors(path).metadata)


def load_to_device(path: Path | str, device, names: Iterable[str] | None = None) -> dict[str, torch.Tensor]:
    """Tensors of ``path`` (all, or ``names``) as device tensors in their stored dtype.

    The file is memory-mapped; bytes move in 64 MiB chunks through two pinned buffers, each chunk
    copied to the device asynchronously on a side stream while the next one is read from the map.
    Returns once every copy has completed."""
    inventory = inspect_safetensors(path)
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("load_to_device loads into GPU memory")
    wanted = None if names is None else set(names)
    if wanted is not None:
        missing = wanted - set(inventory.tensor_names)
        if missing:
            raise KeyError(f"{inventory.path}: no tensors named {sorted(missing)}")
    chosen = [t for t in inventory.tensors if wanted is None or t.name in wanted]
    base = 8 + inventory.header_bytes
    mapped = np.memmap(inventory.path, dtype=np.uint8, mode="r") if chosen else None
    staging = [torch.empty(STAGING_BYTES, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    done = [None, None]
    stream = torch.cuda.Stream(device=device)
    # the destination buffers come from the caching allocator on the current stream: memory it
    # hands back may still be in use by work queued there, so the copy stream waits for it
    stream.wait_stream(torch.cuda.current_stream(device))
    out: dict[str, torch.Tensor] = {}
    which = 0
    for t in sorted(chosen, key=lambda t: t.data_offsets):
        dtype, _ = DTYPES[t.dtype]
        raw = torch.empty(t.byte_count, dtype=torch.uint8, device=device)
        raw.record_stream(stream)
        for offset in range(0, t.byte_count, STAGING_BYTES):
            size = min(STAGING_BYTES, t.byte_count - offset)
            if done[which] is not None:
                done[which].synchronize()
            begin = base + t.data_offsets[0] + offset
            staging[which][:size].numpy()[:] = mapped[begin:begin + size]
            with torch.cuda.stream(stream):
                raw[offset:offset + size].copy_(staging[which][:size], non_blocking=True)
                done[which] = torch.cuda.Event()
                done[which].record(stream)
            which ^= 1
        out[t.name] = raw.view(dtype).view(t.shape) if t.byte_count else torch.empty(t.shape, dtype=dtype,
                                                                                       device=device)
    # the tensors are used on the current stream: it waits for the last copies
    torch.cuda.current_stream(device).wait_stream(stream)
    stream.synchronize()
    return out


__all__ = [
    "DTYPES",
    "SafetensorsInventory",
    "SafetensorsTensor",
    "inspect_safetensors",
    "load_to_device",
    "read_dtypes",
    "read_header",
    "read_metadata",
]
