"""Checkpoint I/O (mirror of the reading side of ``kinomlx/io``)."""

from .safetensors import (
    SafetensorsInventory,
    SafetensorsTensor,
    inspect_safetensors,
    load_to_device,
    read_dtypes,
    read_header,
    read_metadata,
)

__all__ = [
    "SafetensorsInventory",
    "SafetensorsTensor",
    "inspect_safetensors",
    "load_to_device",
    "read_dtypes",
    "read_header",
    "read_metadata",
]
