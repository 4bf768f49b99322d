"""The second HIP stream LTX-2's joint audio/video block runs its audio stream on: one per device,
default priority."""

from __future__ import annotations

import torch

_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}


def side_stream(device: torch.device) -> torch.cuda.Stream:
    """This device's side stream (created on first use, kept for the process)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _SIDE_STREAMS.get(index)
    if stream is None:
        stream = torch.cuda.Stream(device=index)
        _SIDE_STREAMS[index] = stream
    return stream
