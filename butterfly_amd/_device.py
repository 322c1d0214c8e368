"""Current-device and current-stream helpers for the native calls (cheap on the hot path)."""
from __future__ import annotations

import contextlib

import torch

_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", torch.cuda.current_device)


def stream_of(device) -> int:
    """Handle of the current stream of ``device`` (a torch.device, index or tensor)."""
    if isinstance(device, torch.Tensor):
        device = device.device
    idx = device.index if isinstance(device, torch.device) else device
    if idx is None:
        idx = _GET_DEVICE()
    if _RAW_STREAM is not None:
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(idx).cuda_stream


_NULL = contextlib.nullcontext()   # stateless, so one instance serves every call


def on(device):
    """Make ``device`` current for a native call; no switch when it already is."""
    idx = device.index if isinstance(device, torch.device) else torch.device(device).index
    if idx is None or idx == _GET_DEVICE():
        return _NULL
    return torch.cuda.device(idx)
