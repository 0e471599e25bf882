"""Device and stream plumbing for the native calls on the per-step paths.

Each decode step makes a few native calls per layer, and at small batches
their host cost bounds the step: ``torch.cuda.current_stream(device)``
builds a Python stream object on every call, and ``torch.cuda.device(...)``
switches the current device even when it is already current.  These helpers
give the same answers without that work.
"""

from __future__ import annotations

import contextlib

import torch

_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
# the current device's index without torch.cuda.current_device()'s Python
# wrapper (the C++ side initialises the runtime itself when it has to)
_current = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device
_NULL = contextlib.nullcontext()


def device_index(device) -> int:
    """The index of ``device``: a torch.device (no index: the current
    device) or an int, which is returned as it is."""
    if isinstance(device, int):
        return device
    return device.index if device.index is not None else _current()


def stream_handle(device) -> int:
    """The HIP stream handle of ``device``'s current stream (the stream
    ``torch.cuda.current_stream(device)`` names)."""
    if _raw_stream is not None:
        return _raw_stream(device_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device):
    """A context in which ``device`` (a torch.device or an index) is the
    current device: no switch when it already is."""
    idx = device_index(device)
    if _current() == idx:
        return _NULL
    return torch.cuda.device(idx)
