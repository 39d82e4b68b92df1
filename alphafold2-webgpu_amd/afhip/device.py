"""Device plumbing: opening the device, streams, tensor pointers, memory.

PyTorch provides device memory and the stream; every kernel is libafhip's.
"""
from __future__ import annotations

import json
import time

from . import _lib

_opened = None


def _torch():
    import torch  # deferred: CPU-only callers of the host logic need no torch

    return torch


def open_device(ordinal: int = 0) -> None:
    """afhip_open once per process (the counterpart of requestAlphaFoldDevice)."""
    global _opened
    torch = _torch()
    if not torch.cuda.is_available():
        raise _lib.AfhipUnavailable("no HIP device is visible; afhip has no CPU fallback")
    if _opened == ordinal:
        return
    torch.cuda.set_device(ordinal)
    _lib.call("afhip_open", ordinal)
    _opened = ordinal


def device():
    torch = _torch()
    open_device(0 if _opened is None else _opened)
    return torch.device("cuda", _opened)


def stream_handle():
    """hipStream_t of torch's current stream, as an int for ctypes."""
    torch = _torch()
    return torch.cuda.current_stream().cuda_stream


def ptr(tensor) -> int | None:
    if tensor is None:
        return None
    if not tensor.is_cuda:
        raise _lib.RangeError("afhip takes device tensors")
    if not tensor.is_contiguous():
        raise _lib.RangeError("afhip takes contiguous tensors")
    return tensor.data_ptr()


def empty_bytes(nbytes: int):
    torch = _torch()
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device())


def synchronize() -> None:
    _torch().cuda.synchronize()


def memory_snapshot() -> dict:
    """The AllocationSnapshot fields each reference run() returns
    (src/runtime/allocator.ts:8-29), read from the allocator that holds this
    process's device tensors (PyTorch's caching allocator). Its pools are not
    labelled, so peakComposition is empty."""
    torch = _torch()
    stats = torch.cuda.memory_stats()
    current = int(torch.cuda.memory_allocated())
    resident = int(torch.cuda.memory_reserved())
    return {"currentBytes": current, "peakBytes": int(torch.cuda.max_memory_allocated()), "peakComposition": [],
            "residentBytes": resident, "peakResidentBytes": int(torch.cuda.max_memory_reserved()),
            "pooledBytes": max(resident - current, 0),
            "allocationCount": int(stats.get("allocation.all.allocated", 0)),
            "bufferCount": int(stats.get("segment.all.current", 0))}


def device_report() -> dict:
    open_device(0 if _opened is None else _opened)
    import ctypes

    buf = ctypes.create_string_buffer(4096)
    _lib.call("afhip_device_report", buf, len(buf))
    return json.loads(buf.value.decode())


class Timer:
    """Wall time around a synchronised region, in milliseconds."""

    def __enter__(self):
        synchronize()
        self.start = time.perf_counter()
        return self

    def __exit__(self, *exc):
        synchronize()
        self.milliseconds = (time.perf_counter() - self.start) * 1e3


def timing_enable(enable: bool) -> None:
    _lib.call("afhip_timing_enable", int(bool(enable)))


def timing_reset() -> None:
    _lib.call("afhip_timing_reset")


def timing_report() -> dict:
    import ctypes

    buf = ctypes.create_string_buffer(1 << 16)
    _lib.call("afhip_timing_report", buf, len(buf))
    return json.loads(buf.value.decode())
