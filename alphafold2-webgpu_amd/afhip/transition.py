"""Transition: LayerNorm, linear + ReLU, linear.

Mirrors src/evoformer/transition.ts (TransitionGpu.run :264-361, validate
:140-156, packTransitionWeights :157-177) over afhip_transition_*.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np

from . import _lib
from .device import device, empty_bytes, memory_snapshot, open_device, ptr, stream_handle, synchronize

ORDER = ("layerNormScale", "layerNormOffset", "firstWeight", "firstBias", "secondWeight", "secondBias")
_DT = {"f32": _lib.F32, "f16": _lib.F16}


def validate(inp: dict) -> None:
    rows, c, h = inp["rows"], inp["channels"], inp["hiddenChannels"]
    if not all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) and v > 0 for v in (rows, c, h)):
        raise _lib.RangeError("transition dimensions must be positive safe integers")
    w = inp["weights"]
    for name, value, size in [("activations", inp["activations"], rows * c), ("layerNormScale", w["layerNormScale"], c),
                              ("layerNormOffset", w["layerNormOffset"], c), ("firstWeight", w["firstWeight"], c * h),
                              ("firstBias", w["firstBias"], h), ("secondWeight", w["secondWeight"], h * c),
                              ("secondBias", w["secondBias"], c)]:
        n = int(np.asarray(value).size)
        if n != size:
            raise _lib.RangeError(f"{name} has {n} values; expected {size}")


def pack_weights(weights: dict) -> np.ndarray:
    return np.concatenate([np.ascontiguousarray(weights[n], np.float32).reshape(-1) for n in ORDER])


class Transition:
    """Device-resident operator over [rows][channels]."""

    def __init__(self, rows: int, channels: int, hidden: int, *, precision: str = "f32", in_dtype: str = "f32",
                 out_dtype: str = "f32", residual: bool = False, epsilon: float = 1e-5):
        open_device()
        self.desc = _lib.TransitionDesc(rows, channels, hidden,
                                        _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32,
                                        _DT[in_dtype], _DT[out_dtype], int(residual), epsilon)
        size = ctypes.c_size_t()
        _lib.call("afhip_transition_workspace_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.workspace_bytes = size.value
        self.workspace = empty_bytes(size.value)
        _lib.call("afhip_transition_weights_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.prepared = empty_bytes(size.value)
        self.out_dtype = out_dtype
        self.shape = (rows, channels, hidden)

    def prepare(self, weights) -> None:
        import torch

        packed = pack_weights(weights) if isinstance(weights, dict) else np.asarray(weights, np.float32)
        src = torch.from_numpy(packed).to(device())
        _lib.call("afhip_transition_prepare_weights", ctypes.byref(self.desc), ptr(src), ptr(self.prepared),
                  stream_handle())
        synchronize()

    def __call__(self, activations, out=None):
        import torch

        rows, c, _ = self.shape
        if out is None:
            out = torch.empty((rows, c), dtype=torch.float32 if self.out_dtype == "f32" else torch.float16,
                              device=device())
        _lib.call("afhip_transition_run", ctypes.byref(self.desc), ptr(activations), ptr(self.prepared), ptr(out),
                  ptr(self.workspace), self.workspace_bytes, stream_handle())
        return out


class TransitionGpu:
    def run(self, inp: dict, options: dict | None = None) -> dict:
        import torch

        options = options or {}
        validate(inp)
        rows, c, h = inp["rows"], inp["channels"], inp["hiddenChannels"]
        op = Transition(rows, c, h, precision=options.get("precision", "f32"), epsilon=float(inp.get("epsilon") or 1e-5))
        op.prepare(inp["weights"])
        x = torch.from_numpy(np.ascontiguousarray(inp["activations"], np.float32).reshape(rows, c))
        start = time.perf_counter()
        out = op(x.to(device()))
        result = out.cpu().numpy()
        return {"output": result.reshape(-1), "elapsedMilliseconds": (time.perf_counter() - start) * 1e3,
                "memory": memory_snapshot()}
