"""Triangle multiplication, outgoing and incoming.

Mirrors src/triangle/webgpu.ts (TriangleMultiplication{Outgoing,Incoming}Gpu,
run(input, options) -> {output, elapsedMilliseconds, memory}) and
src/triangle/types.ts (validateTriangleInput, errorMetrics) over
afhip_triangle_*. The device-resident class TriangleMultiplication is what an
execution layer chains without host round trips.
"""
from __future__ import annotations

import ctypes
import math
import time

import numpy as np

from . import _lib
from .device import device, empty_bytes, memory_snapshot, open_device, ptr, stream_handle, synchronize

ORDER = (
    "layerNormInWeight", "layerNormInBias",
    "linearAPWeight", "linearAPBias", "linearAGWeight", "linearAGBias",
    "linearBPWeight", "linearBPBias", "linearBGWeight", "linearBGBias",
    "layerNormOutWeight", "layerNormOutBias",
    "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
)


def _positive_integer(name: str, value) -> None:
    if not isinstance(value, (int, np.integer)) or isinstance(value, bool) or value <= 0 or value > 2 ** 53 - 1:
        raise _lib.RangeError(f"{name} must be a positive safe integer; received {value}")


def _expect_length(name: str, value, length: int) -> None:
    n = int(np.asarray(value).size) if not hasattr(value, "numel") else int(value.numel())
    if n != length:
        raise _lib.RangeError(f"{name} has {n} values; expected {length}")


def triangle_shape(inp: dict) -> tuple:
    """(length, cZ, cHidden) of an input whose shape is the reference's
    TriangleShape {length, cZ, cHidden} (src/triangle/types.ts:3-7) or a
    (length, cZ, cHidden) tuple."""
    shape = inp["shape"]
    if isinstance(shape, dict):
        return shape.get("length"), shape.get("cZ"), shape.get("cHidden")
    return tuple(shape)


def validate_triangle_input(inp: dict) -> None:
    """validateTriangleInput (src/triangle/types.ts:54-89)."""
    length, cz, ch = triangle_shape(inp)
    _positive_integer("length", length)
    _positive_integer("cZ", cz)
    _positive_integer("cHidden", ch)
    pairs = length * length
    if pairs * max(cz, ch) > 2 ** 53 - 1:
        raise _lib.RangeError("tensor dimensions exceed the safe integer range")
    _expect_length("z", inp["z"], pairs * cz)
    _expect_length("mask", inp["mask"], pairs)
    w = inp["weights"]
    sizes = {"layerNormInWeight": cz, "layerNormInBias": cz, "linearAPWeight": ch * cz, "linearAPBias": ch,
             "linearAGWeight": ch * cz, "linearAGBias": ch, "linearBPWeight": ch * cz, "linearBPBias": ch,
             "linearBGWeight": ch * cz, "linearBGBias": ch, "layerNormOutWeight": ch, "layerNormOutBias": ch,
             "linearZWeight": cz * ch, "linearZBias": cz, "linearGWeight": cz * cz, "linearGBias": cz}
    for name in ORDER:
        _expect_length(name, w[name], sizes[name])
    eps = inp.get("epsilon")
    if eps is not None and (not eps > 0 or not math.isfinite(eps)):
        raise _lib.RangeError(f"epsilon must be finite and positive; received {eps}")


def error_metrics(actual, expected) -> dict:
    """errorMetrics (src/triangle/types.ts:91-110)."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    if a.size != e.size or a.size == 0:
        raise _lib.RangeError("error metrics require equally sized, non-empty arrays")
    d = np.abs(a - e)
    return {"meanAbsoluteError": float(d.mean()), "maxAbsoluteError": float(d.max()),
            "rootMeanSquareError": float(np.sqrt((d * d).mean()))}


def pack_weights(weights: dict) -> np.ndarray:
    """packWeights (src/triangle/weights.ts:20-34), f32, ORDER."""
    return np.concatenate([np.ascontiguousarray(weights[n], dtype=np.float32).reshape(-1) for n in ORDER])


_DT = {"f32": _lib.F32, "f16": _lib.F16}


class TriangleMultiplication:
    """Device-resident operator: prepare weights once, then call on device
    tensors z [L][L][cZ] and mask [L][L]."""

    def __init__(self, length: int, c_z: int, c_hidden: int, *, direction: str = "outgoing",
                 precision: str = "f32", pair_dtype: str = "f32", out_dtype: str = "f32", block_rows: int = 0,
                 residual: bool = False, epsilon: float = 1e-5):
        open_device()
        if direction not in ("outgoing", "incoming"):
            raise _lib.RangeError(f"unknown direction {direction}")
        self.desc = _lib.TriangleDesc(length, c_z, c_hidden,
                                      _lib.TRIANGLE_OUTGOING if direction == "outgoing" else _lib.TRIANGLE_INCOMING,
                                      _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32,
                                      _DT[pair_dtype], _DT[out_dtype], block_rows, int(residual), epsilon)
        size = ctypes.c_size_t()
        _lib.call("afhip_triangle_workspace_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.workspace_bytes = size.value
        self.workspace = empty_bytes(size.value)
        _lib.call("afhip_triangle_weights_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.prepared = empty_bytes(size.value)
        self.out_dtype = out_dtype
        self.shape = (length, c_z, c_hidden)

    def prepare(self, weights) -> None:
        """weights: dict of the sixteen tensors or the packed f32 array."""
        import torch

        packed = pack_weights(weights) if isinstance(weights, dict) else np.asarray(weights, np.float32)
        src = torch.from_numpy(packed).to(device())
        _lib.call("afhip_triangle_prepare_weights", ctypes.byref(self.desc), ptr(src), ptr(self.prepared),
                  stream_handle())
        synchronize()

    def __call__(self, z, mask, out=None):
        import torch

        length, cz, _ = self.shape
        if out is None:
            out = torch.empty((length, length, cz), dtype=torch.float32 if self.out_dtype == "f32" else torch.float16,
                              device=device())
        _lib.call("afhip_triangle_run", ctypes.byref(self.desc), ptr(z), ptr(mask), ptr(self.prepared), ptr(out),
                  ptr(self.workspace), self.workspace_bytes, stream_handle())
        return out


class _TriangleMultiplicationGpu:
    direction = "outgoing"

    def run(self, inp: dict, options: dict | None = None) -> dict:
        """run(input, {precision?, blockRows?, pairStorage?}) (webgpu.ts:56-201).

        precision "f32" keeps every product and sum in f32; "f16" rounds the
        operands of every product to f16 and accumulates in f32. The output is
        f32, as the reference returns a Float32Array.
        """
        import torch

        options = options or {}
        validate_triangle_input(inp)
        length, cz, ch = triangle_shape(inp)
        precision = options.get("precision", "f32")
        if precision not in ("f32", "f16"):
            raise _lib.RangeError(f"unknown precision {precision}")
        block_rows = max(1, min(length, int(options.get("blockRows", length))))
        pair_storage = options.get("pairStorage", "f32")
        op = TriangleMultiplication(length, cz, ch, direction=self.direction, precision=precision,
                                    pair_dtype=pair_storage, out_dtype="f32", block_rows=block_rows,
                                    epsilon=float(inp.get("epsilon") or 1e-5))
        op.prepare(inp["weights"])
        z = torch.from_numpy(np.ascontiguousarray(inp["z"], np.float32).reshape(length, length, cz))
        if pair_storage == "f16":
            z = z.half()
        mask = torch.from_numpy(np.ascontiguousarray(inp["mask"], np.float32).reshape(length, length))
        start = time.perf_counter()
        zd, md = z.to(device()), mask.to(device())
        out = op(zd, md)
        result = out.cpu().numpy()
        elapsed = (time.perf_counter() - start) * 1e3
        return {"output": result.reshape(-1), "elapsedMilliseconds": elapsed, "memory": memory_snapshot()}


class TriangleMultiplicationOutgoingGpu(_TriangleMultiplicationGpu):
    direction = "outgoing"


class TriangleMultiplicationIncomingGpu(_TriangleMultiplicationGpu):
    direction = "incoming"
