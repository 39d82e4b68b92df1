"""Outer-product mean.

Mirrors src/evoformer/outer-product-mean.ts (OuterProductMeanGpu.run
:549-646, input validation :42-62, packOuterProductMeanWeights :64-79,
outerProductMeanRowBlock :523-536) over afhip_opm_*.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np

from . import _lib
from .device import device, empty_bytes, memory_snapshot, open_device, ptr, stream_handle, synchronize

ORDER = ("layerNormScale", "layerNormOffset", "leftWeight", "leftBias", "rightWeight", "rightBias",
         "outputWeight", "outputBias")
_DT = {"f32": _lib.F32, "f16": _lib.F16}


def validate(inp: dict) -> None:
    """validate (outer-product-mean.ts:42-62)."""
    dims = [inp["sequences"], inp["length"], inp["cM"], inp["cOuter"], inp["cZ"]]
    if not all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) and 0 < v <= 2 ** 53 - 1 for v in dims):
        raise _lib.RangeError("outer product mean dimensions must be positive safe integers")
    S, L, cm, co, cz = dims
    w = inp["weights"]
    expected = [("activations", inp["activations"], S * L * cm), ("mask", inp["mask"], S * L),
                ("layerNormScale", w["layerNormScale"], cm), ("layerNormOffset", w["layerNormOffset"], cm),
                ("leftWeight", w["leftWeight"], cm * co), ("leftBias", w["leftBias"], co),
                ("rightWeight", w["rightWeight"], cm * co), ("rightBias", w["rightBias"], co),
                ("outputWeight", w["outputWeight"], co * co * cz), ("outputBias", w["outputBias"], cz)]
    for name, value, size in expected:
        n = int(np.asarray(value).size)
        if n != size:
            raise _lib.RangeError(f"{name} has {n} values; expected {size}")


def pack_weights(weights: dict) -> np.ndarray:
    """packOuterProductMeanWeights (outer-product-mean.ts:64-79)."""
    return np.concatenate([np.ascontiguousarray(weights[n], np.float32).reshape(-1) for n in ORDER])


def row_block(length: int, c_outer: int, budget_bytes: int = 16 * 1024 * 1024, storage: str = "f32") -> int:
    """outerProductMeanRowBlock (outer-product-mean.ts:523-536)."""
    for v in (length, c_outer, budget_bytes):
        if not isinstance(v, int) or v <= 0:
            raise _lib.RangeError("outer-product block dimensions and budget must be positive safe integers")
    per = length * c_outer * c_outer * (2 if storage == "f16" else 4)
    return max(1, min(length, budget_bytes // per))


class OuterProductMean:
    """Device-resident operator: activations [S][L][cM], mask [S][L] -> [L][L][cZ]."""

    def __init__(self, sequences: int, length: int, c_m: int, c_outer: int, c_z: int, *, precision: str = "f32",
                 msa_dtype: str = "f32", out_dtype: str = "f32", row_block: int = 0, residual: bool = False,
                 layer_norm_epsilon: float = 1e-5, normalization_epsilon: float = 1e-3):
        open_device()
        self.desc = _lib.OpmDesc(sequences, length, c_m, c_outer, c_z,
                                 _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32, _DT[msa_dtype],
                                 _DT[out_dtype], row_block, int(residual), layer_norm_epsilon, normalization_epsilon)
        size = ctypes.c_size_t()
        _lib.call("afhip_opm_workspace_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.workspace_bytes = size.value
        self.workspace = empty_bytes(size.value)
        _lib.call("afhip_opm_weights_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.prepared = empty_bytes(size.value)
        self.out_dtype = out_dtype
        self.shape = (sequences, length, c_m, c_outer, c_z)

    def prepare(self, weights) -> None:
        import torch

        packed = pack_weights(weights) if isinstance(weights, dict) else np.asarray(weights, np.float32)
        src = torch.from_numpy(packed).to(device())
        _lib.call("afhip_opm_prepare_weights", ctypes.byref(self.desc), ptr(src), ptr(self.prepared), stream_handle())
        synchronize()

    def __call__(self, activations, mask, out=None):
        import torch

        _, length, _, _, cz = self.shape
        if out is None:
            out = torch.empty((length, length, cz), dtype=torch.float32 if self.out_dtype == "f32" else torch.float16,
                              device=device())
        _lib.call("afhip_opm_run", ctypes.byref(self.desc), ptr(activations), ptr(mask), ptr(self.prepared), ptr(out),
                  ptr(self.workspace), self.workspace_bytes, stream_handle())
        return out


class OuterProductMeanGpu:
    def run(self, inp: dict, options: dict | None = None) -> dict:
        """run(input) (outer-product-mean.ts:549-646); options {precision?}."""
        import torch

        options = options or {}
        validate(inp)
        S, L, cm, co, cz = inp["sequences"], inp["length"], inp["cM"], inp["cOuter"], inp["cZ"]
        precision = options.get("precision", "f32")
        op = OuterProductMean(S, L, cm, co, cz, precision=precision, row_block=int(inp.get("rowBlockResidues") or 0),
                              layer_norm_epsilon=float(inp.get("layerNormEpsilon") or 1e-5),
                              normalization_epsilon=float(inp.get("normalizationEpsilon") or 1e-3))
        op.prepare(inp["weights"])
        act = torch.from_numpy(np.ascontiguousarray(inp["activations"], np.float32).reshape(S, L, cm))
        mask = torch.from_numpy(np.ascontiguousarray(inp["mask"], np.float32).reshape(S, L))
        start = time.perf_counter()
        out = op(act.to(device()), mask.to(device()))
        result = out.cpu().numpy()
        return {"output": result.reshape(-1), "elapsedMilliseconds": (time.perf_counter() - start) * 1e3,
                "memory": memory_snapshot()}
