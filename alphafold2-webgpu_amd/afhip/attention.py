"""Gated multi-head attention with an optional pair bias: the Evoformer's MSA
row attention (separate pair bias), MSA column attention (transposed) and
triangle attention around the starting and ending node (normalized-input
bias, the ending node transposed).

Mirrors src/evoformer/attention.ts (AttentionGpu.run :1321-1452, validate
:102-141, packAttentionWeights :179-201) over afhip_attention_*.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np

from . import _lib
from .device import device, empty_bytes, memory_snapshot, open_device, ptr, stream_handle, synchronize

ORDER = ("queryNormScale", "queryNormOffset", "queryWeight", "keyWeight", "valueWeight", "gatingWeight",
         "gatingBias", "outputWeight", "outputBias")
_DT = {"f32": _lib.F32, "f16": _lib.F16}
_SOURCES = {None: _lib.PAIR_BIAS_NONE, "normalized-input": _lib.PAIR_BIAS_NORMALIZED_INPUT,
            "separate": _lib.PAIR_BIAS_SEPARATE}


def _count(x) -> int:
    return int(np.asarray(x).size)


def validate(inp: dict) -> None:
    """validate (attention.ts:102-141), the same checks and messages."""
    b, q, c, h = inp["batch"], inp["queryLength"], inp["channels"], inp["heads"]
    if not all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) and v > 0 for v in (b, q, c, h)):
        raise _lib.RangeError("attention dimensions must be positive safe integers")
    if c % h != 0 or c // h > 32:
        raise _lib.RangeError(
            "the fused WebGPU attention path requires an integral head dimension no larger than 32")
    w = inp["weights"]
    expected = [("activations", inp["activations"], b * q * c), ("mask", inp["mask"], b * q),
                ("queryNormScale", w["queryNormScale"], c), ("queryNormOffset", w["queryNormOffset"], c),
                ("queryWeight", w["queryWeight"], c * c), ("keyWeight", w["keyWeight"], c * c),
                ("valueWeight", w["valueWeight"], c * c), ("gatingWeight", w["gatingWeight"], c * c),
                ("gatingBias", w["gatingBias"], c), ("outputWeight", w["outputWeight"], c * c),
                ("outputBias", w["outputBias"], c)]
    for name, value, size in expected:
        if _count(value) != size:
            raise _lib.RangeError(f"{name} has {_count(value)} values; expected {size}")
    pair = inp.get("pairBias")
    if pair is not None and pair["source"] == "separate":
        pc = pair["channels"]
        for name, value, size in [("pair activations", pair["activations"], q * q * pc),
                                  ("pair norm scale", pair["layerNormScale"], pc),
                                  ("pair norm offset", pair["layerNormOffset"], pc),
                                  ("pair projection", pair["projectionWeight"], pc * h)]:
            if _count(value) != size:
                raise _lib.RangeError(f"{name} has {_count(value)} values; expected {size}")
    elif pair is not None and _count(pair["projectionWeight"]) != c * h:
        raise _lib.RangeError("normalized-input pair projection has an invalid size")


def pack_weights(weights: dict, pair_bias: dict | None = None) -> np.ndarray:
    """packAttentionWeights (attention.ts:179-201): the nine tensors, then the
    separate bias's LayerNorm scale, offset and projection, or the
    normalized-input bias's projection."""
    tensors = [np.ascontiguousarray(weights[n], np.float32).reshape(-1) for n in ORDER]
    if pair_bias is not None:
        names = (("layerNormScale", "layerNormOffset", "projectionWeight") if pair_bias["source"] == "separate"
                 else ("projectionWeight",))
        tensors += [np.ascontiguousarray(pair_bias[n], np.float32).reshape(-1) for n in names]
    return np.concatenate(tensors)


class Attention:
    """Device-resident operator: activations [batch * queries][channels] and
    mask [batch * queries] in source order (entry (b, q) of the attention
    batch is row b * queries + q, or q * batch + b when transposed)."""

    def __init__(self, batch: int, queries: int, channels: int, heads: int, *, transpose: bool = False,
                 pair_bias: str | None = None, pair_channels: int = 0, precision: str = "f32",
                 in_dtype: str = "f32", out_dtype: str = "f32", residual: bool = False, epsilon: float = 1e-5):
        open_device()
        if pair_bias not in _SOURCES:
            raise _lib.RangeError(f"unknown pair bias source {pair_bias!r}")
        self.desc = _lib.AttentionDesc(batch, queries, channels, heads, int(transpose), _SOURCES[pair_bias],
                                       pair_channels, _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32,
                                       _DT[in_dtype], _DT[out_dtype], int(residual), epsilon)
        size = ctypes.c_size_t()
        _lib.call("afhip_attention_workspace_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.workspace_bytes = size.value
        self.workspace = empty_bytes(size.value)
        _lib.call("afhip_attention_weights_size", ctypes.byref(self.desc), ctypes.byref(size))
        self.prepared = empty_bytes(size.value)
        self.out_dtype = out_dtype
        self.shape = (batch * queries, channels)

    def prepare(self, packed) -> None:
        """packed: pack_weights(weights, pair_bias) (f32)."""
        import torch

        src = torch.from_numpy(np.ascontiguousarray(packed, np.float32).reshape(-1)).to(device())
        _lib.call("afhip_attention_prepare_weights", ctypes.byref(self.desc), ptr(src), ptr(self.prepared),
                  stream_handle())
        synchronize()

    def __call__(self, activations, mask, pair_activations=None, out=None):
        import torch

        if out is None:
            out = torch.empty(self.shape, dtype=torch.float32 if self.out_dtype == "f32" else torch.float16,
                              device=device())
        _lib.call("afhip_attention_run", ctypes.byref(self.desc), ptr(activations), ptr(mask),
                  ptr(pair_activations), ptr(self.prepared), ptr(out), ptr(self.workspace), self.workspace_bytes,
                  stream_handle())
        return out


class AttentionGpu:
    """AttentionGpu (attention.ts:1321-1452): run(input) takes host arrays in
    the reference's AttentionInput shape and returns its AttentionResult."""

    def run(self, inp: dict, options: dict | None = None) -> dict:
        import torch

        options = options or {}
        validate(inp)
        b, q, c, h = inp["batch"], inp["queryLength"], inp["channels"], inp["heads"]
        pair = inp.get("pairBias")
        op = Attention(b, q, c, h, transpose=bool(inp.get("transpose")),
                       pair_bias=None if pair is None else pair["source"],
                       pair_channels=int(pair["channels"]) if pair is not None and pair["source"] == "separate" else 0,
                       precision=options.get("precision", "f32"), epsilon=float(inp.get("epsilon") or 1e-5))
        op.prepare(pack_weights(inp["weights"], pair))
        dev = device()
        x = torch.from_numpy(np.ascontiguousarray(inp["activations"], np.float32).reshape(b * q, c)).to(dev)
        m = torch.from_numpy(np.ascontiguousarray(inp["mask"], np.float32).reshape(-1)).to(dev)
        p = None
        if pair is not None and pair["source"] == "separate":
            p = torch.from_numpy(np.ascontiguousarray(pair["activations"], np.float32).reshape(-1)).to(dev)
        start = time.perf_counter()
        out = op(x, m, p)
        result = out.cpu().numpy()
        return {"output": result.reshape(-1), "elapsedMilliseconds": (time.perf_counter() - start) * 1e3,
                "memory": memory_snapshot()}
