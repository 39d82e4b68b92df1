"""The execution layer: device-resident tensors across operator calls and the
pair-representation steps of an Evoformer block chained on the device.

`Execution` mirrors WebGpuExecution (src/runtime/execution.ts:153-555) with
its pooled allocator (src/runtime/allocator.ts:168-388): allocate, upload,
release, checkpoint / release_since, note_submitted, snapshot, add_in_place.
`PairStack` runs the pair steps of encodeEvoformerBlock (src/evoformer/block.ts:
1673-1759) in place on one pair tensor, and `EvoformerBlock` the whole block
(the MSA steps, then the pair steps), with every workspace taken from the
execution's pool. Tensors are plain device pointers
(ints); torch tensors are accepted wherever a pointer is.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _lib
from . import attention as _attention
from . import opm as _opm
from . import transition as _transition
from . import triangle as _triangle
from .device import open_device, stream_handle, synchronize

_DT = {"f32": _lib.F32, "f16": _lib.F16}


def _address(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if not x.is_cuda or not x.is_contiguous():
        raise _lib.RangeError("afhip takes contiguous device tensors")
    return x.data_ptr()


def set_memory_budget(nbytes: int | None) -> None:
    """setGpuMemoryBudget (allocator.ts:66-71): cap the resident bytes of every
    execution on the device together; None removes the cap."""
    open_device()
    if nbytes is not None and nbytes <= 0:
        raise _lib.RangeError("GPU memory budget must be a positive safe integer")
    _lib.call("afhip_set_memory_budget", int(nbytes or 0))


def memory_resident() -> int:
    """gpuMemoryResident (allocator.ts:74)."""
    out = ctypes.c_uint64()
    _lib.call("afhip_memory_resident", ctypes.byref(out))
    return out.value


class Execution:
    def __init__(self, max_pooled_bytes: int = 0):
        open_device()
        handle = ctypes.c_void_p()
        _lib.call("afhip_execution_create", int(max_pooled_bytes), stream_handle(), ctypes.byref(handle))
        self._h = handle

    @property
    def handle(self):
        if self._h is None:
            raise _lib.RangeError("the execution has been released")
        return self._h

    def allocate(self, label: str, nbytes: int) -> int:
        out = ctypes.c_void_p()
        _lib.call("afhip_execution_allocate", self.handle, label.encode(), int(nbytes), ctypes.byref(out))
        return out.value

    def upload(self, label: str, data: np.ndarray) -> int:
        data = np.ascontiguousarray(data)
        out = ctypes.c_void_p()
        _lib.call("afhip_execution_upload", self.handle, label.encode(), data.ctypes.data, data.nbytes,
                  ctypes.byref(out))
        return out.value

    def download(self, tensor, shape, dtype=np.float32) -> np.ndarray:
        synchronize()
        out = np.empty(shape, dtype)
        _lib.call("afhip_buffer_read", _address(tensor), 0, out.ctypes.data, out.nbytes)
        return out

    def release_tensor(self, tensor) -> None:
        _lib.call("afhip_execution_release", self.handle, _address(tensor))

    def checkpoint(self) -> int:
        out = ctypes.c_uint64()
        _lib.call("afhip_execution_checkpoint", self.handle, ctypes.byref(out))
        return out.value

    def release_since(self, checkpoint: int) -> None:
        _lib.call("afhip_execution_release_since", self.handle, int(checkpoint))

    def note_submitted(self) -> None:
        _lib.call("afhip_execution_note_submitted", self.handle)

    def snapshot(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 16)
        _lib.call("afhip_execution_snapshot", self.handle, buf, len(buf))
        return json.loads(buf.value.decode())

    def add_in_place(self, base, update, elements: int, base_dtype: str = "f32", update_dtype: str = "f32") -> None:
        _lib.call("afhip_execution_add_in_place", self.handle, _address(base), _DT[base_dtype], _address(update),
                  _DT[update_dtype], int(elements))

    def release(self) -> None:
        """WebGpuExecution.release (execution.ts:549-554)."""
        if self._h is not None:
            _lib.call("afhip_execution_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class PairStack:
    """The pair steps of an Evoformer block, in the block's order, each adding
    into the pair in place: outer-product mean, triangle multiplication
    outgoing and incoming, triangle attention around the starting and the
    ending node, pair transition (block.ts:1683-1750). Weights are prepared
    once into the execution's pool."""

    def __init__(self, execution: Execution, length: int, *, sequences: int, c_m: int, c_z: int = 128,
                 c_outer: int = 32, c_hidden: int = 128, transition_factor: int = 4, precision: str = "f16",
                 pair_dtype: str = "f16", msa_dtype: str = "f16", opm_row_block: int = 0,
                 triangle_block_rows: int = 0, attention_heads: int = 4):
        self.execution = execution
        prec = _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32
        pdt = _DT[pair_dtype]
        self.desc = _lib.PairStackDesc()
        self.desc.opm = _lib.OpmDesc(sequences, length, c_m, c_outer, c_z, prec, _DT[msa_dtype], pdt, opm_row_block,
                                     1, 1e-5, 1e-3)
        self.desc.outgoing = _lib.TriangleDesc(length, c_z, c_hidden, _lib.TRIANGLE_OUTGOING, prec, pdt, pdt,
                                               triangle_block_rows, 1, 1e-5)
        self.desc.incoming = _lib.TriangleDesc(length, c_z, c_hidden, _lib.TRIANGLE_INCOMING, prec, pdt, pdt,
                                               triangle_block_rows, 1, 1e-5)
        for attr, transpose in (("attention_start", 0), ("attention_end", 1)):
            setattr(self.desc, attr, _lib.AttentionDesc(length, length, c_z, attention_heads, transpose,
                                                        _lib.PAIR_BIAS_NORMALIZED_INPUT, 0, prec, pdt, pdt, 1, 1e-5))
        self.desc.transition = _lib.TransitionDesc(length * length, c_z, transition_factor * c_z, prec, pdt, pdt, 1,
                                                   1e-5)
        self.weights = _lib.PairStackWeights()
        self.shape = (length, c_z)

    def _prepare(self, name: str, desc, packed: np.ndarray, size_fn: str, prepare_fn: str) -> int:
        ex = self.execution
        size = ctypes.c_size_t()
        _lib.call(size_fn, ctypes.byref(desc), ctypes.byref(size))
        src = ex.upload(f"pair-stack.{name}.weights-f32", np.ascontiguousarray(packed, np.float32))
        dst = ex.allocate(f"pair-stack.{name}.weights", size.value)
        _lib.call(prepare_fn, ctypes.byref(desc), src, dst, stream_handle())
        synchronize()
        ex.release_tensor(src)
        return dst

    def prepare(self, weights: dict) -> None:
        """weights: {"outerProductMean", "triangleMultiplicationOutgoing",
        "triangleMultiplicationIncoming", "triangleAttentionStarting",
        "triangleAttentionEnding", "pairTransition"}, each the operator's
        weight dict (or its packed f32 array) — the attentions as the block's
        {"attention": AttentionWeights, "pairProjectionWeight": [c_z][heads]}
        (block.ts:1727-1745); a missing one skips that step."""
        d = self.desc
        if weights.get("outerProductMean") is not None:
            w = weights["outerProductMean"]
            self.weights.opm = self._prepare("outer-product-mean", d.opm, _opm.pack_weights(w) if isinstance(w, dict)
                                             else w, "afhip_opm_weights_size", "afhip_opm_prepare_weights")
        for key, attr, desc in (("triangleMultiplicationOutgoing", "outgoing", d.outgoing),
                                ("triangleMultiplicationIncoming", "incoming", d.incoming)):
            if weights.get(key) is not None:
                w = weights[key]
                setattr(self.weights, attr, self._prepare(
                    f"triangle-{attr}", desc, _triangle.pack_weights(w) if isinstance(w, dict) else w,
                    "afhip_triangle_weights_size", "afhip_triangle_prepare_weights"))
        for key, attr in (("triangleAttentionStarting", "attention_start"),
                          ("triangleAttentionEnding", "attention_end")):
            if weights.get(key) is not None:
                w = weights[key]
                packed = w if not isinstance(w, dict) else _attention.pack_weights(
                    w["attention"], {"source": "normalized-input", "projectionWeight": w["pairProjectionWeight"]})
                setattr(self.weights, attr, self._prepare(
                    attr.replace("_", "-"), getattr(d, attr), packed, "afhip_attention_weights_size",
                    "afhip_attention_prepare_weights"))
        if weights.get("pairTransition") is not None:
            w = weights["pairTransition"]
            self.weights.transition = self._prepare(
                "transition", d.transition, _transition.pack_weights(w) if isinstance(w, dict) else w,
                "afhip_transition_weights_size", "afhip_transition_prepare_weights")

    def __call__(self, pair, pair_mask, msa=None, msa_mask=None) -> None:
        _lib.call("afhip_execution_pair_stack", self.execution.handle, ctypes.byref(self.desc),
                  ctypes.byref(self.weights), _address(msa), _address(msa_mask), _address(pair), _address(pair_mask))


class EvoformerBlock:
    """encodeEvoformerBlock (block.ts:1673-1759): MSA row attention with the
    pair bias, MSA column attention, MSA transition, then the pair steps
    (outer-product mean first instead when opm_first). The MSA and the pair
    are updated in place and share one dtype."""

    def __init__(self, execution: Execution, length: int, *, sequences: int, c_m: int = 256, c_z: int = 128,
                 msa_heads: int = 8, pair_heads: int = 4, msa_transition_factor: int = 4, opm_first: bool = False,
                 precision: str = "f16", dtype: str = "f16", **pair_options):
        self.execution = execution
        self.stack = PairStack(execution, length, sequences=sequences, c_m=c_m, c_z=c_z, precision=precision,
                               pair_dtype=dtype, msa_dtype=dtype, attention_heads=pair_heads, **pair_options)
        prec = _lib.PRECISION_F16 if precision == "f16" else _lib.PRECISION_F32
        dt = _DT[dtype]
        self.desc = _lib.EvoformerBlockDesc()
        self.desc.msa_row = _lib.AttentionDesc(sequences, length, c_m, msa_heads, 0, _lib.PAIR_BIAS_SEPARATE, c_z, prec,
                                               dt, dt, 1, 1e-5)
        self.desc.msa_column = _lib.AttentionDesc(length, sequences, c_m, msa_heads, 1, _lib.PAIR_BIAS_NONE, 0, prec,
                                                  dt, dt, 1, 1e-5)
        self.desc.msa_transition = _lib.TransitionDesc(sequences * length, c_m, msa_transition_factor * c_m, prec, dt,
                                                       dt, 1, 1e-5)
        self.desc.opm_first = int(opm_first)
        self.weights = _lib.EvoformerBlockWeights()

    def prepare(self, weights: dict) -> None:
        """weights: the pair stack's keys, plus "msaRowAttention" ({"attention",
        "pairLayerNormScale", "pairLayerNormOffset", "pairProjectionWeight"},
        block.ts:1690-1702), "msaColumnAttention" ({"attention"}) and
        "msaTransition" (a transition weight dict); a missing one skips that
        step."""
        st, d = self.stack, self.desc
        st.prepare(weights)
        row = weights.get("msaRowAttention")
        if row is not None:
            pb = {"source": "separate", "layerNormScale": row["pairLayerNormScale"],
                  "layerNormOffset": row["pairLayerNormOffset"], "projectionWeight": row["pairProjectionWeight"]}
            self.weights.msa_row = st._prepare("msa-row-attention", d.msa_row,
                                               _attention.pack_weights(row["attention"], pb),
                                               "afhip_attention_weights_size", "afhip_attention_prepare_weights")
        col = weights.get("msaColumnAttention")
        if col is not None:
            self.weights.msa_column = st._prepare("msa-column-attention", d.msa_column,
                                                  _attention.pack_weights(col["attention"]),
                                                  "afhip_attention_weights_size", "afhip_attention_prepare_weights")
        tr = weights.get("msaTransition")
        if tr is not None:
            self.weights.msa_transition = st._prepare(
                "msa-transition", d.msa_transition, _transition.pack_weights(tr) if isinstance(tr, dict) else tr,
                "afhip_transition_weights_size", "afhip_transition_prepare_weights")
        self.desc.pair = st.desc
        self.weights.pair = st.weights

    def __call__(self, msa, msa_mask, pair, pair_mask) -> None:
        _lib.call("afhip_execution_evoformer_block", self.execution.handle, ctypes.byref(self.desc),
                  ctypes.byref(self.weights), _address(msa), _address(msa_mask), _address(pair), _address(pair_mask))
