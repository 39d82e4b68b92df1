"""The GEMM plan and dispatch surface.

Mirrors src/runtime/gemm.ts (gemmGrid :368-379, GemmVariant :150-206,
TiledGemmShader :230-339) and src/runtime/gemm-selection.ts
(calibrateGemmVariant :560-660, forceGemmVariant :122-125) over libafhip's
plan API. A WGSL TiledGemmShader carried operand and epilogue fragments; a
plan here carries the enumerated equivalent (dtypes, weight layout,
epilogue flags), since the kernels are compiled ahead of time.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from .device import device, empty_bytes, open_device, ptr, stream_handle

GEMM_GRID_LIMIT = 65_535
GEMM_TILE_ROWS = 64
GEMM_TILE_COLUMNS = 128

_DTYPE_CODES = {"f32": _lib.F32, "f16": _lib.F16, "i8": _lib.I8}
_PRECISION_CODES = {"f32": _lib.PRECISION_F32, "f16": _lib.PRECISION_F16}
_KERNEL_CODES = {"register": _lib.KERNEL_REGISTER_STAGED, "lds_dma": _lib.KERNEL_LDS_DMA,
                 "stream": _lib.KERNEL_STREAM}
_KERNEL_NAMES = {v: k for k, v in _KERNEL_CODES.items()}


def gemm_grid(rows: int, columns: int, tile_columns: int = GEMM_TILE_COLUMNS,
              tile_rows: int = GEMM_TILE_ROWS) -> tuple:
    """gemmGrid (gemm.ts:368-379): workgroups for an M x N output, folding
    row tiles past 65,535 into x. Raises RangeError for non-positive sizes."""
    for v in (rows, columns):
        if not isinstance(v, int) or isinstance(v, bool) or v <= 0 or v > 2 ** 53 - 1:
            raise _lib.RangeError("GEMM dispatch dimensions must be positive safe integers")
    out = (ctypes.c_uint32 * 2)()
    _lib.call("afhip_gemm_grid", rows, columns, tile_columns, tile_rows, out)
    return (int(out[0]), int(out[1]))


@dataclass(frozen=True)
class GemmVariant:
    """The kernel a shape runs with (GemmVariant, gemm.ts:150-206): arithmetic,
    kernel family and output tile. `kernel` is "register" (operands staged
    through VGPRs; any dtype) or "lds_dma" (f16 operands loaded straight into
    LDS, several k-steps in flight). `source` says whether it came from the
    heuristic, a calibration or a pin. "stream" keeps the weight in registers
    and streams 64-row activation tiles past it (tall f16-output projections
    with K of 64, 128 or 256)."""

    precision: str
    tile_rows: int
    tile_columns: int
    tile_inner: int = 32
    source: str = "heuristic"
    kernel: str = "register"

    @staticmethod
    def _from_c(v: _lib.Variant) -> "GemmVariant":
        return GemmVariant("f16" if v.precision == _lib.PRECISION_F16 else "f32", v.tile_rows, v.tile_columns,
                           v.tile_inner, ("heuristic", "calibrated", "pinned")[v.source],
                           _KERNEL_NAMES[v.kernel])

    def _to_c(self) -> _lib.Variant:
        return _lib.Variant(_PRECISION_CODES[self.precision], self.tile_rows, self.tile_columns, self.tile_inner, 1, 2,
                            _KERNEL_CODES[self.kernel])

    @property
    def name(self) -> str:
        return f"mfma-{self.kernel}-{self.precision}-{self.tile_rows}x{self.tile_columns}k{self.tile_inner}"


def _torch_dtype(code: str):
    import torch

    return {"f32": torch.float32, "f16": torch.float16, "i8": torch.int8}[code]


def _code_of(tensor) -> str:
    import torch

    return {torch.float32: "f32", torch.float16: "f16", torch.int8: "i8"}[tensor.dtype]


class TiledGemm:
    """A GEMM plan: C = epilogue(A . W) with W given [K][N] ("column", the
    linear's layout) or [N][K] ("k", the triangle's [out][in]).

    a_layout is the reference's sourceContiguous (gemm.ts:308-321): "k" for
    A[M][K], "row" for A stored [K][M] (GemmOperandArray.columnMajor,
    :341-360). c_layout "row" stores C[M][N], "column" stores it [N][M].
    epilogue: any of "scale", "bias", "attention", "relu", "residual", applied
    in that order to the f32 accumulator (see include/afhip.h).
    """

    def __init__(self, rows: int, inner: int, columns: int, *, precision: str = "f32", a_dtype: str = "f32",
                 w_dtype: str = "f32", w_layout: str = "column", out_dtype: str = "f32", epilogue=(),
                 heads: int = 0, head_dim: int = 0, batch: int = 1, lda: int = 0, ldw: int = 0, ldc: int = 0,
                 batch_stride_a: int = 0, batch_stride_w: int = 0, batch_stride_c: int = 0, a_layout: str = "k",
                 c_layout: str = "row"):
        if a_layout not in ("k", "row"):
            raise _lib.RangeError(f"unknown source layout {a_layout!r}")
        if c_layout not in ("row", "column"):
            raise _lib.RangeError(f"unknown output layout {c_layout!r}")
        open_device()
        flags = 0
        for e in epilogue:
            flags |= {"scale": _lib.EPILOGUE_SCALE, "bias": _lib.EPILOGUE_BIAS,
                      "attention": _lib.EPILOGUE_ATTENTION, "relu": _lib.EPILOGUE_RELU,
                      "residual": _lib.EPILOGUE_RESIDUAL}[e]
        self.desc = _lib.GemmDesc(rows, inner, columns, batch, _PRECISION_CODES[precision], _DTYPE_CODES[a_dtype],
                                  _DTYPE_CODES[w_dtype],
                                  _lib.WEIGHT_COLUMN_CONTIGUOUS if w_layout == "column" else _lib.WEIGHT_K_CONTIGUOUS,
                                  _DTYPE_CODES[out_dtype], flags, heads, head_dim, lda, ldw, ldc, batch_stride_a,
                                  batch_stride_w, batch_stride_c,
                                  _lib.SOURCE_ROW_CONTIGUOUS if a_layout == "row" else _lib.SOURCE_K_CONTIGUOUS,
                                  _lib.OUTPUT_COLUMN_MAJOR if c_layout == "column" else _lib.OUTPUT_ROW_MAJOR)
        handle = ctypes.c_void_p()
        _lib.call("afhip_gemm_plan_create", ctypes.byref(self.desc), ctypes.byref(handle))
        self._plan = handle
        self._destroy = _lib._lib.afhip_gemm_plan_destroy
        size = ctypes.c_size_t()
        _lib.call("afhip_gemm_workspace_size", self._plan, ctypes.byref(size))
        self.workspace_bytes = size.value
        self._workspace = empty_bytes(size.value) if size.value else None
        self.out_dtype = out_dtype
        self.shape = (batch, rows, columns)
        self.c_layout = c_layout

    def __del__(self):
        # The destroy entry point is held by the object itself: at interpreter
        # exit the module globals may already be gone.
        plan = getattr(self, "_plan", None)
        destroy = getattr(self, "_destroy", None)
        if plan is not None and plan.value and destroy is not None:
            destroy(plan)
            self._plan = None

    def variant(self) -> GemmVariant:
        v = _lib.Variant()
        _lib.call("afhip_gemm_select", ctypes.byref(self.desc), ctypes.byref(v))
        return GemmVariant._from_c(v)

    def run(self, a, w, *, scale=None, bias=None, residual=None, out=None):
        import torch

        batch, rows, columns = self.shape
        if out is None:
            if self.c_layout == "column":
                shape = (columns, self.desc.ldc or rows)
            else:
                shape = (rows, self.desc.ldc or columns)
            shape = shape if batch == 1 else (batch,) + shape
            out = torch.empty(shape, dtype=_torch_dtype(self.out_dtype), device=device())
        ws = self._workspace
        _lib.call("afhip_gemm_run", self._plan, ptr(a), ptr(w), ptr(scale), ptr(bias), ptr(residual), ptr(out),
                  None if ws is None else ws.data_ptr(), self.workspace_bytes, stream_handle())
        return out


def select_variant(rows: int, inner: int, columns: int, *, precision: str = "f32", a_dtype: str = "f32",
                   w_dtype: str = "f32", out_dtype: str = "f32", batch: int = 1) -> GemmVariant:
    desc = _lib.GemmDesc(rows, inner, columns, batch, _PRECISION_CODES[precision], _DTYPE_CODES[a_dtype],
                         _DTYPE_CODES[w_dtype], _lib.WEIGHT_K_CONTIGUOUS, _DTYPE_CODES[out_dtype], 0, 0, 0,
                         0, 0, 0, 0, 0, 0)
    v = _lib.Variant()
    _lib.call("afhip_gemm_select", ctypes.byref(desc), ctypes.byref(v))
    return GemmVariant._from_c(v)


def calibrate_variant(rows: int, inner: int, columns: int, *, precision: str = "f16", a_dtype: str = "f16",
                      w_dtype: str = "f16", out_dtype: str = "f32", batch: int = 1) -> GemmVariant:
    """calibrateGemmVariant (gemm-selection.ts:560-660) for one shape class."""
    open_device()
    desc = _lib.GemmDesc(rows, inner, columns, batch, _PRECISION_CODES[precision], _DTYPE_CODES[a_dtype],
                         _DTYPE_CODES[w_dtype], _lib.WEIGHT_K_CONTIGUOUS, _DTYPE_CODES[out_dtype], 0, 0, 0,
                         0, 0, 0, 0, 0, 0)
    v = _lib.Variant()
    _lib.call("afhip_gemm_calibrate", ctypes.byref(desc), ctypes.byref(v))
    return GemmVariant._from_c(v)


def force_variant(variant: GemmVariant | None) -> None:
    """forceGemmVariant (gemm-selection.ts:122-125): pin for every later plan."""
    if variant is None:
        _lib.call("afhip_gemm_force_variant", None)
    else:
        c = variant._to_c()
        _lib.call("afhip_gemm_force_variant", ctypes.byref(c))


def calibration_load(path: str) -> None:
    _lib.call("afhip_calibration_load", path.encode())


def calibration_save(path: str) -> None:
    _lib.call("afhip_calibration_save", path.encode())


def calibration_clear() -> None:
    """Forgets every calibrated answer this process holds."""
    _lib.call("afhip_calibration_clear")


CALIBRATION_FAULTS = {"none": 0, "run": 1, "result": 2, "last-batch": 3}


def calibration_inject(kernel: str, tile_rows: int, tile_columns: int, fault: str) -> None:
    """Forces a fault on one calibration candidate from the host: "run" (it
    counts as failing to run and is dropped), "result" (its result reads 5%
    off and is refused) or "none"; kernel "all" with fault "none" clears
    every fault. For tests of the calibration's failure handling."""
    code = -1 if kernel == "all" else _KERNEL_CODES[kernel]
    _lib.call("afhip_calibration_inject", code, tile_rows, tile_columns, CALIBRATION_FAULTS[fault])


def pack_weight(w, precision: str = "f32"):
    """[K][N] device weight -> [N][K] in the precision's dtype (int8 stays int8):
    the counterpart of packWeights (src/triangle/weights.ts:20-34)."""
    import torch

    K, N = w.shape
    src = _code_of(w)
    dst = "i8" if src == "i8" else ("f16" if precision == "f16" else "f32")
    out = torch.empty((N, K), dtype=_torch_dtype(dst), device=device())
    _lib.call("afhip_pack_weight", ptr(w), _DTYPE_CODES[src], K, N, ptr(out), _DTYPE_CODES[dst], stream_handle())
    return out


def linear(x, w, bias=None, *, relu: bool = False, residual=None, precision: str = "f32", out_dtype=None,
           w_layout: str = "column"):
    """createLinearShader (src/evoformer/transition.ts:91-138): A . W + bias,
    ReLU when asked, added into `residual` when given (which is also the
    output, as the reference's += store is)."""
    rows, inner = x.shape
    columns = w.shape[1] if w_layout == "column" else w.shape[0]
    epi = []
    if bias is not None:
        epi.append("bias")
    if relu:
        epi.append("relu")
    if residual is not None:
        epi.append("residual")
    out_code = out_dtype or (_code_of(residual) if residual is not None else "f32")
    plan = TiledGemm(rows, inner, columns, precision=precision, a_dtype=_code_of(x), w_dtype=_code_of(w),
                     w_layout=w_layout, out_dtype=out_code, epilogue=epi)
    return plan.run(x, w, bias=bias, residual=residual, out=residual)


def attention_project(x, w, *, heads: int, head_dim: int, scale=None, gate_bias=None, out_dtype: str = "f16",
                      w_layout: str = "column"):
    """The fused q/k/v/gate projection (src/evoformer/attention.ts:497-589):
    W holds [q | k | v | g] as columns; q is scaled by 1/sqrt(head_dim) and
    g = sigmoid(x + gate_bias). An int8 W takes a per-column f32 `scale`
    (mixed-q8, dequantised in the epilogue). Returns (q, k, v, g) views of
    one [M][4*H*D] output."""
    import torch

    rows, inner = x.shape
    hd = heads * head_dim
    columns = 4 * hd
    epi = []
    if scale is not None:
        epi.append("scale")
    bias = None
    if gate_bias is not None:
        bias = torch.zeros(columns, dtype=torch.float32, device=device())
        bias[3 * hd:] = gate_bias
        epi.append("bias")
    epi.append("attention")
    precision = "f16" if _code_of(w) in ("f16", "i8") or _code_of(x) == "f16" else "f32"
    plan = TiledGemm(rows, inner, columns, precision=precision, a_dtype=_code_of(x), w_dtype=_code_of(w),
                     w_layout=w_layout, out_dtype=out_dtype, epilogue=epi, heads=heads, head_dim=head_dim)
    out = plan.run(x, w, scale=scale, bias=bias)
    return out[:, :hd], out[:, hd:2 * hd], out[:, 2 * hd:3 * hd], out[:, 3 * hd:]


def dequant_q8_channel(q, scale):
    """w[k][n] = f32(q[k][n]) * scale[n], on the device."""
    import torch

    K, N = q.shape
    out = torch.empty((K, N), dtype=torch.float32, device=device())
    _lib.call("afhip_dequant_q8_channel", ptr(q), ptr(scale), K, N, ptr(out), stream_handle())
    return out


def pack_weight_q8_block(codes, scales_f16_bits, rows_k: int, columns_n: int, *, block: int = 64, start: int = 0,
                         dtype: str = "f16"):
    """The bundle's mixed-q8 weight [rows_k][columns_n] (flat from element
    `start` of `codes`) decoded on the device straight into the packed GEMM
    operand W[n][k] of `dtype` (readTensorRange's int8 branch,
    src/reference/dtype.ts:66-99, without the f32 copy). Use it with a plan of
    w_dtype `dtype` and w_layout "k"."""
    import torch

    if rows_k <= 0 or columns_n <= 0:
        raise _lib.RangeError("weight dimensions must be positive")
    if block <= 0:
        raise _lib.RangeError("int8 tensor has an invalid block size")
    if start < 0 or start + rows_k * columns_n > codes.numel():
        raise _lib.RangeError("tensor range is out of bounds")
    if (start + rows_k * columns_n - 1) // block >= scales_f16_bits.numel():
        raise _lib.RangeError("int8 tensor has too few scales")
    out = torch.empty((columns_n, rows_k), dtype=torch.float16 if dtype == "f16" else torch.float32,
                      device=device())
    _lib.call("afhip_pack_weight_q8_block", ptr(codes), ptr(scales_f16_bits), block, start, rows_k, columns_n,
              ptr(out), _lib.F16 if dtype == "f16" else _lib.F32, stream_handle())
    return out


def dequant_q8_block(codes, scales_f16_bits, block: int = 64, start: int = 0, count: int | None = None):
    """readTensorRange's int8 branch (src/reference/dtype.ts:66-99) on the device."""
    import torch

    total = codes.numel()
    if count is None:
        count = total - start
    if start < 0 or count < 0 or start + count > total:
        raise _lib.RangeError("tensor range is out of bounds")
    out = torch.empty(count, dtype=torch.float32, device=device())
    _lib.call("afhip_dequant_q8_block", ptr(codes), ptr(scales_f16_bits), block, start, count, ptr(out),
              stream_handle())
    return out
