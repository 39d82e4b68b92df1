"""ctypes binding of libafhip.so (include/afhip.h).

The library is the product; this module only declares its signatures and
turns status codes into exceptions. There is no fallback: if libafhip.so is
missing or cannot be loaded, every call raises AfhipUnavailable.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libafhip.so")

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_OUT_OF_MEMORY = -2
ERR_HIP = -3
ERR_UNSUPPORTED = -4
ERR_NOT_OPEN = -5

F32, F16, I8 = 0, 1, 2
PRECISION_F32, PRECISION_F16 = 0, 1

EPILOGUE_SCALE = 1
EPILOGUE_BIAS = 2
EPILOGUE_ATTENTION = 4
EPILOGUE_RELU = 8
EPILOGUE_RESIDUAL = 16

WEIGHT_COLUMN_CONTIGUOUS = 0
WEIGHT_K_CONTIGUOUS = 1

SOURCE_K_CONTIGUOUS = 0
SOURCE_ROW_CONTIGUOUS = 1

OUTPUT_ROW_MAJOR = 0
OUTPUT_COLUMN_MAJOR = 1

KERNEL_REGISTER_STAGED = 0
KERNEL_LDS_DMA = 1
KERNEL_STREAM = 2

TRIANGLE_OUTGOING = 0
TRIANGLE_INCOMING = 1

PAIR_BIAS_NONE = 0
PAIR_BIAS_NORMALIZED_INPUT = 1
PAIR_BIAS_SEPARATE = 2


class AfhipUnavailable(RuntimeError):
    """libafhip.so is not built or cannot be loaded; nothing falls back."""


class RangeError(ValueError):
    """A shape, size or argument the library refuses (the reference's RangeError)."""


class AfhipError(RuntimeError):
    """A HIP failure or unsupported request reported by the library."""


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int32), ("inner", ctypes.c_int32), ("columns", ctypes.c_int32),
        ("batch", ctypes.c_int32), ("precision", ctypes.c_int32), ("a_dtype", ctypes.c_int32),
        ("w_dtype", ctypes.c_int32), ("w_layout", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("epilogue", ctypes.c_uint32), ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("lda", ctypes.c_int64), ("ldw", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("batch_stride_a", ctypes.c_int64), ("batch_stride_w", ctypes.c_int64),
        ("batch_stride_c", ctypes.c_int64), ("a_layout", ctypes.c_int32), ("c_layout", ctypes.c_int32),
    ]


class Variant(ctypes.Structure):
    _fields_ = [
        ("precision", ctypes.c_int32), ("tile_rows", ctypes.c_int32), ("tile_columns", ctypes.c_int32),
        ("tile_inner", ctypes.c_int32), ("vectorized", ctypes.c_int32), ("source", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
    ]


class TriangleDesc(ctypes.Structure):
    _fields_ = [
        ("length", ctypes.c_int32), ("c_z", ctypes.c_int32), ("c_hidden", ctypes.c_int32),
        ("direction", ctypes.c_int32), ("precision", ctypes.c_int32), ("pair_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32), ("block_rows", ctypes.c_int32), ("residual", ctypes.c_int32),
        ("epsilon", ctypes.c_float),
    ]


class OpmDesc(ctypes.Structure):
    _fields_ = [
        ("sequences", ctypes.c_int32), ("length", ctypes.c_int32), ("c_m", ctypes.c_int32),
        ("c_outer", ctypes.c_int32), ("c_z", ctypes.c_int32), ("precision", ctypes.c_int32),
        ("msa_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32), ("row_block", ctypes.c_int32),
        ("residual", ctypes.c_int32), ("layer_norm_epsilon", ctypes.c_float),
        ("normalization_epsilon", ctypes.c_float),
    ]


class TransitionDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int64), ("channels", ctypes.c_int32), ("hidden", ctypes.c_int32),
        ("precision", ctypes.c_int32), ("in_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("residual", ctypes.c_int32), ("epsilon", ctypes.c_float),
    ]


class AttentionDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("queries", ctypes.c_int32), ("channels", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("transpose", ctypes.c_int32), ("pair_bias", ctypes.c_int32),
        ("pair_channels", ctypes.c_int32), ("precision", ctypes.c_int32), ("in_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32), ("residual", ctypes.c_int32), ("epsilon", ctypes.c_float),
    ]


class PairStackDesc(ctypes.Structure):
    _fields_ = [("opm", OpmDesc), ("outgoing", TriangleDesc), ("incoming", TriangleDesc),
                ("attention_start", AttentionDesc), ("attention_end", AttentionDesc), ("transition", TransitionDesc)]


class PairStackWeights(ctypes.Structure):
    _fields_ = [("opm", ctypes.c_void_p), ("outgoing", ctypes.c_void_p), ("incoming", ctypes.c_void_p),
                ("attention_start", ctypes.c_void_p), ("attention_end", ctypes.c_void_p),
                ("transition", ctypes.c_void_p)]


class EvoformerBlockDesc(ctypes.Structure):
    _fields_ = [("msa_row", AttentionDesc), ("msa_column", AttentionDesc), ("msa_transition", TransitionDesc),
                ("pair", PairStackDesc), ("opm_first", ctypes.c_int32)]


class EvoformerBlockWeights(ctypes.Structure):
    _fields_ = [("msa_row", ctypes.c_void_p), ("msa_column", ctypes.c_void_p), ("msa_transition", ctypes.c_void_p),
                ("pair", PairStackWeights)]


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_szp = ctypes.POINTER(ctypes.c_size_t)

# name -> (argtypes); every function returns int status unless listed in _RESTYPES.
SIGNATURES = {
    "afhip_last_error": [],
    "afhip_abi_version": [],
    "afhip_open": [ctypes.c_int],
    "afhip_close": [],
    "afhip_device_report": [ctypes.c_char_p, _sz],
    "afhip_buffer_create": [_sz, ctypes.POINTER(_vp)],
    "afhip_buffer_destroy": [_vp],
    "afhip_buffer_write": [_vp, _sz, _vp, _sz],
    "afhip_buffer_read": [_vp, _sz, _vp, _sz],
    "afhip_synchronize": [_vp],
    "afhip_gemm_plan_create": [ctypes.POINTER(GemmDesc), ctypes.POINTER(_vp)],
    "afhip_gemm_plan_destroy": [_vp],
    "afhip_gemm_workspace_size": [_vp, _szp],
    "afhip_gemm_run": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "afhip_gemm_run_static": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "afhip_gemm_static_scratch_bytes": [_szp],
    "afhip_gemm_grid": [_i64, _i64, _i32, _i32, ctypes.POINTER(ctypes.c_uint32)],
    "afhip_gemm_select": [ctypes.POINTER(GemmDesc), ctypes.POINTER(Variant)],
    "afhip_gemm_calibrate": [ctypes.POINTER(GemmDesc), ctypes.POINTER(Variant)],
    "afhip_gemm_force_variant": [ctypes.POINTER(Variant)],
    "afhip_calibration_load": [ctypes.c_char_p],
    "afhip_calibration_save": [ctypes.c_char_p],
    "afhip_calibration_clear": [],
    "afhip_calibration_inject": [_i32, _i32, _i32, _i32],
    "afhip_pack_weight": [_vp, _i32, _i32, _i32, _vp, _i32, _vp],
    "afhip_dequant_q8_channel": [_vp, _vp, _i32, _i32, _vp, _vp],
    "afhip_dequant_q8_block": [_vp, _vp, _i32, _i64, _i64, _vp, _vp],
    "afhip_pack_weight_q8_block": [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp],
    "afhip_triangle_weights_size": [ctypes.POINTER(TriangleDesc), _szp],
    "afhip_triangle_workspace_size": [ctypes.POINTER(TriangleDesc), _szp],
    "afhip_triangle_fast_path": [ctypes.POINTER(TriangleDesc), ctypes.POINTER(ctypes.c_int32)],
    "afhip_triangle_prepare_weights": [ctypes.POINTER(TriangleDesc), _vp, _vp, _vp],
    "afhip_triangle_run": [ctypes.POINTER(TriangleDesc), _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "afhip_opm_weights_size": [ctypes.POINTER(OpmDesc), _szp],
    "afhip_opm_workspace_size": [ctypes.POINTER(OpmDesc), _szp],
    "afhip_opm_prepare_weights": [ctypes.POINTER(OpmDesc), _vp, _vp, _vp],
    "afhip_opm_run": [ctypes.POINTER(OpmDesc), _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "afhip_transition_weights_size": [ctypes.POINTER(TransitionDesc), _szp],
    "afhip_transition_workspace_size": [ctypes.POINTER(TransitionDesc), _szp],
    "afhip_transition_prepare_weights": [ctypes.POINTER(TransitionDesc), _vp, _vp, _vp],
    "afhip_transition_run": [ctypes.POINTER(TransitionDesc), _vp, _vp, _vp, _vp, _sz, _vp],
    "afhip_attention_weights_size": [ctypes.POINTER(AttentionDesc), _szp],
    "afhip_attention_workspace_size": [ctypes.POINTER(AttentionDesc), _szp],
    "afhip_attention_prepare_weights": [ctypes.POINTER(AttentionDesc), _vp, _vp, _vp],
    "afhip_attention_run": [ctypes.POINTER(AttentionDesc), _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "afhip_set_memory_budget": [ctypes.c_uint64],
    "afhip_memory_resident": [ctypes.POINTER(ctypes.c_uint64)],
    "afhip_execution_create": [ctypes.c_uint64, _vp, ctypes.POINTER(_vp)],
    "afhip_execution_destroy": [_vp],
    "afhip_execution_allocate": [_vp, ctypes.c_char_p, ctypes.c_uint64, ctypes.POINTER(_vp)],
    "afhip_execution_upload": [_vp, ctypes.c_char_p, _vp, ctypes.c_uint64, ctypes.POINTER(_vp)],
    "afhip_execution_release": [_vp, _vp],
    "afhip_execution_checkpoint": [_vp, ctypes.POINTER(ctypes.c_uint64)],
    "afhip_execution_release_since": [_vp, ctypes.c_uint64],
    "afhip_execution_note_submitted": [_vp],
    "afhip_execution_snapshot": [_vp, ctypes.c_char_p, _sz],
    "afhip_execution_add_in_place": [_vp, _vp, _i32, _vp, _i32, _i64],
    "afhip_execution_pair_stack": [_vp, ctypes.POINTER(PairStackDesc), ctypes.POINTER(PairStackWeights), _vp, _vp,
                                   _vp, _vp],
    "afhip_execution_evoformer_block": [_vp, ctypes.POINTER(EvoformerBlockDesc), ctypes.POINTER(EvoformerBlockWeights),
                                        _vp, _vp, _vp, _vp],
    "afhip_timing_enable": [ctypes.c_int],
    "afhip_timing_reset": [],
    "afhip_timing_report": [ctypes.c_char_p, _sz],
}
_RESTYPES = {"afhip_last_error": ctypes.c_char_p}

_lib = None


def library() -> ctypes.CDLL:
    """The loaded libafhip.so, with every signature declared."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AfhipUnavailable(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C alphafold2-webgpu_amd). "
            "afhip has no CPU fallback.")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the host
        raise AfhipUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            # A symbol the header declares but this build lacks fails when
            # called, not at load; tests/test_abi.py requires all of them.
            continue
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def last_error() -> str:
    return library().afhip_last_error().decode("utf-8", "replace")


def check(status: int, what: str = "") -> None:
    if status == OK:
        return
    message = last_error()
    prefix = f"{what}: " if what else ""
    if status == ERR_INVALID_ARGUMENT:
        raise RangeError(prefix + message)
    raise AfhipError(f"{prefix}{message} (status {status})")


def call(name: str, *args) -> None:
    fn = getattr(library(), name, None)
    if fn is None:
        raise AfhipUnavailable(f"{LIB_PATH} does not export {name}")
    check(fn(*args), name)
