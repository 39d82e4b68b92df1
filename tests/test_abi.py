"""The C ABI on the CPU: the library loads, exports every symbol
include/afhip.h declares, and its host-only logic (the reference's gemmGrid,
the selection record, validation) behaves without a GPU."""
import os
import re

import pytest

from conftest import ROOT


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "afhip.h")).read()
    return sorted(set(re.findall(r"AFHIP_API\s+(?:const\s+char\*|int)\s+(afhip_\w+)\s*\(", text)))


def test_header_declares_the_surface():
    names = declared_symbols()
    assert len(names) >= 38
    for needed in ("afhip_gemm_run", "afhip_triangle_run", "afhip_opm_run", "afhip_transition_run",
                   "afhip_gemm_calibrate", "afhip_dequant_q8_channel"):
        assert needed in names


def test_library_exports_every_declared_symbol():
    from afhip import _lib

    lib = _lib.library()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert missing == []
    assert set(declared_symbols()) <= set(_lib.SIGNATURES)


def test_abi_version_and_not_open_errors():
    import ctypes

    from afhip import _lib

    lib = _lib.library()
    assert lib.afhip_abi_version() == 3
    size = ctypes.c_size_t()
    # A call that needs the device reports NOT_OPEN rather than touching HIP.
    assert lib.afhip_buffer_create(16, ctypes.byref(ctypes.c_void_p())) == _lib.ERR_NOT_OPEN
    assert "afhip_open" in _lib.last_error()
    desc = _lib.TriangleDesc(384, 128, 128, 0, 1, 1, 0, 0, 0, 1e-5)
    assert lib.afhip_triangle_workspace_size(ctypes.byref(desc), ctypes.byref(size)) == _lib.OK
    # a, b (f16, channel-major) and the contracted block: 3 x 128 x 147456 x 2 bytes
    assert size.value >= 3 * 128 * 147456 * 2
    # The pair transition at f16 precision runs fused: no workspace. At f32 it
    # needs the normalised rows and the hidden activation.
    tdesc = _lib.TransitionDesc(1 << 20, 128, 512, 1, 1, 1, 1, 1e-5)
    assert lib.afhip_transition_workspace_size(ctypes.byref(tdesc), ctypes.byref(size)) == _lib.OK
    assert size.value == 0
    tdesc.precision = 0
    assert lib.afhip_transition_workspace_size(ctypes.byref(tdesc), ctypes.byref(size)) == _lib.OK
    assert size.value >= (1 << 20) * (128 + 512) * 4
    # The execution layer needs the device as well.
    handle = ctypes.c_void_p()
    assert lib.afhip_execution_create(0, None, ctypes.byref(handle)) == _lib.ERR_NOT_OPEN


def test_gemm_grid_matches_reference():
    # test/gemm-selection.test.ts:239-262 and test/gemm.test.ts:57-61
    from afhip import _lib, gemm

    assert gemm.gemm_grid(64, 128) == (1, 1)
    assert gemm.gemm_grid(65, 129) == (2, 2)
    assert gemm.gemm_grid(65_535 * 64, 256) == (2, 65_535)
    assert gemm.gemm_grid(256, 128) == (1, 4)
    assert gemm.gemm_grid(256, 128, 128, 128) == (1, 2)
    rows = 65_536 * 64
    x, y = gemm.gemm_grid(rows, 128)
    assert x <= 65_535 and y <= 65_535 and x * y >= rows // 64
    for bad in [(0, 1), (1, 0), (-3, 4)]:
        with pytest.raises(_lib.RangeError):
            gemm.gemm_grid(*bad)


def test_triangle_fast_path_bounds():
    # Which triangle shapes take the persistent f16 kernels, decided on the
    # host: AlphaFold's widths at f16 precision, any length whose operands
    # fit, except an incoming z past 4 GiB (read with 32-bit lane offsets).
    import ctypes

    from afhip import _lib

    lib = _lib.library()

    def fast(length, direction=0, pair=1, cz=128, precision=1):
        flag = ctypes.c_int32(-1)
        desc = _lib.TriangleDesc(length, cz, 128, direction, precision, pair, 0, 0, 0, 1e-5)
        assert lib.afhip_triangle_fast_path(ctypes.byref(desc), ctypes.byref(flag)) == _lib.OK
        return flag.value

    assert fast(384) == 1 and fast(384, direction=1) == 1
    assert fast(3072) == 1 and fast(3072, direction=1) == 1 and fast(3300, direction=1) == 1
    assert fast(4095, direction=1) == 1 and fast(4096, direction=1) == 0 and fast(4096) == 1
    assert fast(3072, pair=0) == 1 and fast(3072, direction=1, pair=0) == 0 and fast(2896, direction=1, pair=0) == 1
    assert fast(384, cz=64) == 0 and fast(384, precision=0) == 0
    # At L = 3072 the output kernels' blocks of rows shrink so their buffer
    # offsets stay below 2 GiB: the contracted block is smaller than all rows.
    size = ctypes.c_size_t()
    desc = _lib.TriangleDesc(3072, 128, 128, 0, 1, 1, 0, 0, 0, 1e-5)
    assert lib.afhip_triangle_workspace_size(ctypes.byref(desc), ctypes.byref(size)) == _lib.OK
    full = 128 * 3072 * 3072 * 2
    assert 2 * full <= size.value < 3 * full


def test_descriptor_validation_is_host_side():
    import ctypes

    from afhip import _lib

    lib = _lib.library()
    size = ctypes.c_size_t()
    bad = _lib.TriangleDesc(0, 128, 128, 0, 1, 1, 0, 0, 0, 1e-5)
    assert lib.afhip_triangle_workspace_size(ctypes.byref(bad), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    assert "positive" in _lib.last_error()
    bad = _lib.TriangleDesc(8, 128, 128, 2, 1, 1, 0, 0, 0, 1e-5)
    assert lib.afhip_triangle_workspace_size(ctypes.byref(bad), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    bad = _lib.TriangleDesc(8, 128, 128, 0, 1, 1, 0, 0, 0, -1.0)
    assert lib.afhip_triangle_workspace_size(ctypes.byref(bad), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    opm = _lib.OpmDesc(512, 256, 256, 32, 128, 1, 1, 0, 0, 0, 1e-5, 1e-3)
    assert lib.afhip_opm_workspace_size(ctypes.byref(opm), ctypes.byref(size)) == _lib.OK
    tr = _lib.TransitionDesc(0, 128, 512, 1, 1, 0, 0, 1e-5)
    assert lib.afhip_transition_workspace_size(ctypes.byref(tr), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    # attention: validate (src/evoformer/attention.ts:102-141) and the pair bias sources
    att = _lib.AttentionDesc(64, 64, 128, 4, 0, _lib.PAIR_BIAS_NORMALIZED_INPUT, 0, 1, 1, 1, 1, 1e-5)
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.OK
    assert lib.afhip_attention_weights_size(ctypes.byref(att), ctypes.byref(size)) == _lib.OK
    att.heads = 3
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    assert "head dimension no larger than 32" in _lib.last_error()
    att.heads, att.channels = 2, 128  # head dimension 64
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    att.heads, att.batch = 4, 63
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    assert "batch == queries" in _lib.last_error()
    att.pair_bias = _lib.PAIR_BIAS_SEPARATE
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    assert "pair channels" in _lib.last_error()
    att.pair_channels = 128
    assert lib.afhip_attention_workspace_size(ctypes.byref(att), ctypes.byref(size)) == _lib.OK
    assert lib.afhip_attention_run(ctypes.byref(att), None, None, None, None, None, None, 0,
                                   None) == _lib.ERR_NOT_OPEN


def test_variant_selection_without_device():
    from afhip import gemm

    # BASELINE config 2 (tall, K = 256, int8 weights, f16 out) streams past
    # register-resident weights; with an f32 output it takes the LDS_DMA
    # family, its plan widening the int8 weight to f16 first; so does the
    # reference's trans2 shape (K = 1024) with int8 weights.
    v = gemm.select_variant(131072, 256, 1024, precision="f16", a_dtype="f16", w_dtype="i8", out_dtype="f16")
    assert (v.kernel, v.tile_rows, v.tile_columns, v.source) == ("stream", 64, 512, "heuristic")
    assert v.name == "mfma-stream-f16-64x512k32"
    v = gemm.select_variant(131072, 256, 1024, precision="f16", a_dtype="f16", w_dtype="i8", out_dtype="f32")
    assert v.kernel == "lds_dma" and v.source == "heuristic"
    assert gemm.select_variant(29972, 1024, 256, precision="f16", a_dtype="f16", w_dtype="i8",
                               out_dtype="f16").kernel == "lds_dma"
    # An odd K stays on the register-staged kernel (no 4-byte chunk holds it).
    assert gemm.select_variant(100, 33, 64, precision="f16", a_dtype="f16", w_dtype="f16").kernel == "register"
    # f16 operands on both sides take the LDS_DMA family; the triangle
    # contraction at L = 384 (128 channels) tiles 192 x 192, two per CU.
    v = gemm.select_variant(384, 384, 384, precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16",
                            batch=128)
    assert (v.kernel, v.tile_rows, v.tile_columns) == ("lds_dma", 192, 192)
    v = gemm.select_variant(81, 256, 132, precision="f16", a_dtype="f16", w_dtype="f16")
    assert (v.kernel, v.tile_rows, v.tile_columns) == ("lds_dma", 128, 128)
    # Long K on large outputs (the L = 1024 contraction) takes 256 x 256, the
    # L = 512 one 128 x 256; the outer-product-mean contraction
    # (8192 x 512 x 8192) 192 x 192 with its 0.8% ragged edge; its narrow
    # output GEMM stays on 128 x 128.
    v = gemm.select_variant(1024, 1024, 1024, precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16",
                            batch=128)
    assert (v.kernel, v.tile_rows, v.tile_columns) == ("lds_dma", 256, 256)
    v = gemm.select_variant(512, 512, 512, precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16",
                            batch=128)
    assert (v.kernel, v.tile_rows, v.tile_columns) == ("lds_dma", 128, 256)
    v = gemm.select_variant(8192, 512, 8192, precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16")
    assert (v.tile_rows, v.tile_columns) == (192, 192)
    v = gemm.select_variant(65536, 1024, 128, precision="f16", a_dtype="f16", w_dtype="f16")
    assert (v.tile_rows, v.tile_columns) == (128, 128)
    # The reference's SHAPES (tools/gemm-candidates.ts:637-669), as measured
    # by bench.py --gemm-shapes: STREAM from ~16k rows only; a K that is even
    # but not a multiple of 8 (opm-contract, K = 508) takes LDS_DMA with
    # 4-byte loads, on 128 x 128 tiles.
    f16 = dict(precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16")
    assert gemm.select_variant(29972, 256, 1024, **f16).kernel == "stream"
    assert gemm.select_variant(8192, 128, 512, **f16).kernel == "lds_dma"
    v = gemm.select_variant(128, 508, 32000, **f16)
    assert v.kernel == "lds_dma"


def test_plan_variant_names_the_family_that_runs():
    # afhip_gemm_select on a whole description (no device): where its
    # layouts, strides, K or M rule the selected family out, the variant is
    # the one the run falls back to, so it names the kernel family that runs.
    import ctypes

    from afhip import _lib, gemm

    def select(rows, inner, columns, a_dtype=1, w_layout=_lib.WEIGHT_K_CONTIGUOUS, w_dtype=1, out_dtype=1,
               epilogue=0, lda=0, sa=0, batch=1, a_layout=_lib.SOURCE_K_CONTIGUOUS, c_layout=_lib.OUTPUT_ROW_MAJOR):
        desc = _lib.GemmDesc(rows, inner, columns, batch, 1, a_dtype, w_dtype, w_layout, out_dtype, epilogue, 0, 0,
                             lda, 0, 0, sa, 0, rows * columns, a_layout, c_layout)
        v = _lib.Variant()
        _lib.call("afhip_gemm_select", ctypes.byref(desc), ctypes.byref(v))
        return gemm.GemmVariant._from_c(v).kernel

    row = dict(a_layout=_lib.SOURCE_ROW_CONTIGUOUS)
    # A row-contiguous source on LDS_DMA needs whole 16-byte chunks of m.
    assert select(4096, 256, 4096, **row) == "lds_dma"
    assert select(4090, 256, 4096, lda=4096, **row) == "register"
    assert select(4096, 256, 4096, lda=4100, **row) == "register"
    # An f32 source needs 16-byte rows (lda a multiple of 4) and K % 8 == 0.
    assert select(4096, 256, 4096, a_dtype=0) == "lds_dma"
    assert select(4096, 256, 4096, a_dtype=0, lda=258) == "register"
    assert select(4096, 252, 4096, a_dtype=0) == "register"
    # An f32 [K][N] weight under f16 precision is converted into the
    # workspace and takes the f16 families.
    assert select(4096, 256, 4096, w_dtype=0, w_layout=_lib.WEIGHT_COLUMN_CONTIGUOUS) == "lds_dma"
    # STREAM shapes with what STREAM does not take: a residual, a
    # column-major output, a row-contiguous source.
    assert select(29972, 256, 1024) == "stream"
    assert select(29972, 256, 1024, epilogue=_lib.EPILOGUE_RESIDUAL) == "lds_dma"
    assert select(29972, 256, 1024, c_layout=_lib.OUTPUT_COLUMN_MAJOR) == "lds_dma"
    assert select(29976, 256, 1024, **row) == "lds_dma"
    # f32 arithmetic (precision 0): LDS_DMA for k-contiguous f32 operands
    # with K and lda multiples of 4; otherwise register-staged (and the
    # variant a refused LDS_DMA selection falls back to is register-staged).
    def select32(rows, inner, columns, **kw):
        desc = _lib.GemmDesc(rows, inner, columns, 1, 0, 0, 0, _lib.WEIGHT_K_CONTIGUOUS, 0, 0, 0, 0,
                             kw.get("lda", 0), 0, 0, 0, 0, rows * columns, kw.get("a_layout", 0), 0)
        v = _lib.Variant()
        _lib.call("afhip_gemm_select", ctypes.byref(desc), ctypes.byref(v))
        return gemm.GemmVariant._from_c(v).kernel

    assert select32(4096, 128, 512) == "lds_dma"
    assert select32(4096, 98, 512) == "register"
    assert select32(4096, 128, 512, lda=130) == "register"
    assert select32(4096, 128, 512, a_layout=_lib.SOURCE_ROW_CONTIGUOUS) == "register"


def test_calibration_document_round_trip(tmp_path):
    from afhip import gemm

    path = tmp_path / "calibration.json"
    gemm.calibration_save(str(path))
    text = path.read_text()
    assert '"schema": 1' in text
    # A corrupted document is ignored, not trusted (gemm-selection.ts:543-558).
    path.write_text('{"schema": 1, "entries": {"x|y": {"precision": 1, "tile_rows": 96, '
                    '"tile_columns": 128, "tile_inner": 32}}}')
    gemm.calibration_load(str(path))
    shape = dict(precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16", batch=1)
    assert gemm.select_variant(200, 96, 128, **shape).source == "heuristic"
    path.write_text("not json at all")
    gemm.calibration_load(str(path))
    assert gemm.select_variant(200, 96, 128, **shape).source == "heuristic"
    assert gemm.select_variant(384, 384, 384, **dict(shape, batch=128)).tile_rows == 192
