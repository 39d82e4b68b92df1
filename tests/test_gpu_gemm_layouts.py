"""Operand and output layouts of the GEMM plan against float64.

The reference checks its staged kernel on every pairing of a row-contiguous
source and a k-contiguous weight (test/gemm-matrix-units.gpu.test.ts:80-170:
130 x 96 x 132, LCG operands, max|d|/max|ref| < 4e-3 for the f16 units).
These are the same cases through afhip_gemm_desc's a_layout and w_layout,
plus the column-major output (the reference's column-major matrixEpilogue,
src/runtime/gemm.ts:268-285) and the outer-product mean's contraction
written as a plan, both operands sequence-major as
src/evoformer/outer-product-mean.ts:376-389 describes them.
"""
import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu

TILES = [(64, 64), (64, 128), (128, 64), (128, 128)]


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def rel_max(actual, expected):
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def to_dev(x, dev, half=False):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t.half() if half else t


@pytest.mark.parametrize("precision,tol", [("f32", 1e-5), ("f16", 4e-3)])
@pytest.mark.parametrize("source,weight", [("k", "column"), ("row", "column"), ("k", "k"), ("row", "k")])
def test_reference_layout_cases(dev, precision, tol, source, weight):
    # gemm-matrix-units.gpu.test.ts:84-89, :99-102, :155-168: the operands are
    # written transposed when the layout says so, and every tile of the
    # family that takes a row-contiguous source computes the same product.
    from afhip import gemm

    rows, inner, columns = 130, 96, 132
    source_values = ref.lcg_values(0x2244668, rows * inner)
    weight_values = ref.lcg_values(0x1133557, inner * columns)
    a = source_values.reshape(inner, rows).T if source == "row" else source_values.reshape(rows, inner)
    w = weight_values.reshape(columns, inner).T if weight == "k" else weight_values.reshape(inner, columns)
    if precision == "f16":
        a, w = ref.round_f16(a), ref.round_f16(w)
    expect = a.astype(np.float64) @ w.astype(np.float64)
    a_stored = source_values.reshape(inner, rows) if source == "row" else source_values.reshape(rows, inner)
    w_stored = weight_values.reshape(columns, inner) if weight == "k" else weight_values.reshape(inner, columns)
    dtype = precision
    # a k-contiguous weight is given in the precision's dtype (the plan rule)
    ad = to_dev(a_stored, dev, half=dtype == "f16")
    wd = to_dev(w_stored, dev, half=dtype == "f16")
    for tr, tc in TILES:
        gemm.force_variant(gemm.GemmVariant(precision, tr, tc, source="pinned"))
        try:
            plan = gemm.TiledGemm(rows, inner, columns, precision=precision, a_dtype=dtype, w_dtype=dtype,
                                  w_layout=weight, out_dtype="f32", a_layout=source)
            assert plan.variant().kernel == "register"
            out = plan.run(ad, wd).cpu().numpy()
        finally:
            gemm.force_variant(None)
        assert rel_max(out, expect) <= tol, (tr, tc)


@pytest.mark.parametrize("out_dtype", ["f32", "f16"])
def test_row_contiguous_source_column_major_output_epilogue(dev, out_dtype):
    # A batched plan with A stored [K][M] (ragged M whose rows are padded to
    # 136, so the 16-byte loads run and the last chunk of each k-row is
    # guarded) and C stored [N][M], through bias, ReLU and residual. An M
    # that is not a multiple of 8 leaves LDS_DMA's whole-chunk k rows, so the
    # plan names, and runs, the register-staged kernel.
    import torch

    from afhip import gemm

    B, M, K, N, lda = 3, 130, 72, 100, 136
    a_stored = ref.round_f16(ref.normal(101, (B, K, lda)))
    w = ref.round_f16(ref.normal(102, (B, N, K), 1 / K))
    bias = ref.normal(103, (N,), 0.1)
    residual = ref.round_f16(ref.normal(104, (B, N, M)))
    a = np.transpose(a_stored[:, :, :M], (0, 2, 1))
    expect = np.einsum("bmk,bnk->bmn", a.astype(np.float64), w.astype(np.float64)) + bias
    expect = np.maximum(expect, 0) + np.transpose(residual, (0, 2, 1))
    plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k", out_dtype=out_dtype,
                          epilogue=("bias", "relu", "residual"), batch=B, lda=lda, batch_stride_a=K * lda,
                          batch_stride_w=N * K, batch_stride_c=N * M, a_layout="row", c_layout="column")
    assert plan.variant().kernel == "register"
    res = to_dev(residual, dev).to(torch.float32 if out_dtype == "f32" else torch.float16)
    out = plan.run(to_dev(a_stored, dev, half=True), to_dev(w, dev, half=True), bias=to_dev(bias, dev),
                   residual=res, out=res.clone())
    got = np.transpose(out.float().cpu().numpy(), (0, 2, 1))
    assert rel_max(got, expect) <= (4e-3 if out_dtype == "f32" else 1e-2)


LDS_DMA_TILES = [(128, 128), (192, 192), (128, 256), (256, 256)]


@pytest.mark.parametrize("out_dtype", ["f32", "f16"])
@pytest.mark.parametrize("K,epilogue", [(104, ()), (104, ("bias", "relu", "residual")), (98, ("bias", "residual"))])
def test_column_major_output_on_lds_dma_matches_register_kernel(dev, out_dtype, K, epilogue):
    # A column-major output (C stored [N][M], the reference's column-major
    # matrixEpilogue) on the LDS_DMA family: its tiles leave through each
    # wave's LDS square with the lanes along m, applying the register-staged
    # kernel's epilogue steps: the same bits on every tile, a batch of two with
    # ragged M and N, and rows only 4-byte aligned at K = 98.
    import torch

    from afhip import gemm

    B, M, N = 2, 333, 200
    a = ref.round_f16(ref.normal(131, (B, M, K)))
    w = ref.round_f16(ref.normal(132, (B, N, K), 1 / K))
    bias = to_dev(ref.normal(133, (N,), 0.1), dev)
    tdt = torch.float16 if out_dtype == "f16" else torch.float32
    start = to_dev(ref.round_f16(ref.normal(134, (B, N, M))), dev).to(tdt)
    ad, wd = to_dev(a, dev, half=True), to_dev(w, dev, half=True)
    results = {}
    for kernel, tiles in (("register", [(128, 128)]), ("lds_dma", LDS_DMA_TILES)):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                                      out_dtype=out_dtype, epilogue=epilogue, batch=B, batch_stride_a=M * K,
                                      batch_stride_w=N * K, batch_stride_c=N * M, c_layout="column")
                assert plan.variant().kernel == kernel
                out = start.clone()
                kw = {}
                if "bias" in epilogue:
                    kw["bias"] = bias
                if "residual" in epilogue:
                    kw["residual"] = out
                results[(kernel, tr, tc)] = plan.run(ad, wd, out=out, **kw).float().cpu().numpy()
            finally:
                gemm.force_variant(None)
    base = results[("register", 128, 128)]
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), key
    expect = np.einsum("bmk,bnk->bnm", a.astype(np.float64), w.astype(np.float64))
    if "bias" in epilogue:
        expect = expect + ref.normal(133, (N,), 0.1)[None, :, None]
    if "relu" in epilogue:
        expect = np.maximum(expect, 0)
    if "residual" in epilogue:
        expect = expect + start.float().cpu().numpy().astype(np.float64)
    assert rel_max(base, expect) <= (4e-3 if out_dtype == "f32" else 1e-2)


@pytest.mark.parametrize("c_layout", ["row", "column"])
@pytest.mark.parametrize("K,epilogue", [(104, ()), (72, ("bias", "relu", "residual")), (40, ("scale", "bias"))])
def test_row_contiguous_source_on_lds_dma_matches_register_kernel(dev, c_layout, K, epilogue):
    # A stored [K][M] (the outer-product mean's and the incoming triangle
    # contraction's sequence- and k-major operands) on the LDS_DMA family,
    # whose stages keep k rows and hand the MFMAs k-contiguous fragments
    # through transposing LDS reads: the same bits as the register-staged
    # kernel on every tile, in a batch of two with M and N ragged against
    # every tile and K not a multiple of the 32-deep k-step. The rows' padding
    # past M holds NaN, which must reach no stored output.
    import torch

    from afhip import gemm

    B, M, N, lda = 2, 200, 300, 216
    sa = K * lda + 64
    rows = np.full((B, K, lda), np.nan, np.float32)
    rows[:, :, :M] = ref.round_f16(ref.normal(141, (B, K, M)))
    a_stored = np.full((B, sa), np.nan, np.float32)
    a_stored[:, :K * lda] = rows.reshape(B, K * lda)
    a = np.transpose(rows[:, :, :M], (0, 2, 1))
    w = ref.round_f16(ref.normal(142, (B, N, K), 1 / K))
    scale = ref.normal(143, (N,), 0.5)
    bias = ref.normal(144, (N,), 0.1)
    cshape = (B, N, M) if c_layout == "column" else (B, M, N)
    start = to_dev(ref.round_f16(ref.normal(145, cshape)), dev)
    ad, wd = to_dev(a_stored, dev, half=True), to_dev(w, dev, half=True)
    results = {}
    for kernel, tiles in (("register", [(128, 128)]), ("lds_dma", LDS_DMA_TILES)):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                                      out_dtype="f32", epilogue=epilogue, batch=B, lda=lda, batch_stride_a=sa,
                                      batch_stride_w=N * K, batch_stride_c=M * N, a_layout="row", c_layout=c_layout)
                assert plan.variant().kernel == kernel
                out = start.clone()
                kw = {}
                if "scale" in epilogue:
                    kw["scale"] = to_dev(scale, dev)
                if "bias" in epilogue:
                    kw["bias"] = to_dev(bias, dev)
                if "residual" in epilogue:
                    kw["residual"] = out
                results[(kernel, tr, tc)] = plan.run(ad, wd, out=out, **kw).cpu().numpy()
            finally:
                gemm.force_variant(None)
    base = results[("register", 128, 128)]
    assert np.isfinite(base).all()
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), key
    expect = np.einsum("bmk,bnk->bmn", a.astype(np.float64), w.astype(np.float64))
    if "scale" in epilogue:
        expect = expect * scale
    if "bias" in epilogue:
        expect = expect + bias
    if "relu" in epilogue:
        expect = np.maximum(expect, 0)
    if c_layout == "column":
        expect = np.transpose(expect, (0, 2, 1))
    if "residual" in epilogue:
        expect = expect + start.cpu().numpy().astype(np.float64)
    assert rel_max(base, expect) <= 4e-3


@pytest.mark.parametrize("c_layout", ["row", "column"])
@pytest.mark.parametrize("K,epilogue,pad", [(104, (), 8), (64, ("bias", "relu", "residual"), 4), (40, ("scale",), 2)])
def test_f32_source_on_lds_dma_matches_register_kernel(dev, c_layout, K, epilogue, pad):
    # An f32 A under f16 precision (the reference's f32 activations into its
    # f16 matrix units) on the LDS_DMA family, which stages the f32 rows and
    # rounds them to f16 as the MFMA fragments are read: the same bits as the
    # register-staged kernel, which rounds in its loader, on every tile, with
    # NaN in the rows' padding past K. lda = K + 2 leaves the rows 8-byte
    # aligned, which LDS_DMA does not take: that plan names, and runs, the
    # register-staged kernel even with LDS_DMA pinned.
    import torch

    from afhip import gemm

    B, M, N = 2, 333, 200
    lda = K + pad
    sa = M * lda + 4
    rows = np.full((B, M, lda), np.nan, np.float32)
    rows[:, :, :K] = ref.normal(151, (B, M, K))
    a_stored = np.full((B, sa), np.nan, np.float32)
    a_stored[:, :M * lda] = rows.reshape(B, M * lda)
    a = rows[:, :, :K]
    w = ref.round_f16(ref.normal(152, (B, N, K), 1 / K))
    scale = ref.normal(153, (N,), 0.5)
    bias = ref.normal(154, (N,), 0.1)
    cshape = (B, N, M) if c_layout == "column" else (B, M, N)
    start = to_dev(ref.round_f16(ref.normal(155, cshape)), dev)
    ad, wd = to_dev(a_stored, dev), to_dev(w, dev, half=True)
    results = {}
    for kernel, tiles in (("register", [(128, 128)]), ("lds_dma", LDS_DMA_TILES)):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f32", w_dtype="f16", w_layout="k",
                                      out_dtype="f32", epilogue=epilogue, batch=B, lda=lda, batch_stride_a=sa,
                                      batch_stride_w=N * K, batch_stride_c=M * N, c_layout=c_layout)
                assert plan.variant().kernel == (kernel if pad % 4 == 0 else "register")
                out = start.clone()
                kw = {}
                if "scale" in epilogue:
                    kw["scale"] = to_dev(scale, dev)
                if "bias" in epilogue:
                    kw["bias"] = to_dev(bias, dev)
                if "residual" in epilogue:
                    kw["residual"] = out
                results[(kernel, tr, tc)] = plan.run(ad, wd, out=out, **kw).cpu().numpy()
            finally:
                gemm.force_variant(None)
    base = results[("register", 128, 128)]
    assert np.isfinite(base).all()
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), key
    expect = np.einsum("bmk,bnk->bmn", ref.round_f16(a).astype(np.float64), w.astype(np.float64))
    if "scale" in epilogue:
        expect = expect * scale
    if "bias" in epilogue:
        expect = expect + bias
    if "relu" in epilogue:
        expect = np.maximum(expect, 0)
    if c_layout == "column":
        expect = np.transpose(expect, (0, 2, 1))
    if "residual" in epilogue:
        expect = expect + start.cpu().numpy().astype(np.float64)
    assert rel_max(base, expect) <= 4e-3


@pytest.mark.parametrize("shape", [(2, 333, 200, 104, 0), (1, 4096, 512, 128, 0), (3, 130, 70, 36, 44),
                                   (1, 200, 96, 98, 0)])
@pytest.mark.parametrize("epilogue", [(), ("bias", "relu"), ("bias", "residual")])
def test_f32_precision_on_lds_dma_matches_register_kernel(dev, shape, epilogue):
    # f32 arithmetic on the LDS_DMA family (f32 operands staged as 128-byte
    # rows, the f32 MFMA with the register-staged kernel's k pairs and order):
    # the register-staged kernel's bits, ragged M, N and K tails, padded rows
    # holding NaN past K, and config 1's shape (4096 x 128 x 512). K = 98 is
    # not a multiple of 4: that plan names, and runs, the register-staged
    # kernel even with LDS_DMA pinned; so does a run whose source is only
    # 4-byte aligned. Against float64 within config 1's 1e-5.
    import torch

    from afhip import gemm

    B, M, N, K, lda = shape
    lda = lda or K
    rows = np.full((B, M, lda), np.nan, np.float32)
    rows[:, :, :K] = ref.normal(161 + M, (B, M, K))
    w = ref.normal(162 + N, (B, N, K), 1 / K)
    bias = ref.normal(163, (N,), 0.02)
    start = to_dev(ref.normal(164, (B, M, N)), dev)
    ad, wd = to_dev(rows, dev), to_dev(w, dev)
    eligible = K % 4 == 0 and lda % 4 == 0
    results = {}
    for kernel, tiles in (("register", [(64, 64), (128, 128)]), ("lds_dma", [(128, 128), (256, 256)])):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f32", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f32", a_dtype="f32", w_dtype="f32", w_layout="k",
                                      out_dtype="f32", epilogue=epilogue, batch=B, lda=lda,
                                      batch_stride_a=M * lda, batch_stride_w=N * K, batch_stride_c=M * N)
                assert plan.variant().kernel == (kernel if eligible else "register")
                out = start.clone()
                kw = {}
                if "bias" in epilogue:
                    kw["bias"] = to_dev(bias, dev)
                if "residual" in epilogue:
                    kw["residual"] = out
                results[(kernel, tr, tc)] = plan.run(ad, wd, out=out, **kw).cpu().numpy()
            finally:
                gemm.force_variant(None)
    # A source only 4-byte aligned (one float into its buffer): the LDS_DMA
    # plan refuses it at run time and runs the register-staged kernel.
    shifted = torch.empty(ad.numel() + 1, dtype=torch.float32, device=dev)
    shifted[1:] = ad.reshape(-1)
    gemm.force_variant(gemm.GemmVariant("f32", 128, 128, source="pinned", kernel="lds_dma"))
    try:
        plan = gemm.TiledGemm(M, K, N, precision="f32", a_dtype="f32", w_dtype="f32", w_layout="k",
                              out_dtype="f32", epilogue=epilogue, batch=B, lda=lda,
                              batch_stride_a=M * lda, batch_stride_w=N * K, batch_stride_c=M * N)
        out = start.clone()
        kw = {}
        if "bias" in epilogue:
            kw["bias"] = to_dev(bias, dev)
        if "residual" in epilogue:
            kw["residual"] = out
        results["shifted"] = plan.run(shifted[1:], wd, out=out, **kw).cpu().numpy()
    finally:
        gemm.force_variant(None)
    base = results[("register", 64, 64)]
    assert np.isfinite(base).all()
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), key
    expect = np.einsum("bmk,bnk->bmn", rows[:, :, :K].astype(np.float64), w.astype(np.float64))
    if "bias" in epilogue:
        expect = expect + bias
    if "relu" in epilogue:
        expect = np.maximum(expect, 0)
    if "residual" in epilogue:
        expect = expect + start.cpu().numpy().astype(np.float64)
    assert rel_max(base, expect) <= 1e-5


@pytest.mark.parametrize("epilogue", [(), ("bias", "relu", "residual")])
def test_f32_precision_column_major_output_on_lds_dma(dev, epilogue):
    # f32 arithmetic on LDS_DMA with a column-major output (C stored [N][M]),
    # which leaves straight from the f32 MFMA's accumulators: the
    # register-staged kernel's bits, a batch of two, ragged M and N.
    import torch

    from afhip import gemm

    B, M, N, K = 2, 333, 200, 104
    a = ref.normal(171, (B, M, K))
    w = ref.normal(172, (B, N, K), 1 / K)
    bias = to_dev(ref.normal(173, (N,), 0.02), dev)
    start = to_dev(ref.normal(174, (B, N, M)), dev)
    ad, wd = to_dev(a, dev), to_dev(w, dev)
    results = {}
    for kernel in ("register", "lds_dma"):
        gemm.force_variant(gemm.GemmVariant("f32", 128, 128, source="pinned", kernel=kernel))
        try:
            plan = gemm.TiledGemm(M, K, N, precision="f32", a_dtype="f32", w_dtype="f32", w_layout="k",
                                  out_dtype="f32", epilogue=epilogue, batch=B, batch_stride_a=M * K,
                                  batch_stride_w=N * K, batch_stride_c=N * M, c_layout="column")
            assert plan.variant().kernel == kernel
            out = start.clone()
            kw = {"bias": bias, "residual": out} if epilogue else {}
            results[kernel] = plan.run(ad, wd, out=out, **kw).cpu().numpy()
        finally:
            gemm.force_variant(None)
    assert np.array_equal(results["lds_dma"].view(np.uint32), results["register"].view(np.uint32))
    expect = np.einsum("bmk,bnk->bnm", a.astype(np.float64), w.astype(np.float64))
    if epilogue:
        expect = np.maximum(expect + bias.cpu().numpy()[None, :, None], 0) + start.cpu().numpy()
    assert rel_max(results["lds_dma"], expect) <= 1e-5


@pytest.mark.parametrize("case", ["trans2-f32a", "opmcon32-rowA"])
def test_new_lds_dma_sources_at_model_size(dev, case):
    # The f32 source (trans2, 29,972 x 1024 x 256) and the row-contiguous
    # source (the outer-product mean's contraction, 128 x 512 x 32,000 with A
    # given [K][M]) at the model's sizes, where every workgroup runs its
    # steady state: bit-identical to the register-staged kernel over the whole
    # output, and within f16 rounding of float64 on 512 seeded rows.
    import torch

    from afhip import gemm

    if case == "trans2-f32a":
        M, K, N, a_dtype, a_layout = 29972, 1024, 256, "f32", "k"
    else:
        M, K, N, a_dtype, a_layout = 128, 512, 32000, "f16", "row"
    g = torch.Generator(device="cpu").manual_seed(0xAF3001 + M)
    a = torch.randn(K, M, generator=g) if a_layout == "row" else torch.randn(M, K, generator=g)
    a = a if a_dtype == "f32" else a.half()
    w = (torch.randn(N, K, generator=g) / K ** 0.5).half()
    ad, wd = a.to(dev), w.to(dev)
    results = {}
    for kernel in ("register", "lds_dma"):
        gemm.force_variant(gemm.GemmVariant("f16", 128, 128, source="pinned", kernel=kernel))
        try:
            plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype=a_dtype, w_dtype="f16", w_layout="k",
                                  out_dtype="f32", a_layout=a_layout)
            assert plan.variant().kernel == kernel
            results[kernel] = plan.run(ad, wd)
            torch.cuda.synchronize()
        finally:
            gemm.force_variant(None)
    assert torch.equal(results["lds_dma"].view(torch.int32), results["register"].view(torch.int32))
    rows = np.sort(np.random.default_rng(M).choice(M, size=min(M, 512), replace=False))
    a_mk = (a.T if a_layout == "row" else a).half().double().numpy()
    expect = a_mk[rows] @ w.double().numpy().T
    got = results["lds_dma"].cpu().double().numpy()[rows]
    assert rel_max(got, expect) <= 4e-3


def test_column_major_output_selects_lds_dma(dev):
    # Without a pin, an f16-precision plan with a column-major output, a
    # row-contiguous source or an f32 source takes the tile heuristic's
    # family (LDS_DMA here).
    from afhip import gemm

    plan = gemm.TiledGemm(4096, 256, 4096, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                          out_dtype="f16", c_layout="column")
    assert plan.variant().kernel == "lds_dma"
    plan = gemm.TiledGemm(4096, 256, 4096, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                          out_dtype="f16", a_layout="row", c_layout="column")
    assert plan.variant().kernel == "lds_dma"
    plan = gemm.TiledGemm(4096, 256, 4096, precision="f16", a_dtype="f32", w_dtype="f16", w_layout="k",
                          out_dtype="f16")
    assert plan.variant().kernel == "lds_dma"


def test_opm_contraction_as_a_plan(dev):
    # outer[i a][j b] = sum_s left[s][i a] right[s][j b]: the outer-product
    # mean's contraction with both operands accumulated over sequences, as
    # the reference's plan describes it (sourceContiguous "row", the weight
    # [k][column]); S and L * c_outer not multiples of a tile.
    from afhip import gemm

    S, L, co = 37, 5, 32
    P = L * co
    left = ref.round_f16(ref.normal(111, (S, P)))
    right = ref.round_f16(ref.normal(112, (S, P)))
    expect = left.T.astype(np.float64) @ right.astype(np.float64)
    for precision in ("f16", "f32"):
        dtype = "f16" if precision == "f16" else "f32"
        plan = gemm.TiledGemm(P, S, P, precision=precision, a_dtype=dtype, w_dtype=dtype, w_layout="column",
                              out_dtype="f32", a_layout="row")
        out = plan.run(to_dev(left, dev, half=dtype == "f16"), to_dev(right, dev, half=dtype == "f16"))
        assert rel_max(out.cpu().numpy(), expect) <= (4e-3 if precision == "f16" else 1e-5), precision


def test_layouts_are_validated(dev):
    from afhip import _lib, gemm

    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(64, 32, 64, a_layout="column")
    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(64, 32, 64, c_layout="k")
    # a k-major source's stride runs over rows: shorter than M is refused
    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(64, 32, 64, a_layout="row", lda=63)
    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(64, 32, 48, c_layout="column", ldc=40)
