"""GEMM parity on the GPU: libafhip against the CPU oracle.

Tolerances are the reference's: max|d|/max|ref| <= 1e-5 for the f32 path
the per-variant bounds of
test/gemm-half-precision.gpu.test.ts:35-41 for ragged shapes, 1e-2 for the
f16 and mixed-q8 paths, and bit-exact for dequantised int8 weights.
"""
import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu


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


def to_dev(x, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def test_config1_pair_transition_linear_f32(dev):
    # X [4096x128] ~N(0,1), W [128x512] ~N(0,1/128),
    # bias ~N(0,0.02), ReLU; seed 0xAF2000 + 0.
    from afhip import gemm

    seed = 0xAF2000
    x = ref.normal(seed, (4096, 128))
    w = ref.normal(seed + 1, (128, 512), 1 / 128)
    b = ref.normal(seed + 2, (512,), 0.02)
    expect = ref.linear(x, w, b, relu=True)
    out = gemm.linear(to_dev(x, dev), to_dev(w, dev), to_dev(b, dev), relu=True, precision="f32")
    assert rel_max(out.cpu().numpy(), expect) <= 1e-5


@pytest.mark.parametrize("inner", [256, 1024])
@pytest.mark.parametrize("precision,tol", [("f32", 1e-4), ("f16", 5e-3)])
def test_ragged_projection_matches_f64(dev, inner, precision, tol):
    # test/gemm-half-precision.gpu.test.ts:206-261: rows 81, columns 132.
    from afhip import gemm

    a = ref.lcg_values(1, 81 * inner).reshape(81, inner)
    w = ref.lcg_values(2, inner * 132).reshape(inner, 132)
    b = ref.lcg_values(3, 132)
    expect = ref.gemm_f64(a, w, b)
    out = gemm.linear(to_dev(a, dev), to_dev(w, dev), to_dev(b, dev), precision=precision)
    assert rel_max(out.cpu().numpy(), expect) <= tol


@pytest.mark.parametrize("m,k,n", [(130, 96, 132), (1, 8, 1), (64, 32, 64), (257, 40, 31)])
@pytest.mark.parametrize("precision", ["f32", "f16"])
def test_odd_shapes(dev, m, k, n, precision):
    from afhip import gemm

    a = ref.normal(m * 7 + k, (m, k))
    w = ref.normal(n * 3 + k, (k, n), 1 / k)
    expect = ref.gemm_f64(a, w)
    out = gemm.linear(to_dev(a, dev), to_dev(w, dev), precision=precision)
    assert rel_max(out.cpu().numpy(), expect) <= (1e-5 if precision == "f32" else 5e-3)


def test_every_tile_variant_agrees(dev):
    from afhip import gemm

    a = ref.normal(5, (300, 256))
    w = ref.normal(6, (256, 200), 1 / 256)
    expect = ref.gemm_f64(a, w)
    for tr, tc in [(64, 64), (64, 128), (128, 64), (128, 128)]:
        gemm.force_variant(gemm.GemmVariant("f32", tr, tc, source="pinned"))
        try:
            out = gemm.linear(to_dev(a, dev), to_dev(w, dev), precision="f32")
        finally:
            gemm.force_variant(None)
        assert rel_max(out.cpu().numpy(), expect) <= 1e-5, (tr, tc)


LDS_DMA_TILES = [(128, 128), (192, 192), (128, 256), (256, 256)]


def _batched_f16_plan(gemm, B, M, N, K, out_dtype, lda=0):
    lda = lda or K
    return gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                          out_dtype=out_dtype, batch=B, lda=lda, batch_stride_a=M * lda, batch_stride_w=N * K,
                          batch_stride_c=M * N)


@pytest.mark.parametrize("out_dtype", ["f16", "f32"])
@pytest.mark.parametrize("shape", [(3, 200, 136, 104, 0), (2, 64, 448, 40, 56), (1, 385, 193, 392, 0),
                                   (2, 200, 300, 508, 0), (1, 130, 257, 98, 102), (3, 65, 70, 30, 34)])
def test_lds_dma_tiles_match_register_kernel_bitwise(dev, out_dtype, shape):
    # Both kernel families walk K in the same 32-deep steps of two 16-deep
    # MFMAs, so they accumulate in one order: every tile gives the register-
    # staged kernel's result bit for bit, ragged M, N and K tails included.
    # The last three shapes have rows that are only 4-byte aligned (K or lda
    # not a multiple of 8, as the reference's opm-contract K = 508): LDS_DMA
    # loads them 4 bytes a lane.
    from afhip import gemm

    B, M, N, K, lda = shape
    lda = lda or K
    a = ref.round_f16(ref.normal(31 + M, (B, M, lda)))
    w = ref.round_f16(ref.normal(32 + N, (B, N, K), 1 / K))
    ad, wd = to_dev(a, dev).half(), to_dev(w, dev).half()
    results = {}
    for kernel, tiles in (("register", [(128, 128)]), ("lds_dma", LDS_DMA_TILES)):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = _batched_f16_plan(gemm, B, M, N, K, out_dtype, lda)
                assert plan.variant().kernel == kernel
                results[(kernel, tr, tc)] = plan.run(ad, wd).float().cpu().numpy()
            finally:
                gemm.force_variant(None)
    base = results[("register", 128, 128)]
    expect = np.einsum("bmk,bnk->bmn", a[:, :, :K].astype(np.float64), w.astype(np.float64))
    assert rel_max(base, expect) <= 2e-3
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), key


@pytest.mark.parametrize("out_dtype", ["f16", "f32"])
@pytest.mark.parametrize("w_layout", ["column", "k"])
def test_int8_weights_on_lds_dma_match_register_kernel(dev, out_dtype, w_layout):
    # The reference's trans2 shape class with mixed-q8 weights (K = 1024):
    # a plan on the LDS_DMA family widens the int8 weight to f16 (exact) and
    # applies the per-column scale to the f32 accumulator, as the register-
    # staged kernel does inside its loader: the same bits. Against float64
    # with the oracle-decoded weight within the q8 path's 1e-2.
    from afhip import gemm

    M, K, N = 500, 1024, 256
    x = ref.round_f16(ref.normal(51, (M, K)))
    q = ref.uniform_i8(52, (K, N))
    s = ref.uniform(53, (N,), 1e-3, 1e-2)
    w = q if w_layout == "column" else np.ascontiguousarray(q.T)
    xd, wd, sd = to_dev(x, dev).half(), to_dev(w, dev), to_dev(s, dev)
    results = {}
    for pin in (gemm.GemmVariant("f16", 128, 128, source="pinned", kernel="register"), None):
        gemm.force_variant(pin)
        try:
            plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="i8", w_layout=w_layout,
                                  out_dtype=out_dtype, epilogue=("scale",))
            kernel = plan.variant().kernel
            results[kernel] = plan.run(xd, wd, scale=sd).float().cpu().numpy()
        finally:
            gemm.force_variant(None)
    assert set(results) == {"register", "lds_dma"}
    assert np.array_equal(results["lds_dma"].view(np.uint32), results["register"].view(np.uint32))
    expect = x.astype(np.float64) @ ref.q8_channel_decode(q, s).astype(np.float64)
    err = np.abs(results["lds_dma"] - expect)
    assert np.all(err <= 1e-2 * np.maximum(1.0, np.abs(expect))), float(err.max())


@pytest.mark.parametrize("out_dtype", ["f16", "f32"])
@pytest.mark.parametrize("epilogue", [("bias", "relu"), ("scale", "bias", "residual"), ("bias", "relu", "residual")])
def test_lds_dma_epilogues_match_register_kernel_bitwise(dev, out_dtype, epilogue):
    # The row-wise epilogues the LDS_DMA family applies straight from its
    # accumulators (four columns a lane, vector residual reads and stores)
    # round every step as the register-staged kernel does: the same bits, a
    # ragged last row and column tile included.
    import torch

    from afhip import gemm

    M, K, N = 333, 192, 200
    a = ref.round_f16(ref.normal(41, (M, K)))
    w = ref.round_f16(ref.normal(42, (N, K), 1 / K))
    scale = to_dev(ref.uniform(43, (N,), 0.5, 2.0), dev)
    bias = to_dev(ref.normal(44, (N,), 0.1), dev)
    tdt = torch.float16 if out_dtype == "f16" else torch.float32
    base = to_dev(ref.round_f16(ref.normal(45, (M, N))), dev).to(tdt)
    ad, wd = to_dev(a, dev).half(), to_dev(w, dev).half()
    results = {}
    for kernel, tiles in (("register", [(128, 128)]), ("lds_dma", LDS_DMA_TILES)):
        for tr, tc in tiles:
            gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype="f16", w_layout="k",
                                      out_dtype=out_dtype, epilogue=epilogue)
                assert plan.variant().kernel == kernel
                out = base.clone()
                kw = {"bias": bias}
                if "scale" in epilogue:
                    kw["scale"] = scale
                if "residual" in epilogue:
                    kw["residual"] = out
                results[(kernel, tr, tc)] = plan.run(ad, wd, out=out, **kw).float().cpu().numpy()
            finally:
                gemm.force_variant(None)
    base_r = results[("register", 128, 128)]
    for key, got in results.items():
        assert np.array_equal(got.view(np.uint32), base_r.view(np.uint32)), key


@pytest.mark.parametrize("shape", [
    # rows, K, N, weight dtype, epilogue, lda
    (5000, 256, 1024, "i8", ("scale", "attention"), 0),  # config 2's shape, ragged last tile
    (777, 128, 512, "f16", ("bias", "relu"), 0),
    (4096, 64, 576, "i8", ("scale",), 0),                # a second slice with one wave's columns
    (300, 128, 512, "f16", (), 136),                     # strided rows
])
def test_stream_matches_register_kernel_bitwise(dev, shape):
    # The STREAM kernel accumulates K in the same ascending 16-deep MFMA steps
    # as the register-staged kernel and applies the epilogue in the same order,
    # so its f16 output is the register kernel's bit for bit.
    import torch

    from afhip import gemm

    M, K, N, wd, epi, lda = shape
    lda = lda or K
    a = ref.round_f16(ref.normal(61 + M, (M, lda)))
    if wd == "i8":
        w = ref.uniform_i8(62 + N, (N, K))
        wt = to_dev(w, dev)
    else:
        w = ref.round_f16(ref.normal(62 + N, (N, K), 1 / K))
        wt = to_dev(w, dev).half()
    scale = to_dev(ref.uniform(63, (N,), 1e-3, 1e-2), dev) if "scale" in epi else None
    bias = to_dev(ref.normal(64, (N,), 0.5), dev) if "bias" in epi else None
    heads = dict(heads=N // 128, head_dim=32) if "attention" in epi else {}
    ad = to_dev(a, dev).half()
    results = {}
    for kernel, tr, tc in (("register", 128, 128), ("stream", 64, 512)):
        gemm.force_variant(gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel))
        try:
            plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype="f16", w_dtype=wd, w_layout="k", out_dtype="f16",
                                  epilogue=epi, lda=lda, **heads)
            assert plan.variant().kernel == kernel
            results[kernel] = plan.run(ad, wt, scale=scale, bias=bias)
            torch.cuda.synchronize()
            results[kernel] = results[kernel].cpu().numpy()
        finally:
            gemm.force_variant(None)
    assert np.array_equal(results["stream"].view(np.uint16), results["register"].view(np.uint16))
    acc = a[:, :K].astype(np.float64) @ w.astype(np.float64).T
    if scale is not None:
        acc = acc * scale.cpu().numpy()
    if bias is not None:
        acc = acc + bias.cpu().numpy()
    if "attention" in epi:
        hd = N // 4
        acc[:, :hd] /= np.sqrt(32.0)
        acc[:, 3 * hd:] = 1 / (1 + np.exp(-acc[:, 3 * hd:]))
    if "relu" in epi:
        acc = np.maximum(acc, 0)
    err = np.abs(results["stream"].astype(np.float64) - acc)
    assert np.all(err <= 1e-2 * np.maximum(1.0, np.abs(acc))), float(err.max())


def test_config3_contraction_full_size(dev):
    # BASELINE config 3's contraction: 128 channels of a 384 x 384 x 384
    # f16 product with f32 accumulation and f16 output, against torch's f32
    # batched product of the same f16 values.
    import torch

    from afhip import gemm

    C, L = 128, 384
    g = torch.Generator(device="cpu").manual_seed(0xAF2002)
    a = torch.randn(C, L, L, generator=g).half().to(dev)
    b = torch.randn(C, L, L, generator=g).half().to(dev)
    plan = _batched_f16_plan(gemm, C, L, L, L, "f16")
    assert plan.variant().kernel == "lds_dma"
    out = plan.run(a, b).float()
    expect = torch.bmm(a.float(), b.float().transpose(1, 2).contiguous())
    err = (out - expect).abs().max().item() / expect.abs().max().item()
    assert err <= 2e-3, err


@pytest.mark.parametrize("tile", [(128, 256), (256, 256)])
def test_config5_contraction_full_size(dev, tile):
    # BASELINE config 5's contraction (128 channels of 1024 x 1024 x 1024)
    # on the tiles chosen for long K, against torch's f32 batched product of
    # the same f16 values.
    import torch

    from afhip import gemm

    C, L = 128, 1024
    g = torch.Generator(device="cpu").manual_seed(0xAF2005)
    a = torch.randn(C, L, L, generator=g).half().to(dev)
    b = torch.randn(C, L, L, generator=g).half().to(dev)
    gemm.force_variant(gemm.GemmVariant("f16", tile[0], tile[1], source="pinned", kernel="lds_dma"))
    try:
        plan = _batched_f16_plan(gemm, C, L, L, L, "f16")
        assert plan.variant().kernel == "lds_dma"
        out = plan.run(a, b).float()
    finally:
        gemm.force_variant(None)
    expect = torch.bmm(a.float(), b.float().transpose(1, 2).contiguous())
    err = (out - expect).abs().max().item() / expect.abs().max().item()
    assert err <= 2e-3, err


def test_relu_residual_epilogue(dev):
    from afhip import gemm

    a = ref.normal(11, (96, 64))
    w = ref.normal(12, (64, 80), 1 / 64)
    b = ref.normal(13, (80,), 0.02)
    r = ref.normal(14, (96, 80))
    expect = ref.linear(a, w, b, relu=True, residual=r)
    out = gemm.linear(to_dev(a, dev), to_dev(w, dev), to_dev(b, dev), relu=True, residual=to_dev(r, dev))
    assert rel_max(out.cpu().numpy(), expect) <= 1e-5


def test_batched_k_contiguous(dev):
    import torch

    from afhip import gemm

    B, M, N, K = 5, 70, 90, 48
    a = ref.normal(21, (B, M, K))
    w = ref.normal(22, (B, N, K), 1 / K)  # [n][k]
    plan = gemm.TiledGemm(M, K, N, precision="f32", w_layout="k", batch=B, batch_stride_a=M * K,
                          batch_stride_w=N * K, batch_stride_c=M * N)
    out = plan.run(to_dev(a, dev), to_dev(w, dev)).cpu().numpy()
    expect = np.einsum("bmk,bnk->bmn", a.astype(np.float64), w.astype(np.float64))
    assert rel_max(out, expect) <= 1e-5
    assert torch.cuda.is_available()


def test_q8_channel_dequant_bit_exact(dev):
    from afhip import gemm

    q = ref.uniform_i8(0xAF2001, (256, 1024))
    s = ref.uniform(0xAF2002, (1024,), 1e-3, 1e-2)
    out = gemm.dequant_q8_channel(to_dev(q, dev), to_dev(s, dev)).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), ref.q8_channel_decode(q, s).view(np.uint32))


def test_q8_block_dequant_known_answer_and_bit_exact(dev):
    from afhip import gemm

    codes = np.array([1, -2, 3, -4, 5], np.int8)
    scales = np.array([0x3800, 0x4000], np.uint16)
    out = gemm.dequant_q8_block(to_dev(codes, dev), to_dev(scales.view(np.int16), dev), 4).cpu().numpy()
    assert list(out) == [0.5, -1, 1.5, -2, 10]
    w = ref.normal(3, (4096,), 0.02)
    c, s = ref.q8_block_encode(w, 64)
    got = gemm.dequant_q8_block(to_dev(c, dev), to_dev(s.view(np.int16), dev), 64, 100, 3000).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.q8_block_decode(c, s, 64, 100, 3000).view(np.uint32))


@pytest.mark.parametrize("K,N,start,dtype", [(256, 1024, 0, "f16"), (130, 96, 100, "f32"), (37, 200, 64, "f16")])
def test_q8_bundle_packs_straight_into_gemm_operand(dev, K, N, start, dtype):
    # A mixed-q8 bundle tensor [in][out] inside a longer int8 stream, with
    # block-64 f16 scales that vary with k as well as n (quantize-web-model.ts:
    # 98-119): the device decode into the packed operand W[n][k] equals the
    # host decode (dtype.ts:66-99) bit for bit (then rounded to nearest even
    # for f16), and a plan on that operand matches the f64 product over the
    # host-decoded weight.
    from afhip import gemm

    total = start + K * N + 50
    codes, scales = ref.q8_block_encode(ref.normal(0xAF2011 + K, (total,), 0.02), 64)
    decoded = ref.q8_block_decode(codes, scales, 64, start, K * N).reshape(K, N)
    expect_w = np.ascontiguousarray(decoded.T)
    if dtype == "f16":
        expect_w = ref.round_f16(expect_w)
    packed = gemm.pack_weight_q8_block(to_dev(codes, dev), to_dev(scales.view(np.int16), dev), K, N, start=start,
                                       dtype=dtype)
    got = packed.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), expect_w.astype(np.float32).view(np.uint32))
    x = ref.normal(0xAF2012 + N, (300, K))
    x = x if dtype == "f32" else ref.round_f16(x)
    plan = gemm.TiledGemm(300, K, N, precision=dtype, a_dtype=dtype, w_dtype=dtype, w_layout="k", out_dtype="f32")
    xd = to_dev(x, dev) if dtype == "f32" else to_dev(x, dev).half()
    out = plan.run(xd, packed).cpu().numpy()
    assert rel_max(out, ref.gemm_f64(x, decoded)) <= (1e-5 if dtype == "f32" else 1e-2)


def test_q8_bundle_pack_rejects_bad_ranges(dev):
    from afhip import _lib, gemm

    codes, scales = ref.q8_block_encode(ref.normal(7, (1000,), 0.02), 64)
    c, s = to_dev(codes, dev), to_dev(scales.view(np.int16), dev)
    with pytest.raises(_lib.RangeError, match="out of bounds"):
        gemm.pack_weight_q8_block(c, s, 40, 30, start=1)
    with pytest.raises(_lib.RangeError, match="invalid block size"):
        gemm.pack_weight_q8_block(c, s, 10, 10, block=0)


def _config2_inputs(rows):
    seed = 0xAF2001
    x = ref.round_f16(ref.normal(seed, (rows, 256)))
    q = ref.uniform_i8(seed + 1, (256, 1024))
    s = ref.uniform(seed + 2, (1024,), 1e-3, 1e-2)
    return x, q, s


@pytest.mark.parametrize("rows", [4096, 131072])
def test_config2_mixed_q8_attention_projection(dev, rows):
    # BASELINE config 2 (M = 512 * 256 = 131,072 at full size): f16 X, int8 W
    # with per-column f32 scales, f32 accumulation, f16 q/k/v/gate.
    from afhip import gemm

    x, q, s = _config2_inputs(rows)
    xd = to_dev(x.astype(np.float16), dev)
    outs = gemm.attention_project(xd, to_dev(q, dev), heads=8, head_dim=32, scale=to_dev(s, dev))
    got = [o.float().cpu().numpy() for o in outs]
    wq = ref.q8_channel_decode(q, s)

    def close(g, exp, what):
        err = np.abs(g - exp)
        assert np.all(err <= 1e-2 * np.maximum(1.0, np.abs(exp))), (what, float(err.max()))

    # Every row against a float64 product with the oracle-decoded weight
    # (columns [q | k | v | g], q scaled by 1/sqrt(32), g through the
    # sigmoid), in blocks of rows.
    w64 = wq.astype(np.float64)
    for r0 in range(0, rows, 8192):
        y = x[r0:r0 + 8192].astype(np.float64) @ w64
        exp = (y[:, :256] / np.sqrt(32.0), y[:, 256:512], y[:, 512:768], 1.0 / (1.0 + np.exp(-y[:, 768:])))
        for i, (g, e) in enumerate(zip(got, exp)):
            close(g[r0:r0 + 8192], e, ("qkvg"[i], r0))
    # The oracle's own epilogue on seeded rows that cover every position in
    # a 32-row activation tile, tiles of both parities and the last tile.
    rng = np.random.default_rng(0xAF2001)
    check = np.unique(np.concatenate([rng.choice(rows, 512, replace=False), np.arange(64), np.arange(rows - 64, rows)]))
    assert set(check % 32) == set(range(32)) and set((check // 32) % 2) == {0, 1}
    expect = ref.attention_project(x[check], wq, None, heads=8, head_dim=32)
    for i, (g, exp) in enumerate(zip(got, expect)):
        close(g[check], exp, ("qkvg"[i], "oracle rows"))


def test_attention_gate_bias_and_f32_path(dev):
    from afhip import gemm

    x = ref.normal(41, (100, 64))
    w = ref.normal(42, (64, 4 * 2 * 8), 1 / 64)
    gb = ref.normal(43, (16,), 0.02)
    outs = gemm.attention_project(to_dev(x, dev), to_dev(w, dev), heads=2, head_dim=8, gate_bias=to_dev(gb, dev),
                                  out_dtype="f32")
    expect = ref.attention_project(x, w, gb, heads=2, head_dim=8)
    for got, exp in zip(outs, expect):
        assert rel_max(got.cpu().numpy(), exp) <= 1e-5


def test_invalid_plan_raises_range_error(dev):
    from afhip import _lib, gemm

    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(0, 4, 4)
    with pytest.raises(_lib.RangeError):
        gemm.TiledGemm(4, 4, 4, precision="f32", w_dtype="i8")
