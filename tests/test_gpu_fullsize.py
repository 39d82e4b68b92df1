"""Parity at the benched sizes, on the exact kernel instantiations bench.py
times, through size-independent sampling.

Config 3 (the headline): both triangle directions at L = 384, f16 z, f16
operands with f32 accumulation, f32 output. Config 5: the incoming triangle at
L = 1024 with f16 output. Output pair (i, j) reads only rows (outgoing) or
columns (incoming) i and j of z and z[i, j], so a few hundred sampled pairs are
checked against a float64 restatement (oracle/ref.py triangle_pairs, pinned in
tests/test_oracle.py against the whole oracle and the fixtures). Config 4: the
outer-product mean at S = 512, L = 256, c_m = 256 through the fused
contraction + output projection; out[i, j] reads only MSA columns i and j,
so the oracle on the two-residue slice (i, j) is exact for that pair. Inputs
are bench.py's own (same generators and seeds). Tolerance: the north star's
1e-2 of the largest reference value for the f16 paths.
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


def sample_pairs(length, count, seed):
    # The corners and edges, then seeded positions: count x count pairs.
    rng = np.random.default_rng(seed)
    idx = sorted({0, 1, length - 2, length - 1} | set(int(v) for v in rng.choice(length, count - 4, replace=False)))
    jdx = sorted({0, length // 2, length - 1} | set(int(v) for v in rng.choice(length, count - 3, replace=False)))
    return [(i, j) for i in idx for j in jdx]


def check(got, expect, what, tolerance=1e-2):
    scale = float(np.abs(expect).max())
    err = np.abs(np.asarray(got, np.float64) - expect)
    print(f"{what}: max|d| {err.max():.3e} mean|d| {err.mean():.3e} max|ref| {scale:.3f}", flush=True)
    assert err.max() <= tolerance * scale, what


def run_f32_triangle(dev, length, direction, seed, count, pair_seed):
    # The f32 path (precision f32, f32 pair in and out) at full size, on
    # sampled pairs against float64: the north star's 1e-5 of the largest
    # reference value (max|d| / max|ref|, test/gemm-half-precision.gpu.test.ts:193-201).
    import torch

    import bench
    from afhip import triangle

    CZ, CH = bench.CZ, bench.CH
    z = ref.normal(seed, (length, length, CZ))
    mask = (ref.uniform(seed + 1, (length, length), 0, 1) > 0.15).astype(np.float32)
    weights = bench.triangle_weights(seed, CZ, CH)
    op = triangle.TriangleMultiplication(length, CZ, CH, direction=direction, precision="f32", pair_dtype="f32",
                                         out_dtype="f32")
    op.prepare(weights)
    zd = torch.from_numpy(z).to(dev)
    out = op(zd, torch.from_numpy(mask).to(dev)).cpu().numpy()
    del zd, op
    pairs = sample_pairs(length, count, pair_seed)
    check(np.stack([out[i, j] for i, j in pairs]), ref.triangle_pairs(direction, z, mask, weights, pairs),
          f"f32 {direction} L={length}", tolerance=1e-5)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_config3_triangle_l384_f32_precision(dev, direction):
    import bench

    run_f32_triangle(dev, bench.L, direction, bench.SEED + 22, 14, 8 if direction == "outgoing" else 9)


def test_config5_incoming_l1024_f32_precision(dev):
    import bench

    run_f32_triangle(dev, 1024, "incoming", bench.SEED + 24, 10, 10)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_config3_triangle_l384_sampled_pairs(dev, direction):
    import torch

    import bench
    from afhip import gemm, triangle

    L, CZ, CH = bench.L, bench.CZ, bench.CH
    seed = bench.SEED + 2
    z = ref.round_f16(ref.normal(seed, (L, L, CZ)))
    mask = np.ones((L, L), np.float32)
    weights = bench.triangle_weights(seed, CZ, CH)
    # The contraction runs the tile the bench's run uses (192 x 192 at L = 384).
    v = gemm.select_variant(L, L, L, precision="f16", a_dtype="f16", w_dtype="f16", out_dtype="f16", batch=CH)
    assert (v.kernel, v.tile_rows, v.tile_columns) == ("lds_dma", 192, 192)
    op = triangle.TriangleMultiplication(L, CZ, CH, direction=direction, precision="f16", pair_dtype="f16",
                                         out_dtype="f32")
    op.prepare(weights)
    out = op(torch.from_numpy(z).half().to(dev), torch.from_numpy(mask).to(dev)).cpu().numpy()
    pairs = sample_pairs(L, 16, 3 if direction == "outgoing" else 4)
    expect = ref.triangle_pairs(direction, z, mask, weights, pairs)
    check(np.stack([out[i, j] for i, j in pairs]), expect, f"config 3 {direction} L={L}")


def test_config3_masked_outgoing_l384(dev):
    # The same kernels with the reference's 15%-zero mask
    # (src/testing/deterministic-input.ts:48-49).
    import torch

    import bench
    from afhip import triangle

    L, CZ, CH = bench.L, bench.CZ, bench.CH
    z = ref.round_f16(ref.normal(bench.SEED + 12, (L, L, CZ)))
    mask = (ref.uniform(bench.SEED + 13, (L, L), 0, 1) > 0.15).astype(np.float32)
    weights = bench.triangle_weights(bench.SEED + 14, CZ, CH)
    op = triangle.TriangleMultiplication(L, CZ, CH, direction="outgoing", precision="f16", pair_dtype="f16",
                                         out_dtype="f32")
    op.prepare(weights)
    out = op(torch.from_numpy(z).half().to(dev), torch.from_numpy(mask).to(dev)).cpu().numpy()
    pairs = sample_pairs(L, 12, 5)
    check(np.stack([out[i, j] for i, j in pairs]), ref.triangle_pairs("outgoing", z, mask, weights, pairs),
          "config 3 outgoing, masked")


def test_config5_incoming_l1024_sampled_pairs(dev):
    import torch

    import bench
    from afhip import triangle

    L, CZ, CH = 1024, bench.CZ, bench.CH
    seed = bench.SEED + 4
    z = ref.round_f16(ref.normal(seed, (L, L, CZ)))
    mask = np.ones((L, L), np.float32)
    weights = bench.triangle_weights(seed, CZ, CH)
    op = triangle.TriangleMultiplication(L, CZ, CH, direction="incoming", precision="f16", pair_dtype="f16",
                                         out_dtype="f16")
    op.prepare(weights)
    zd = torch.from_numpy(z).half().to(dev)
    out = op(zd, torch.from_numpy(mask).to(dev)).float().cpu().numpy()
    del zd
    pairs = sample_pairs(L, 12, 6)
    check(np.stack([out[i, j] for i, j in pairs]), ref.triangle_pairs("incoming", z, mask, weights, pairs),
          "config 5 incoming L=1024")


def test_config4_outer_product_mean_full_size(dev):
    import torch

    import bench
    from afhip import device, opm

    s = bench.SEED + 3
    S, L, CM, CO, CZ = 512, 256, 256, 32, 128
    act = ref.round_f16(ref.normal(s, (S, L, CM)))
    mask = np.ones((S, L), np.float32)
    w = {"layerNormScale": ref.normal(s + 1, (CM,), 0.01, 1.0), "layerNormOffset": ref.normal(s + 2, (CM,), 0.01),
         "leftWeight": ref.normal(s + 3, (CM, CO), 1 / CM), "leftBias": ref.normal(s + 4, (CO,), 0.02),
         "rightWeight": ref.normal(s + 5, (CM, CO), 1 / CM), "rightBias": ref.normal(s + 6, (CO,), 0.02),
         "outputWeight": ref.normal(s + 7, (CO * CO, CZ), 1 / (CO * CO)), "outputBias": ref.normal(s + 8, (CZ,), 0.02)}
    # The run goes through the launches bench.py times: the projection (with
    # the pair counts) and the fused contraction + output projection.
    op = opm.OuterProductMean(S, L, CM, CO, CZ, precision="f16", msa_dtype="f16", out_dtype="f32")
    op.prepare(w)
    device.timing_reset()
    device.timing_enable(True)
    try:
        out = op(torch.from_numpy(act).half().to(dev), torch.from_numpy(mask).to(dev)).cpu().numpy()
        labels = set(device.timing_report())
    finally:
        device.timing_enable(False)
    assert labels == {"opm.project", "opm.fused"}, labels
    got, expect = [], []
    for i, j in sample_pairs(L, 7, 7):
        cols = [i] if i == j else [i, j]
        sl = ref.opm(np.ascontiguousarray(act[:, cols]), np.ascontiguousarray(mask[:, cols]), w)
        got.append(out[i, j])
        expect.append(sl[0, 0] if i == j else sl[0, 1])
    check(np.stack(got), np.stack(expect).astype(np.float64), "config 4 outer-product mean")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_long_complex_l3072_fast_path(dev, direction):
    # Past the length where an f16 pair outgrows 2 GiB (L = 2,896): the
    # persistent f16 kernels at L = 3072, f16 z (2.4 GB) with the 15%-zero
    # mask, f32 out. z is drawn on the device (seeded); the oracle reads the
    # sampled pairs' rows or columns from a host copy.
    import ctypes

    import torch

    import bench
    from afhip import _lib, triangle

    L, CZ, CH = 3072, bench.CZ, bench.CH
    desc = _lib.TriangleDesc(L, CZ, CH, 0 if direction == "outgoing" else 1, 1, 1, 0, 0, 0, 1e-5)
    flag = ctypes.c_int32(-1)
    _lib.call("afhip_triangle_fast_path", ctypes.byref(desc), ctypes.byref(flag))
    assert flag.value == 1
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xAF2005)
    zd = torch.randn((L, L, CZ), generator=gen, device=dev).half()
    mask = (ref.uniform(bench.SEED + 25, (L, L), 0, 1) > 0.15).astype(np.float32)
    weights = bench.triangle_weights(bench.SEED + 26, CZ, CH)
    op = triangle.TriangleMultiplication(L, CZ, CH, direction=direction, precision="f16", pair_dtype="f16",
                                         out_dtype="f32")
    op.prepare(weights)
    out = op(zd, torch.from_numpy(mask).to(dev))
    pairs = sample_pairs(L, 10, 11 if direction == "outgoing" else 12)
    ii = torch.tensor([i for i, _ in pairs], device=dev)
    jj = torch.tensor([j for _, j in pairs], device=dev)
    got = out[ii, jj].cpu().numpy()
    del out, op
    z = zd.cpu().numpy()
    del zd
    torch.cuda.empty_cache()
    check(got, ref.triangle_pairs(direction, z, mask, weights, pairs), f"f16 {direction} L={L} fast path")
