"""Outer-product mean and transition parity on the GPU.

OPM: test/outer-product-mean-reference.gpu.test.ts:103-130 (9 sequences x 8
residues x 12 channels, c_o 32, c_z 16, every third mask entry zero, residue
blocks of 3) at mean < 2e-5 / max < 2e-4; residue blocking bit-identical
(test/evoformer-outer-product-mean.gpu.test.ts:78-81); f16 within 1e-2.
Transition: the f32 path within 1e-5 of the largest value.
"""
import numpy as np
import pytest

from oracle import ref
from test_oracle import opm_test_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def opm_input(act, mask, w, row_block=None):
    S, L, cm = act.shape
    return {"activations": act, "mask": mask, "sequences": S, "length": L, "cM": cm,
            "cOuter": w["leftBias"].shape[0], "cZ": w["outputBias"].shape[0], "weights": w,
            "layerNormEpsilon": 1e-5, "normalizationEpsilon": 1e-3, "rowBlockResidues": row_block}


def test_opm_reference_case(dev):
    from afhip import opm

    act, mask, w = opm_test_case()
    expect = ref.opm(act, mask, w)
    out = opm.OuterProductMeanGpu().run(opm_input(act, mask, w, 3))["output"]
    m = ref.error_metrics(out, expect)
    assert m["meanAbsoluteError"] < 2e-5 and m["maxAbsoluteError"] < 2e-4


def test_opm_blocking_bit_identical(dev):
    from afhip import opm

    act, mask, w = opm_test_case()
    whole = opm.OuterProductMeanGpu().run(opm_input(act, mask, w))["output"]
    for rb in (3, 1, 5):
        blocked = opm.OuterProductMeanGpu().run(opm_input(act, mask, w, rb))["output"]
        assert np.array_equal(whole.view(np.uint32), blocked.view(np.uint32)), rb


@pytest.mark.parametrize("S,L,cm,co,cz", [(64, 24, 256, 32, 128), (33, 17, 40, 8, 12)])
def test_opm_synthetic(dev, S, L, cm, co, cz):
    from afhip import opm

    act = ref.normal(S + L, (S, L, cm))
    mask = (ref.uniform(S * L, (S, L), 0, 1) > 0.1).astype(np.float32)
    w = {"layerNormScale": ref.normal(1, (cm,), 0.01, 1.0), "layerNormOffset": ref.normal(2, (cm,), 0.01),
         "leftWeight": ref.normal(3, (cm, co), 1 / cm), "leftBias": ref.normal(4, (co,), 0.02),
         "rightWeight": ref.normal(5, (cm, co), 1 / cm), "rightBias": ref.normal(6, (co,), 0.02),
         "outputWeight": ref.normal(7, (co * co, cz), 1 / (co * co)), "outputBias": ref.normal(8, (cz,), 0.02)}
    expect = ref.opm(act, mask, w)
    scale = max(1.0, float(np.abs(expect).max()))
    out = opm.OuterProductMeanGpu().run(opm_input(act, mask, w))["output"].reshape(expect.shape)
    assert np.abs(out - expect).max() <= 1e-5 * scale
    out16 = opm.OuterProductMeanGpu().run(opm_input(act, mask, w), {"precision": "f16"})["output"]
    assert np.abs(out16.reshape(expect.shape) - expect).max() <= 1e-2 * scale


@pytest.mark.parametrize("S,L", [(37, 45), (512, 33), (3, 70)])
def test_opm_fractional_mask_counts(dev, S, L):
    # Fractional mask values (the count is a sum of products, not of ones)
    # with S and L off the 32-wide count tiles, against the oracle.
    from afhip import opm

    cm, co, cz = 16, 8, 12
    act = ref.normal(S * 7 + L, (S, L, cm))
    mask = ref.uniform(S + 3 * L, (S, L), 0, 1)
    mask[mask < 0.2] = 0.0
    w = {"layerNormScale": ref.normal(1, (cm,), 0.01, 1.0), "layerNormOffset": ref.normal(2, (cm,), 0.01),
         "leftWeight": ref.normal(3, (cm, co), 1 / cm), "leftBias": ref.normal(4, (co,), 0.02),
         "rightWeight": ref.normal(5, (cm, co), 1 / cm), "rightBias": ref.normal(6, (co,), 0.02),
         "outputWeight": ref.normal(7, (co * co, cz), 1 / (co * co)), "outputBias": ref.normal(8, (cz,), 0.02)}
    expect = ref.opm(act, mask, w)
    out = opm.OuterProductMeanGpu().run(opm_input(act, mask, w))["output"].reshape(expect.shape)
    assert np.abs(out - expect).max() <= 1e-5 * max(1.0, float(np.abs(expect).max()))


@pytest.mark.parametrize("S,L,cm,msa_dtype", [(100, 9, 256, "f16"), (130, 5, 64, "f32"), (64, 7, 128, "f16")])
def test_opm_f16_fast_projection(dev, S, L, cm, msa_dtype):
    # The persistent f16 projection (c_outer 32, c_m 64/128/256): ragged
    # sequence tiles, f16 and f32 MSA input, against the f64 oracle within the
    # f16 tolerance.
    import torch

    from afhip import opm

    co, cz = 32, 16
    act = ref.normal(S * 3 + L, (S, L, cm))
    if msa_dtype == "f16":
        act = ref.round_f16(act)
    mask = (ref.uniform(S + 7 * L, (S, L), 0, 1) > 0.2).astype(np.float32)
    w = {"layerNormScale": ref.normal(11, (cm,), 0.1, 1.0), "layerNormOffset": ref.normal(12, (cm,), 0.1),
         "leftWeight": ref.normal(13, (cm, co), 1 / cm), "leftBias": ref.normal(14, (co,), 0.02),
         "rightWeight": ref.normal(15, (cm, co), 1 / cm), "rightBias": ref.normal(16, (co,), 0.02),
         "outputWeight": ref.normal(17, (co * co, cz), 1 / (co * co)), "outputBias": ref.normal(18, (cz,), 0.02)}
    expect = ref.opm(act, mask, w)
    op = opm.OuterProductMean(S, L, cm, co, cz, precision="f16", msa_dtype=msa_dtype, out_dtype="f32")
    op.prepare(w)
    tdt = torch.float16 if msa_dtype == "f16" else torch.float32
    out = op(torch.from_numpy(act).to(dev, tdt), torch.from_numpy(mask).to(dev)).cpu().numpy()
    scale = max(1.0, float(np.abs(expect).max()))
    assert np.abs(out - expect).max() <= 1e-2 * scale


def fused_case(S, L, cm, cz, seed):
    co = 32
    act = ref.round_f16(ref.normal(seed, (S, L, cm)))
    mask = (ref.uniform(seed + 1, (S, L), 0, 1) > 0.2).astype(np.float32)
    mask[:, L // 2] = 0.0  # residue L / 2 never aligned: its pairs count 0 (bias / eps)
    w = {"layerNormScale": ref.normal(seed + 2, (cm,), 0.1, 1.0), "layerNormOffset": ref.normal(seed + 3, (cm,), 0.1),
         "leftWeight": ref.normal(seed + 4, (cm, co), 1 / cm), "leftBias": ref.normal(seed + 5, (co,), 0.02),
         "rightWeight": ref.normal(seed + 6, (cm, co), 1 / cm), "rightBias": ref.normal(seed + 7, (co,), 0.02),
         "outputWeight": ref.normal(seed + 8, (co * co, cz), 1 / (co * co)),
         "outputBias": ref.normal(seed + 9, (cz,), 0.02)}
    return act, mask, w


@pytest.mark.parametrize("S,L,cm,cz,out_dtype,residual", [(64, 13, 64, 128, "f32", False),
                                                          (40, 45, 64, 100, "f16", True),
                                                          (512, 8, 256, 128, "f32", True),
                                                          (7, 70, 40, 128, "f16", False)])
def test_opm_fused_contraction_output(dev, S, L, cm, cz, out_dtype, residual):
    # The single-launch contraction + output projection (f16, c_outer 32,
    # c_z in (96, 128]): residue counts off the 8-residue pair blocks, a
    # c_z below the 128 the weights are padded to, an all-masked residue,
    # f16 and f32 output, the residual added to the output's old contents,
    # a sequence count off the 8-sequence chunks after the general
    # projection (c_m 40); against the f64 oracle within the f16 tolerance,
    # and bit-identical whatever the residue blocking.
    import torch

    from afhip import opm

    act, mask, w = fused_case(S, L, cm, cz, 100 + L)
    expect = ref.opm(act, mask, w).astype(np.float64)
    old = ref.normal(7 * L, (L, L, cz)) if residual else np.zeros((L, L, cz))
    if out_dtype == "f16":
        old = ref.round_f16(old)
    tdt = torch.float16 if out_dtype == "f16" else torch.float32
    outs = []
    for rb in (0, 3):
        op = opm.OuterProductMean(S, L, cm, 32, cz, precision="f16", msa_dtype="f16", out_dtype=out_dtype,
                                  row_block=rb, residual=residual)
        op.prepare(w)
        out = torch.from_numpy(old).to(dev, tdt)
        op(torch.from_numpy(act).to(dev, torch.float16), torch.from_numpy(mask).to(dev), out)
        outs.append(out.float().cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want = expect + old
    scale = max(1.0, float(np.abs(want).max()))
    err = np.abs(outs[0] - want)
    print(f"fused S={S} L={L} cz={cz} {out_dtype}: max|d| {err.max():.3e} scale {scale:.3f}", flush=True)
    assert err.max() <= 1e-2 * scale
    # The never-aligned residue: row and column L / 2 are bias / eps exactly
    # up to the output rounding.
    r = L // 2
    assert np.allclose(outs[0][r] - old[r], w["outputBias"] / 1e-3, rtol=2e-3, atol=1e-2)


def test_opm_all_masked_row_gives_bias_over_eps(dev):
    from afhip import opm

    act, mask, w = opm_test_case()
    mask = mask.copy()
    mask[:, 2] = 0  # residue 2 never aligned: count = 0 for its pairs
    expect = ref.opm(act, mask, w)
    out = opm.OuterProductMeanGpu().run(opm_input(act, mask, w))["output"].reshape(expect.shape)
    assert np.allclose(out[2], w["outputBias"] / 1e-3, rtol=1e-5)
    assert np.abs(out - expect).max() <= 1e-5 * np.abs(expect).max()


def transition_case(rows, c, h, seed):
    x = ref.normal(seed, (rows, c))
    w = {"layerNormScale": ref.normal(seed + 1, (c,), 0.01, 1.0), "layerNormOffset": ref.normal(seed + 2, (c,), 0.01),
         "firstWeight": ref.normal(seed + 3, (c, h), 1 / c), "firstBias": ref.normal(seed + 4, (h,), 0.02),
         "secondWeight": ref.normal(seed + 5, (h, c), 1 / h), "secondBias": ref.normal(seed + 6, (c,), 0.02)}
    return {"activations": x, "rows": rows, "channels": c, "hiddenChannels": h, "weights": w}


@pytest.mark.parametrize("rows,c,h", [(4096, 128, 512), (77, 16, 64)])
def test_transition(dev, rows, c, h):
    from afhip import transition

    inp = transition_case(rows, c, h, rows)
    expect = ref.transition(inp["activations"], inp["weights"])
    out = transition.TransitionGpu().run(inp)["output"].reshape(expect.shape)
    assert np.abs(out - expect).max() <= 1e-5 * np.abs(expect).max()
    out16 = transition.TransitionGpu().run(inp, {"precision": "f16"})["output"].reshape(expect.shape)
    assert np.abs(out16 - expect).max() <= 1e-2 * max(1.0, np.abs(expect).max())


@pytest.mark.parametrize("rows,c", [(4099, 128), (1001, 64), (515, 256)])
def test_transition_f16_rows(dev, rows, c):
    """f16 activations in and out (the LayerNorm that spreads rows over lane
    groups), with row counts that leave ragged last blocks."""
    import torch

    from afhip import transition

    inp = transition_case(rows, c, 4 * c, rows + c)
    x16 = ref.round_f16(inp["activations"])
    expect = ref.transition(x16, inp["weights"])
    op = transition.Transition(rows, c, 4 * c, precision="f16", in_dtype="f16", out_dtype="f16")
    op.prepare(inp["weights"])
    out = op(torch.from_numpy(x16).half().to(dev)).float().cpu().numpy()
    assert np.abs(out - expect).max() <= 1e-2 * max(1.0, np.abs(expect).max())


@pytest.mark.parametrize("rows,in_dt,out_dt,residual", [
    (1, "f16", "f16", False), (31, "f32", "f32", False), (33, "f16", "f32", True), (4099, "f32", "f16", True),
    (8191, "f16", "f16", True), (64, "f32", "f32", True)])
def test_transition_fused_pair(dev, rows, in_dt, out_dt, residual):
    """The pair transition at f16 precision, channels 128 and hidden 512, runs
    as one fused kernel: every input/output dtype pair, the residual added
    into the output, and row counts that leave a ragged last 32-row tile."""
    import torch

    from afhip import transition

    c, h = 128, 512
    inp = transition_case(rows, c, h, 7 * rows + 3)
    x = inp["activations"] if in_dt == "f32" else ref.round_f16(inp["activations"])
    base = ref.normal(rows + 11, (rows, c))
    base = base if out_dt == "f32" else ref.round_f16(base)
    expect = ref.transition(x, inp["weights"]) + (base if residual else 0.0)
    op = transition.Transition(rows, c, h, precision="f16", in_dtype=in_dt, out_dtype=out_dt, residual=residual)
    op.prepare(inp["weights"])
    tdt = {"f32": torch.float32, "f16": torch.float16}
    out = torch.from_numpy(base).to(tdt[out_dt]).to(dev)
    op(torch.from_numpy(x).to(tdt[in_dt]).to(dev), out=out)
    got = out.float().cpu().numpy()
    assert np.abs(got - expect).max() <= 1e-2 * max(1.0, np.abs(expect).max())


def test_transition_fused_in_place_full_size(dev):
    """z += transition(z) in place over the 1024^2 rows of a long complex's
    pair representation, against a float32 PyTorch restatement of the same
    LayerNorm and linears on the device."""
    import torch

    from afhip import transition

    rows, c, h = 1 << 20, 128, 512
    inp = transition_case(64, c, h, 5)
    w = {k: torch.from_numpy(np.asarray(v, np.float32)).to(dev) for k, v in inp["weights"].items()}
    g = torch.Generator(device=dev).manual_seed(3)
    z = torch.randn(rows, c, generator=g, device=dev).half()
    zf = z.float()
    y = torch.nn.functional.layer_norm(zf, (c,), w["layerNormScale"], w["layerNormOffset"], 1e-5)
    y = torch.relu(y @ w["firstWeight"] + w["firstBias"]) @ w["secondWeight"] + w["secondBias"]
    expect = zf + y
    del y
    op = transition.Transition(rows, c, h, precision="f16", in_dtype="f16", out_dtype="f16", residual=True)
    op.prepare(inp["weights"])
    op(z, out=z)
    err = (z.float() - expect).abs().max().item()
    assert err <= 1e-2 * max(1.0, expect.abs().max().item())


@pytest.mark.parametrize("rows,out_dt,residual", [
    (1, "f16", False), (37, "f32", True), (300, "f16", True), (515, "f32", False), (4099, "f16", True)])
def test_transition_fused_msa(dev, rows, out_dt, residual):
    """The MSA transition at f16 precision, channels 256 and hidden 1024
    (src/evoformer/block.ts:1713-1716), runs as one fused kernel that streams
    the weights in blocks of 32 hidden units: f16 rows in, f16 or f32 out, the
    residual added into the output, and row counts off the 256-row tiles and
    32-row waves."""
    import ctypes

    import torch

    from afhip import _lib, transition

    c, h = 256, 1024
    inp = transition_case(rows, c, h, 5 * rows + 1)
    x = ref.round_f16(inp["activations"])
    base = ref.normal(rows + 13, (rows, c))
    base = base if out_dt == "f32" else ref.round_f16(base)
    expect = ref.transition(x, inp["weights"]) + (base if residual else 0.0)
    op = transition.Transition(rows, c, h, precision="f16", in_dtype="f16", out_dtype=out_dt, residual=residual)
    size = ctypes.c_size_t()
    _lib.call("afhip_transition_workspace_size", ctypes.byref(op.desc), ctypes.byref(size))
    assert size.value == 0  # no normalised rows and no hidden activation in HBM
    op.prepare(inp["weights"])
    tdt = {"f32": torch.float32, "f16": torch.float16}
    out = torch.from_numpy(base).to(tdt[out_dt]).to(dev)
    op(torch.from_numpy(x).half().to(dev), out=out)
    got = out.float().cpu().numpy()
    assert np.abs(got - expect).max() <= 1e-2 * max(1.0, np.abs(expect).max())


def test_transition_fused_msa_in_place_full_size(dev):
    """m += transition(m) in place over BASELINE config 4's MSA (512
    sequences x 256 residues, 131,072 rows of 256 channels), against the
    oracle on seeded rows that cover every row of a 32-row wave and the last
    tile."""
    import torch

    from afhip import transition

    rows, c, h = 512 * 256, 256, 1024
    inp = transition_case(64, c, h, 9)
    m = ref.round_f16(ref.normal(0xAF2007, (rows, c)))
    md = torch.from_numpy(m).half().to(dev)
    op = transition.Transition(rows, c, h, precision="f16", in_dtype="f16", out_dtype="f16", residual=True)
    op.prepare(inp["weights"])
    op(md, out=md)
    got = md.float().cpu().numpy()
    rng = np.random.default_rng(7)
    check = np.unique(np.concatenate([rng.choice(rows, 480, replace=False), np.arange(32), np.arange(rows - 32, rows)]))
    expect = m[check].astype(np.float64) + ref.transition(m[check], inp["weights"])
    err = np.abs(got[check] - expect)
    assert err.max() <= 1e-2 * max(1.0, np.abs(expect).max()), float(err.max())


def test_invalid_opm_and_transition_raise(dev):
    from afhip import _lib, opm, transition

    act, mask, w = opm_test_case()
    bad = opm_input(act, mask, w)
    bad["mask"] = mask.reshape(-1)[1:]
    with pytest.raises(_lib.RangeError, match="mask has"):
        opm.OuterProductMeanGpu().run(bad)
    inp = transition_case(8, 4, 8, 1)
    inp["rows"] = 0
    with pytest.raises(_lib.RangeError):
        transition.TransitionGpu().run(inp)
