"""Pins the CPU oracle (oracle/afref.c) before any GPU result is judged by it.

Every oracle function is checked against something other than itself: the
reference's golden fixtures and known-answer tests, numpy's IEEE arithmetic,
closed forms, or identities that a plausible indexing mistake breaks.
"""
import os

import numpy as np
import pytest

from oracle import ref
from afhip.reference import load_triangle_reference_bundle
from conftest import GOLDEN, REFERENCE

REFERENCE_59 = [
    "test/fixtures/alphafold-single-sequence/model1-reference-59/manifest.json",
    "test/fixtures/alphafold-a3m/model1-reference-59/manifest.json",
]


def golden(name):
    return load_triangle_reference_bundle(os.path.join(GOLDEN, name, "manifest.json"))


# --- f16 --------------------------------------------------------------------

def test_f16_encode_known_answers():
    # test/float16.test.ts:5-33
    cases = [(0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-2.0, 0xC000), (np.inf, 0x7C00),
             (-np.inf, 0xFC00), (-0.748291015625, 0xB9FC), (16.1171875, 0x4C08), (52.859375, 0x529C),
             (-78.96875, 0xD4F0), (0.000061005353927612305, 0x0400)]
    got = ref.f32_to_f16([c[0] for c in cases])
    assert [int(v) for v in got] == [c[1] for c in cases]
    assert int(ref.f32_to_f16([np.nan])[0]) & 0x7C00 == 0x7C00
    assert list(ref.f32_to_f16([1, 0.5, -4])) == [0x3C00, 0x3800, 0xC400]


def test_f16_decode_known_answers():
    # test/dtype.test.ts:6-11
    got = ref.f16_to_f32(np.array([0x3C00, 0xC000, 0x0001, 0x7C00], np.uint16))
    assert got[0] == 1 and got[1] == -2 and got[2] == 2.0 ** -24 and got[3] == np.inf


def test_f16_decode_matches_ieee_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    ours = ref.f16_to_f32(bits)
    ieee = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ieee[~nan].view(np.uint32))


def test_f16_encode_is_ieee_rne_over_the_normal_range():
    rng = np.random.default_rng(1)
    # Random f32 bit patterns whose f16 result is normal, plus exact ties.
    exps = rng.integers(127 - 14, 127 + 16, 400000)
    mant = rng.integers(0, 1 << 23, 400000)
    sign = rng.integers(0, 2, 400000)
    bits = (sign << 31) | (exps << 23) | mant
    vals = bits.astype(np.uint32).view(np.float32)
    ties = (np.arange(1, 4000, dtype=np.uint32) << 13 | (1 << 12)) | (120 << 23)
    vals = np.concatenate([vals, ties.view(np.float32)])
    ours = ref.f32_to_f16(vals)
    with np.errstate(over="ignore"):
        ieee = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ieee)


def test_f16_encode_subnormals_differ_from_ieee_only_on_truncated_ties():
    # The reference's subnormal branch shifts before rounding (float16.ts:19-21);
    # the only disagreement allowed with IEEE RNE is a result one ulp below it.
    rng = np.random.default_rng(2)
    vals = rng.uniform(-6.0e-5, 6.0e-5, 200000).astype(np.float32)
    ours = ref.f32_to_f16(vals).astype(np.int64)
    ieee = vals.astype(np.float16).view(np.uint16).astype(np.int64)
    diff = np.abs((ours & 0x7FFF) - (ieee & 0x7FFF))
    assert diff.max() <= 1
    assert (diff > 0).mean() < 1e-3


# --- int8 codecs ------------------------------------------------------------

def test_q8_block_decode_known_answer():
    # test/dtype.test.ts:13-23: codes [1,-2,3,-4,5], block 4, scales 0.5, 2.0
    out = ref.q8_block_decode(np.array([1, -2, 3, -4, 5], np.int8), np.array([0x3800, 0x4000], np.uint16), 4)
    assert list(out) == [0.5, -1, 1.5, -2, 10]
    # A range starting inside a block decodes as the whole tensor does (dtype.ts:56-63).
    assert list(ref.q8_block_decode(np.array([1, -2, 3, -4, 5], np.int8),
                                    np.array([0x3800, 0x4000], np.uint16), 4, start=3, count=2)) == [-2, 10]


def test_q8_block_encode_round_trip_bound():
    w = ref.normal(11, (1000,), 0.02)
    codes, scales = ref.q8_block_encode(w, 64)
    back = ref.q8_block_decode(codes, scales, 64)
    s = ref.f16_to_f32(scales)
    per = np.repeat(s, 64)[:1000]
    assert np.all(np.abs(back - w) <= per * 0.5 + 1e-12)
    for b in range(len(scales)):
        assert np.abs(codes[b * 64:(b + 1) * 64]).max() in (126, 127)
    z_codes, z_scales = ref.q8_block_encode(np.zeros(10, np.float32), 64)
    assert list(z_codes) == [0] * 10 and ref.f16_to_f32(z_scales)[0] == 0


def test_q8_channel_decode_is_one_rounded_product():
    q = ref.uniform_i8(5, (64, 48))
    s = ref.uniform(6, (48,), 1e-3, 1e-2)
    expect = q.astype(np.float32) * s[None, :]
    assert np.array_equal(ref.q8_channel_decode(q, s).view(np.uint32), expect.view(np.uint32))


# --- GEMMs ------------------------------------------------------------------

def test_gemm_and_linear_match_numpy():
    a = ref.lcg_values(3, 81 * 256).reshape(81, 256)
    w = ref.lcg_values(4, 256 * 132).reshape(256, 132)
    b = ref.lcg_values(5, 132)
    expect = a.astype(np.float64) @ w.astype(np.float64) + b
    assert np.allclose(ref.gemm_f64(a, w, b), expect, rtol=1e-13, atol=1e-12)
    lin = ref.linear(a, w, b, relu=True)
    assert np.array_equal(lin, np.maximum(expect, 0).astype(np.float32))
    res = ref.linear(a, w, b, relu=False, residual=np.ones((81, 132), np.float32))
    assert np.array_equal(res, (expect.astype(np.float32).astype(np.float64) * 0 + expect + 1).astype(np.float32))


def test_attention_project_closed_form():
    x = ref.normal(7, (33, 40))
    w = ref.normal(8, (40, 4 * 24), 1 / 40)
    gb = ref.normal(9, (24,), 0.02)
    q, k, v, g = ref.attention_project(x, w, gb, heads=3, head_dim=8)
    full = x.astype(np.float64) @ w.astype(np.float64)
    assert np.allclose(q, full[:, :24] / np.sqrt(8), rtol=1e-6, atol=1e-7)
    assert np.allclose(k, full[:, 24:48], rtol=1e-6, atol=1e-7)
    assert np.allclose(v, full[:, 48:72], rtol=1e-6, atol=1e-7)
    assert np.allclose(g, 1 / (1 + np.exp(-(full[:, 72:] + gb))), rtol=1e-6, atol=1e-7)


# --- triangle multiplication ------------------------------------------------

def _numpy_triangle(direction, inp):
    """Float64 restatement in AlphaFold's einsum form, independent of afref.c."""
    L, cz, ch = inp["shape"]
    w = {k: v.astype(np.float64) for k, v in inp["weights"].items()}
    z = inp["z"].astype(np.float64)
    eps = inp["epsilon"]

    def ln(x, g, b):
        m = x.mean(-1, keepdims=True)
        v = ((x - m) ** 2).mean(-1, keepdims=True)
        return (x - m) / np.sqrt(v + eps) * g + b

    zn = ln(z, w["layerNormInWeight"], w["layerNormInBias"])
    sig = lambda x: 1 / (1 + np.exp(-x))
    mask = inp["mask"].astype(np.float64)[..., None]
    a = mask * (zn @ w["linearAPWeight"].T + w["linearAPBias"]) * sig(zn @ w["linearAGWeight"].T + w["linearAGBias"])
    b = mask * (zn @ w["linearBPWeight"].T + w["linearBPBias"]) * sig(zn @ w["linearBGWeight"].T + w["linearBGBias"])
    x = np.einsum("ikc,jkc->ijc", a, b) if direction == "outgoing" else np.einsum("kjc,kic->ijc", a, b)
    x = ln(x, w["layerNormOutWeight"], w["layerNormOutBias"])
    out = x @ w["linearZWeight"].T + w["linearZBias"]
    return out * sig(zn @ w["linearGWeight"].T + w["linearGBias"])


def test_triangle_outgoing_matches_openfold_fixture():
    # test/cpu-reference.test.ts:18-27
    bundle = golden("openfold-triangle-small")
    inp = bundle["input"]
    assert bundle["source"].startswith("OpenFold")
    out = ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    m = ref.error_metrics(out, bundle["expected"])
    assert m["meanAbsoluteError"] < 1e-7 and m["maxAbsoluteError"] < 1e-6


def test_triangle_outgoing_matches_alphafold_short9():
    bundle = golden("alphafold-short-9")
    inp = bundle["input"]
    out = ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    m = ref.error_metrics(out, bundle["expected"])
    assert m["meanAbsoluteError"] < 1e-5 and m["maxAbsoluteError"] < 1e-4


@pytest.mark.parametrize("rel", REFERENCE_59)
def test_triangle_outgoing_matches_alphafold_59(rel):
    path = os.path.join(REFERENCE, rel)
    if not os.path.exists(path):
        pytest.skip("reference checkout not present")
    bundle = load_triangle_reference_bundle(path)
    inp = bundle["input"]
    out = ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    m = ref.error_metrics(out, bundle["expected"])
    assert m["meanAbsoluteError"] < 1e-5 and m["maxAbsoluteError"] < 1e-4


@pytest.mark.parametrize("name", ["openfold-triangle-small", "alphafold-short-9"])
def test_triangle_incoming_is_transposed_outgoing(name):
    inp = golden(name)["input"]
    zt = np.ascontiguousarray(inp["z"].transpose(1, 0, 2))
    mt = np.ascontiguousarray(inp["mask"].T)
    incoming = ref.triangle("incoming", inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    via = ref.triangle("outgoing", zt, mt, inp["weights"], inp["epsilon"]).transpose(1, 0, 2)
    assert np.array_equal(incoming, via)
    assert not np.allclose(incoming, ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"]))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_triangle_matches_independent_float64_restatement(direction):
    inp = ref.deterministic_triangle_input(11, 12, 10, seed=5)
    out = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    expect = _numpy_triangle(direction, inp)
    assert np.abs(out - expect).max() <= 2e-6 * max(1.0, np.abs(expect).max())


def test_deterministic_input_shape_and_mask_rate():
    inp = ref.deterministic_triangle_input(40, 8, 6)
    assert inp["z"].shape == (40, 40, 8) and inp["mask"].shape == (40, 40)
    assert 0.78 < inp["mask"].mean() < 0.92
    assert np.abs(inp["z"]).max() <= 1.0


# --- outer-product mean -----------------------------------------------------

def spread(count, seed):
    # test/outer-product-mean-reference.gpu.test.ts:81-87
    return (np.sin((np.arange(count) + 1) * seed) * 0.7).astype(np.float32)


def opm_test_case():
    S, L, cm, co, cz = 9, 8, 12, 32, 16
    mask = np.ones(S * L, np.float32)
    mask[::3] = 0
    w = {"layerNormScale": spread(cm, 0.31), "layerNormOffset": spread(cm, 0.17),
         "leftWeight": spread(cm * co, 0.11).reshape(cm, co), "leftBias": spread(co, 0.23),
         "rightWeight": spread(cm * co, 0.13).reshape(cm, co), "rightBias": spread(co, 0.29),
         "outputWeight": spread(co * co * cz, 0.07).reshape(co * co, cz), "outputBias": spread(cz, 0.37)}
    return spread(S * L * cm, 0.19).reshape(S, L, cm), mask.reshape(S, L), w


def _numpy_opm(act, mask, w, eps=1e-5, neps=1e-3):
    x = act.astype(np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    xn = (x - m) / np.sqrt(v + eps) * w["layerNormScale"] + w["layerNormOffset"]
    mk = mask.astype(np.float64)
    left = mk[..., None] * (xn @ w["leftWeight"].astype(np.float64) + w["leftBias"])
    right = mk[..., None] * (xn @ w["rightWeight"].astype(np.float64) + w["rightBias"])
    outer = np.einsum("sia,sjb->ijab", left, right)
    L = act.shape[1]
    outer = outer.reshape(L, L, -1)
    count = np.einsum("si,sj->ij", mk, mk)
    return (outer @ w["outputWeight"].astype(np.float64) + w["outputBias"]) / (neps + count)[..., None]


def test_opm_matches_float64_restatement_on_reference_test_case():
    act, mask, w = opm_test_case()
    out = ref.opm(act, mask, w)
    expect = _numpy_opm(act, mask, w)
    assert np.abs(out - expect).max() < 2e-5 * max(1, np.abs(expect).max())


def test_opm_closed_form_rank_one():
    S, L, cm, co, cz = 7, 5, 6, 4, 3
    act = ref.normal(21, (S, L, cm))
    lb, rb = ref.normal(22, (co,)), ref.normal(23, (co,))
    wo, bo = ref.normal(24, (co * co, cz)), ref.normal(25, (cz,))
    w = {"layerNormScale": np.ones(cm, np.float32), "layerNormOffset": np.zeros(cm, np.float32),
         "leftWeight": np.zeros((cm, co), np.float32), "leftBias": lb,
         "rightWeight": np.zeros((cm, co), np.float32), "rightBias": rb,
         "outputWeight": wo, "outputBias": bo}
    out = ref.opm(act, np.ones((S, L), np.float32), w)
    outer = S * np.outer(lb.astype(np.float64), rb).reshape(-1)
    expect = (outer @ wo.astype(np.float64) + bo) / (1e-3 + S)
    assert np.allclose(out, np.broadcast_to(expect, (L, L, cz)), rtol=2e-6, atol=1e-6)


# --- transition --------------------------------------------------------------

def test_transition_matches_float64_restatement():
    rows, c, h = 37, 16, 64
    x = ref.normal(31, (rows, c))
    w = {"layerNormScale": ref.normal(32, (c,), 0.01, 1.0), "layerNormOffset": ref.normal(33, (c,), 0.01),
         "firstWeight": ref.normal(34, (c, h), 1 / c), "firstBias": ref.normal(35, (h,), 0.02),
         "secondWeight": ref.normal(36, (h, c), 1 / h), "secondBias": ref.normal(37, (c,), 0.02)}
    out = ref.transition(x, w)
    xd = x.astype(np.float64)
    m = xd.mean(-1, keepdims=True)
    v = ((xd - m) ** 2).mean(-1, keepdims=True)
    xn = (xd - m) / np.sqrt(v + 1e-5) * w["layerNormScale"] + w["layerNormOffset"]
    hid = np.maximum(xn @ w["firstWeight"].astype(np.float64) + w["firstBias"], 0)
    expect = hid @ w["secondWeight"].astype(np.float64) + w["secondBias"]
    assert np.abs(out - expect).max() < 1e-5 * max(1, np.abs(expect).max())


def test_error_metrics_exact():
    # test/cpu-reference.test.ts:36-42
    m = ref.error_metrics(np.array([1, 3], np.float32), np.array([2, 1], np.float32))
    assert m == {"meanAbsoluteError": 1.5, "maxAbsoluteError": 2.0, "rootMeanSquareError": np.sqrt(2.5)}
