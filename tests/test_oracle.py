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
from afhip.triangle import triangle_shape
from conftest import GOLDEN

REFERENCE_59 = ["alphafold-single-sequence-59", "alphafold-a3m-59"]


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
    L, cz, ch = triangle_shape(inp)
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


@pytest.mark.parametrize("name", REFERENCE_59)
def test_triangle_outgoing_matches_alphafold_59(name):
    # test/cpu-reference.test.ts:18-27's tolerances on the two AlphaFold
    # 59-residue captures (copied under tests/golden by make_golden.py).
    bundle = golden(name)
    inp = bundle["input"]
    out = ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    m = ref.error_metrics(out, bundle["expected"])
    assert m["meanAbsoluteError"] < 1e-5 and m["maxAbsoluteError"] < 1e-4


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("name", ["openfold-triangle-small", "alphafold-short-9", "alphafold-a3m-59"])
def test_triangle_pairs_matches_the_whole_operator(name, direction):
    # The sampled-pair restatement the full-size GPU tests use, against the
    # oracle's whole operator on every pair of a fixture (the oracle stores
    # f32 intermediates, this one keeps float64) and, outgoing, against the
    # fixture's expected output at the reference's CPU tolerances.
    bundle = golden(name)
    inp = bundle["input"]
    L = inp["z"].shape[0]
    pairs = [(i, j) for i in range(L) for j in range(L)] if L <= 9 else \
        [(i, j) for i in range(0, L, 7) for j in range(3, L, 5)]
    got = ref.triangle_pairs(direction, inp["z"], inp["mask"], inp["weights"], pairs, inp["epsilon"])
    whole = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    expect = np.stack([whole[i, j] for i, j in pairs])
    assert np.abs(got - expect).max() <= 2e-6 * max(1.0, np.abs(expect).max())
    if direction == "outgoing":
        fixture = bundle["expected"].reshape(L, L, -1)
        m = ref.error_metrics(got, np.stack([fixture[i, j] for i, j in pairs]))
        assert m["meanAbsoluteError"] < 1e-6 and m["maxAbsoluteError"] < 1e-5


def test_triangle_is_the_same_at_any_thread_count():
    inp = ref.deterministic_triangle_input(20, 16, 8, seed=3)
    outs = []
    for threads in (1, 3, max(ref.max_threads(), 2)):
        ref.set_threads(threads)
        outs.append(ref.triangle("incoming", inp["z"], inp["mask"], inp["weights"]))
    ref.set_threads(ref.max_threads())
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs)


def test_js_cpu_reference_matches_oracle(tmp_path):
    # oracle/cpu_reference.js (bench.py's CPU baseline: the reference's
    # cpu-reference.ts loops in plain JS) on the reference's deterministic
    # input, against the C oracle: both accumulate in doubles and store f32
    # per tensor, so they differ only where Math.exp and libm's exp round a
    # double differently.
    import shutil
    import subprocess

    node = shutil.which("node")
    if node is None:
        pytest.skip("no node executable")
    from conftest import ROOT

    out_file = tmp_path / "js.f32"
    proc = subprocess.run([node, os.path.join(ROOT, "oracle", "cpu_reference.js"), "12", "16", "8", "7", "--output",
                           str(out_file)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stderr
    report = __import__("json").loads(proc.stdout.strip().splitlines()[-1])
    assert report["shape"] == {"length": 12, "cZ": 16, "cHidden": 8} and report["threads"] == 1
    got = np.fromfile(out_file, dtype="<f4").reshape(12, 12, 16)
    inp = ref.deterministic_triangle_input(12, 16, 8, seed=7)
    expect = ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"])
    assert np.abs(got - expect).max() <= 1e-6 * max(1.0, np.abs(expect).max())


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


def _generator_vectors():
    import json
    import os

    from conftest import GOLDEN

    with open(os.path.join(GOLDEN, "generators.json")) as f:
        return json.load(f)


def test_deterministic_input_matches_reference_generator():
    # Vectors written by the reference's own createDeterministicTriangleInput
    # (src/testing/deterministic-input.ts:7-51, run by
    # tests/golden/make_generator_vectors.js): every tensor of the port equals
    # them bit for bit, the mask's draw order and the default seed included.
    g = _generator_vectors()
    for case in g["createDeterministicTriangleInput"]:
        s = case["shape"]
        inp = ref.deterministic_triangle_input(s["length"], s["cZ"], s["cHidden"], seed=case["seed"])
        assert np.array_equal(inp["z"].reshape(-1), np.asarray(case["z"], np.float32))
        assert np.array_equal(inp["mask"].reshape(-1), np.asarray(case["mask"], np.float32))
        for name in ref.TRIANGLE_ORDER:
            assert np.array_equal(inp["weights"][name].reshape(-1), np.asarray(case["weights"][name], np.float32)), name
    d = g["createDeterministicTriangleInputDefaultSeed"]
    inp = ref.deterministic_triangle_input(2, 2, 2)
    assert np.array_equal(inp["z"].reshape(-1), np.asarray(d["z"], np.float32))


def test_lcg_values_match_reference_generators():
    # test/gemm-half-precision.gpu.test.ts:44-50 and the calibration probes'
    # probeValues (src/runtime/gemm-selection.ts:307-313, seed 0x1234567).
    g = _generator_vectors()
    for case in g["gemmTestValues"]:
        assert np.array_equal(ref.lcg_values(case["seed"], case["count"]), np.asarray(case["values"], np.float32))
    assert np.array_equal(ref.lcg_values(0x1234567, 12), np.asarray(g["probeValues"], np.float32))


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


# --- attention (src/evoformer/attention.ts:1334-1452) ------------------------
# The reference's attention goldens (test/evoformer-attention.gpu.test.ts
# against test/fixtures/evoformer/model1-query-59-block0) are not in the
# reference tree, so the oracle is pinned by closed forms and by a second,
# loop-over-keys restatement with a running softmax.

def _pattern_rows(n_rows, C, seed):
    """Rows a_r * u_r with u_r a +-1 pattern of zero mean and unit variance:
    their LayerNorm is u_r * a_r / sqrt(a_r^2 + eps) exactly (scale 1,
    offset 0)."""
    rng = np.random.default_rng(seed)
    u = np.empty((n_rows, C))
    for r in range(n_rows):
        signs = np.array([1.0] * (C // 2) + [-1.0] * (C // 2))
        u[r] = rng.permutation(signs)
    a = rng.uniform(0.5, 2.0, (n_rows, 1))
    return (u * a).astype(np.float32), u * a / np.sqrt(a * a + 1e-5)


def _attention_weights(C, seed, zero_qk=False):
    rng = np.random.default_rng(seed)
    w = {"queryNormScale": np.ones(C, np.float32), "queryNormOffset": np.zeros(C, np.float32),
         "queryWeight": rng.normal(0, C ** -0.5, (C, C)).astype(np.float32),
         "keyWeight": rng.normal(0, C ** -0.5, (C, C)).astype(np.float32),
         "valueWeight": rng.normal(0, C ** -0.5, (C, C)).astype(np.float32),
         "gatingWeight": rng.normal(0, C ** -0.5, (C, C)).astype(np.float32),
         "gatingBias": rng.normal(0, 0.3, C).astype(np.float32),
         "outputWeight": rng.normal(0, C ** -0.5, (C, C)).astype(np.float32),
         "outputBias": rng.normal(0, 0.1, C).astype(np.float32)}
    if zero_qk:
        w["queryWeight"][:] = 0
        w["keyWeight"][:] = 0
    return w


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


@pytest.mark.parametrize("transpose", [False, True])
def test_attention_uniform_weights_closed_form(transpose):
    # Zero query and key weights and no bias: every key weighs 1/Q, so the
    # output is mean_k(v) * g projected, with v and g from closed-form x_hat.
    B, Q, C, H = 3, 5, 8, 2
    x, xhat = _pattern_rows(B * Q, C, 1)
    w = _attention_weights(C, 2, zero_qk=True)
    got = ref.attention(x, np.ones(B * Q), w, B, Q, C, H, transpose=transpose).reshape(-1, C)
    # attention order: entry (b, q) is source row b Q + q, or q B + b transposed
    rows = lambda b, q: q * B + b if transpose else b * Q + q
    for b in range(B):
        v = np.stack([xhat[rows(b, k)] @ w["valueWeight"] for k in range(Q)])
        for q in range(Q):
            g = _sigmoid(xhat[rows(b, q)] @ w["gatingWeight"] + w["gatingBias"])
            y = (v.mean(axis=0) * g) @ w["outputWeight"] + w["outputBias"]
            assert np.allclose(got[rows(b, q)], y, rtol=1e-5, atol=1e-6)


def test_attention_fully_masked_row_averages_values():
    # Every key of batch row 1 masked: each logit is q.k - 1e9, clamped to
    # -1e8, so the weights are uniform whatever q and k are.
    B, Q, C, H = 3, 6, 8, 4
    x, xhat = _pattern_rows(B * Q, C, 3)
    w = _attention_weights(C, 4)
    mask = np.ones(B * Q)
    mask[Q:2 * Q] = 0
    got = ref.attention(x, mask, w, B, Q, C, H).reshape(B, Q, C)
    v = xhat[Q:2 * Q] @ w["valueWeight"]
    for q in range(Q):
        g = _sigmoid(xhat[Q + q] @ w["gatingWeight"] + w["gatingBias"])
        y = (v.mean(axis=0) * g) @ w["outputWeight"] + w["outputBias"]
        assert np.allclose(got[1, q], y, rtol=1e-5, atol=1e-6)


def test_attention_one_hot_pair_bias_selects_a_key():
    # Normalized-input bias through channel 0 only, +-1 there by construction,
    # times 40 per head: the chosen key outweighs every other by e^80, so the
    # output is that key's value times the query's gate.
    Q, C, H = 6, 8, 2
    B = Q
    rng = np.random.default_rng(5)
    pick = rng.integers(0, Q, Q)  # the key each query attends to (the same in every batch row)
    u = np.empty((B * Q, C))
    for b in range(B):
        for k in range(Q):
            first = 1.0 if k == pick[b] else -1.0
            # the other seven channels bring the row to four +1 and four -1
            rest = rng.permutation([1.0] * (3 if first > 0 else 4) + [-1.0] * (4 if first > 0 else 3))
            u[b * Q + k] = np.concatenate([[first], rest])
    # each row has four +1 and four -1 entries: zero mean, unit variance
    assert np.allclose(u.mean(axis=1), 0) and np.allclose((u * u).mean(axis=1), 1)
    x = u.astype(np.float32)
    xhat = u / np.sqrt(1 + 1e-5)
    w = _attention_weights(C, 6, zero_qk=True)
    wb = np.zeros((C, H), np.float32)
    wb[0, :] = 40.0
    got = ref.attention(x, np.ones(B * Q), w, B, Q, C, H,
                        pair_bias={"source": "normalized-input", "projectionWeight": wb}).reshape(B, Q, C)
    for b in range(B):
        for q in range(Q):
            # bias[h][q][k] = xhat[q][k] . wb: query q of every batch row favours key pick[q]
            v = xhat[b * Q + pick[q]] @ w["valueWeight"]
            g = _sigmoid(xhat[b * Q + q] @ w["gatingWeight"] + w["gatingBias"])
            assert np.allclose(got[b, q], (v * g) @ w["outputWeight"] + w["outputBias"], rtol=1e-6, atol=1e-6)


def _attention_by_loops(x, mask, w, B, Q, C, H, transpose, pair_bias, eps=1e-5):
    """A second restatement: per (b, h, q) a loop over keys with a running
    maximum and sum (the reference's flash recurrence, attention.ts:688-723)."""
    d = C // H
    x = np.asarray(x, np.float64).reshape(-1, C)
    src = lambda b, q: q * B + b if transpose else b * Q + q
    xn = np.zeros((B, Q, C))
    for b in range(B):
        for q in range(Q):
            r = x[src(b, q)]
            mu = sum(r) / C
            var = sum((r - mu) ** 2) / C
            xn[b, q] = (r - mu) / np.sqrt(var + eps) * w["queryNormScale"] + w["queryNormOffset"]
    bias = None
    if pair_bias is not None:
        if pair_bias["source"] == "separate":
            Cp = pair_bias["channels"]
            P = np.asarray(pair_bias["activations"], np.float64).reshape(Q, Q, Cp)
            mu = P.mean(axis=-1, keepdims=True)
            var = ((P - mu) ** 2).mean(axis=-1, keepdims=True)
            Pn = (P - mu) / np.sqrt(var + eps) * pair_bias["layerNormScale"] + pair_bias["layerNormOffset"]
            Wb = np.asarray(pair_bias["projectionWeight"], np.float64).reshape(Cp, H)
        else:
            Pn, Wb = xn, np.asarray(pair_bias["projectionWeight"], np.float64).reshape(C, H)
        bias = lambda h, q, k: float(Pn[q, k] @ Wb[:, h])
    out = np.zeros((B * Q, C))
    for b in range(B):
        qs = xn[b] @ w["queryWeight"] / np.sqrt(d)
        ks = xn[b] @ w["keyWeight"]
        vs = xn[b] @ w["valueWeight"]
        gs = _sigmoid(xn[b] @ w["gatingWeight"] + w["gatingBias"])
        o = np.zeros((Q, C))
        for h in range(H):
            cols = slice(h * d, (h + 1) * d)
            for q in range(Q):
                run_max, run_sum, acc = -1e30, 0.0, np.zeros(d)
                for k in range(Q):
                    mk = mask[k * B + b] if transpose else mask[b * Q + k]
                    logit = float(qs[q, cols] @ ks[k, cols]) + 1e9 * (mk - 1.0)
                    if bias is not None:
                        logit += bias(h, q, k)
                    logit = min(max(logit, -1e8), 1e8)
                    new_max = max(run_max, logit)
                    scale, weight = np.exp(run_max - new_max), np.exp(logit - new_max)
                    run_sum = run_sum * scale + weight
                    acc = acc * scale + weight * vs[k, cols]
                    run_max = new_max
                o[q, cols] = acc / run_sum * gs[q, cols]
        y = o @ w["outputWeight"] + w["outputBias"]
        for q in range(Q):
            out[src(b, q)] = y[q]
    return out.reshape(-1)


@pytest.mark.parametrize("transpose,source", [(False, "separate"), (True, None), (False, "normalized-input"),
                                              (True, "normalized-input")])
def test_attention_matches_loop_restatement(transpose, source):
    rng = np.random.default_rng(7)
    Q, C, H, Cp = 5, 8, 2, 6
    B = Q if source == "normalized-input" else 3
    x = rng.normal(0, 1, B * Q * C).astype(np.float32)
    mask = (rng.uniform(0, 1, B * Q) > 0.3).astype(np.float32)
    mask[:Q] = 0.0  # one fully masked stretch of the mask as well
    w = _attention_weights(C, 8)
    w["queryNormScale"] = rng.normal(1, 0.1, C).astype(np.float32)
    w["queryNormOffset"] = rng.normal(0, 0.1, C).astype(np.float32)
    pb = None
    if source == "separate":
        pb = {"source": "separate", "activations": rng.normal(0, 1, Q * Q * Cp).astype(np.float32), "channels": Cp,
              "layerNormScale": rng.normal(1, 0.1, Cp).astype(np.float32),
              "layerNormOffset": rng.normal(0, 0.1, Cp).astype(np.float32),
              "projectionWeight": rng.normal(0, 1, Cp * H).astype(np.float32)}
    elif source is not None:
        pb = {"source": source, "projectionWeight": rng.normal(0, 1, C * H).astype(np.float32)}
    got = ref.attention(x, mask, w, B, Q, C, H, transpose=transpose, pair_bias=pb)
    expect = _attention_by_loops(x, mask, w, B, Q, C, H, transpose, pb)
    assert np.allclose(got, expect, rtol=1e-5, atol=1e-6)
