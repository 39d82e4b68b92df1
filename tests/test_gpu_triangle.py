"""Triangle multiplication parity on the GPU.

Mirrors test/triangle-multiplication-outgoing.gpu.test.ts and
test/evoformer-triangle-incoming.gpu.test.ts: the f32 path against the
fixtures at mean < 1e-5 / max < 1e-4 and against the oracle at 1e-5 of the
largest value; output blocking reproduces the whole result exactly; the f16
path within 1e-2. Incoming has no committed fixture; it is held to the oracle
and to the transpose identity incoming(z) = T(outgoing(T(z))).
"""
import os

import numpy as np
import pytest

from oracle import ref
from afhip.reference import load_triangle_reference_bundle
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

FIXTURES = ["openfold-triangle-small", "alphafold-short-9", "alphafold-single-sequence-59", "alphafold-a3m-59"]


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def bundle(name):
    return load_triangle_reference_bundle(os.path.join(GOLDEN, name, "manifest.json"))


def rel_max(actual, expected):
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def gpu_class(direction):
    from afhip import triangle

    return triangle.TriangleMultiplicationOutgoingGpu if direction == "outgoing" \
        else triangle.TriangleMultiplicationIncomingGpu


@pytest.mark.parametrize("name", FIXTURES)
def test_outgoing_f32_matches_fixture(dev, name):
    b = bundle(name)
    res = gpu_class("outgoing")().run(b["input"], {"precision": "f32"})
    m = ref.error_metrics(res["output"], b["expected"])
    assert m["meanAbsoluteError"] < 1e-5 and m["maxAbsoluteError"] < 1e-4
    assert res["elapsedMilliseconds"] > 0 and res["memory"]["peakBytes"] > 0


@pytest.mark.parametrize("name", FIXTURES)
def test_outgoing_f16_matches_fixture(dev, name):
    # f16 operands with f32 accumulation against the official f32 capture:
    # within the north star's 1e-2 of the largest value.
    b = bundle(name)
    out = gpu_class("outgoing")().run(b["input"], {"precision": "f16"})["output"]
    assert rel_max(out, b["expected"]) <= 1e-2


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_f32_matches_oracle(dev, name, direction):
    inp = bundle(name)["input"]
    expect = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    out = gpu_class(direction)().run(inp, {"precision": "f32"})["output"]
    assert rel_max(out, expect) <= 1e-5


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("block_rows", [4, 2])
def test_blocking_is_bit_identical(dev, direction, block_rows):
    inp = bundle("alphafold-short-9")["input"]
    whole = gpu_class(direction)().run(inp, {"precision": "f32"})["output"]
    blocked = gpu_class(direction)().run(inp, {"precision": "f32", "blockRows": block_rows})["output"]
    assert np.array_equal(whole.view(np.uint32), blocked.view(np.uint32))


def test_incoming_is_transposed_outgoing(dev):
    inp = bundle("alphafold-short-9")["input"]
    t = dict(inp)
    t["z"] = np.ascontiguousarray(inp["z"].transpose(1, 0, 2))
    t["mask"] = np.ascontiguousarray(inp["mask"].T)
    incoming = gpu_class("incoming")().run(inp, {"precision": "f32"})["output"].reshape(inp["z"].shape)
    via = gpu_class("outgoing")().run(t, {"precision": "f32"})["output"].reshape(inp["z"].shape).transpose(1, 0, 2)
    assert rel_max(incoming, via) <= 1e-6


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_f16_within_1e2(dev, name, direction):
    b = bundle(name)
    inp = b["input"]
    expect = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    out = gpu_class(direction)().run(inp, {"precision": "f16"})["output"]
    m = ref.error_metrics(out, expect)
    assert m["meanAbsoluteError"] < 1e-3 and m["maxAbsoluteError"] < 1e-2
    if direction == "outgoing":
        m = ref.error_metrics(out, b["expected"])
        assert m["meanAbsoluteError"] < 1e-3 and m["maxAbsoluteError"] < 1e-2


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("length,cz,ch", [(64, 128, 128), (37, 16, 24), (96, 128, 128), (100, 128, 128)])
def test_synthetic_against_oracle(dev, direction, length, cz, ch):
    inp = ref.deterministic_triangle_input(length, cz, ch, seed=length + cz)
    expect = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], inp["epsilon"])
    out = gpu_class(direction)().run(inp, {"precision": "f32"})["output"]
    assert rel_max(out, expect) <= 1e-5
    out16 = gpu_class(direction)().run(inp, {"precision": "f16"})["output"]
    err = np.abs(out16.reshape(expect.shape) - expect)
    assert np.all(err <= 1e-2 * np.maximum(1.0, np.abs(expect)))


def test_f16_pair_input_and_residual(dev):
    import torch

    from afhip import triangle

    L, cz, ch = 48, 128, 128
    inp = ref.deterministic_triangle_input(L, cz, ch, seed=3)
    z16 = ref.round_f16(inp["z"])
    expect = ref.triangle("outgoing", z16, inp["mask"], inp["weights"])
    op = triangle.TriangleMultiplication(L, cz, ch, precision="f16", pair_dtype="f16", out_dtype="f32",
                                         residual=True)
    op.prepare(inp["weights"])
    base = torch.full((L, L, cz), 0.5, dtype=torch.float32, device=dev)
    out = op(torch.from_numpy(z16).half().to(dev), torch.from_numpy(inp["mask"]).to(dev), out=base)
    got = out.cpu().numpy() - 0.5
    assert np.all(np.abs(got - expect) <= 1e-2 * np.maximum(1.0, np.abs(expect)))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("length,shift", [(37, 0.0), (100, 6.0), (300, -3.0)])
def test_f16_pair_input_against_oracle(dev, direction, length, shift):
    """f16 z (the kernels that take z's rows into the MFMA as loaded, with
    the LayerNorm mean subtracted in the accumulator): ragged last tiles
    (37 * 37 pairs), several tiles a CU (300 * 300), and rows whose mean is
    far from zero, where a lost mean correction would show at once. At
    300 * 300 the expectation is the f32 path (itself held to the oracle at
    1e-5 above), which the oracle would take ~20 s to produce."""
    import torch

    from afhip import triangle

    cz = ch = 128
    inp = ref.deterministic_triangle_input(length, cz, ch, seed=length + 7)
    z16 = ref.round_f16(inp["z"] + np.float32(shift))
    if length <= 128:
        expect = ref.triangle(direction, z16, inp["mask"], inp["weights"])
    else:
        f32 = triangle.TriangleMultiplication(length, cz, ch, direction=direction, precision="f32")
        f32.prepare(inp["weights"])
        expect = f32(torch.from_numpy(z16).to(dev), torch.from_numpy(inp["mask"]).to(dev)).cpu().numpy()
    op = triangle.TriangleMultiplication(length, cz, ch, direction=direction, precision="f16", pair_dtype="f16",
                                         out_dtype="f32")
    op.prepare(inp["weights"])
    out = op(torch.from_numpy(z16).half().to(dev), torch.from_numpy(inp["mask"]).to(dev)).cpu().numpy()
    err = np.abs(out.reshape(expect.shape) - expect)
    assert np.all(err <= 1e-2 * np.maximum(1.0, np.abs(expect)))


def test_invalid_input_raises_range_error(dev):
    from afhip import _lib

    inp = dict(bundle("openfold-triangle-small")["input"])
    inp["z"] = inp["z"].reshape(-1)[1:]
    with pytest.raises(_lib.RangeError, match="z has"):
        gpu_class("outgoing")().run(inp)
