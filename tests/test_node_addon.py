"""The Node-API addon (alphafold2-webgpu_amd/napi): the drop-in boundary the
reference's TypeScript host binds, driven from Node as the reference's own
tests drive its operators."""
import json
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "alphafold2-webgpu_amd", "napi", "afhip.node")
needs_node = pytest.mark.skipif(NODE is None, reason="no node executable on this machine")
needs_addon = pytest.mark.skipif(not os.path.exists(ADDON), reason="afhip.node not built (no Node headers)")


def run_node(script, timeout=120, env=None):
    proc = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", script)], capture_output=True, text=True,
                          timeout=timeout, env=None if env is None else {**os.environ, **env})
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return json.loads(proc.stdout.strip().splitlines()[-1])


@needs_node
@needs_addon
def test_addon_loads_and_validates_without_gpu():
    out = run_node("abi_check.js")
    assert out["ok"] and out["exports"] == 44


def write_expected(directory):
    """The oracle's answers for the cases gpu_parity.js builds in Node: the
    reference's createDeterministicTriangleInput (both directions), the
    reference test's outer-product-mean literal and a transition input, each
    generated here exactly as the Node script generates it."""
    import numpy as np

    from afhip import reference
    from oracle import ref

    # The reference's triangle fixtures, read here (manifest.json + f32
    # tensors) and handed over as one packed f32 file each with its index.
    for name in ("openfold-triangle-small", "alphafold-short-9", "alphafold-single-sequence-59", "alphafold-a3m-59"):
        bundle = reference.load_triangle_reference_bundle(os.path.join(ROOT, "tests", "golden", name, "manifest.json"))
        inp = bundle["input"]
        arrays = [("z", inp["z"]), ("mask", inp["mask"])] + [(n, inp["weights"][n]) for n in reference.WEIGHT_NAMES]
        arrays.append(("expected", bundle["expected"]))
        with open(os.path.join(directory, name + ".json"), "w") as f:
            json.dump({"shape": inp["shape"], "epsilon": inp["epsilon"], "weights": list(reference.WEIGHT_NAMES),
                       "arrays": [[n, int(a.size)] for n, a in arrays]}, f)
        np.concatenate([a.reshape(-1).astype("<f4") for _, a in arrays]).tofile(os.path.join(directory, name + ".f32"))

    shape = {"length": 24, "cZ": 32, "cHidden": 16}
    with open(os.path.join(directory, "deterministic.json"), "w") as f:
        json.dump({"shape": shape, "seed": 7}, f)
    inp = ref.deterministic_triangle_input(shape["length"], shape["cZ"], shape["cHidden"], seed=7)
    for direction in ("outgoing", "incoming"):
        out = ref.triangle(direction, inp["z"], inp["mask"], inp["weights"], 1e-5)
        out.astype(np.float32).tofile(os.path.join(directory, f"deterministic_{direction}.f32"))

    def spread(count, seed):
        # test/outer-product-mean-reference.gpu.test.ts:81-87
        return (np.sin((np.arange(count) + 1) * seed) * 0.7).astype(np.float32)

    S, L, cm, co, cz = 9, 8, 12, 32, 16
    mask = np.ones(S * L, np.float32)
    mask[::3] = 0
    w = {"layerNormScale": spread(cm, 0.31), "layerNormOffset": spread(cm, 0.17),
         "leftWeight": spread(cm * co, 0.11).reshape(cm, co), "leftBias": spread(co, 0.23),
         "rightWeight": spread(cm * co, 0.13).reshape(cm, co), "rightBias": spread(co, 0.29),
         "outputWeight": spread(co * co * cz, 0.07).reshape(co * co, cz), "outputBias": spread(cz, 0.37)}
    ref.opm(spread(S * L * cm, 0.19).reshape(S, L, cm), mask.reshape(S, L), w).tofile(
        os.path.join(directory, "opm_expected.f32"))

    rows, c, h = 37, 16, 64
    tw = {"layerNormScale": spread(c, 0.53), "layerNormOffset": spread(c, 0.29),
          "firstWeight": spread(c * h, 0.17).reshape(c, h), "firstBias": spread(h, 0.23),
          "secondWeight": spread(h * c, 0.07).reshape(h, c), "secondBias": spread(c, 0.31)}
    ref.transition(spread(rows * c, 0.41).reshape(rows, c), tw).tofile(
        os.path.join(directory, "transition_expected.f32"))


@pytest.mark.gpu
@needs_node
@needs_addon
def test_addon_parity_on_gpu(tmp_path):
    write_expected(str(tmp_path))
    out = run_node("gpu_parity.js", timeout=300, env={"AFHIP_NODE_EXPECTED": str(tmp_path)})
    assert len(out["cases"]) == 12
