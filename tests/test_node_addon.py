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


def run_node(script, timeout=120):
    proc = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", script)], capture_output=True, text=True,
                          timeout=timeout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return json.loads(proc.stdout.strip().splitlines()[-1])


@needs_node
@needs_addon
def test_addon_loads_and_validates_without_gpu():
    out = run_node("abi_check.js")
    assert out["ok"] and out["exports"] == 42


@pytest.mark.gpu
@needs_node
@needs_addon
def test_addon_parity_on_gpu():
    out = run_node("gpu_parity.js")
    assert len(out["cases"]) == 7
