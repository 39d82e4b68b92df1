"""The execution layer's allocator policy on the CPU: alphafold2-webgpu_amd/
csrc/pool.h (the code libafhip.so's execution layer runs) compiled against a
mock device and driven through the scenarios of the reference's allocator
tests (test/allocator.test.ts:5-165). Two of the reference's scenarios have no
counterpart: usage flags (a HIP buffer has none, test :129-141) and uploads
overtaking queued commands (one HIP stream orders them, test :88-105)."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

GXX = shutil.which("g++")


@pytest.mark.skipif(GXX is None, reason="no g++ on this machine")
def test_pool_policy_matches_the_reference_allocator(tmp_path):
    exe = tmp_path / "pool_cases"
    src = os.path.join(ROOT, "tests", "cpp", "pool_cases.cpp")
    inc = os.path.join(ROOT, "alphafold2-webgpu_amd", "csrc")
    subprocess.run([GXX, "-std=c++17", "-O1", "-Wall", "-Werror", "-I", inc, src, "-o", str(exe)], check=True,
                   capture_output=True, timeout=120)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("ok ")
    assert int(proc.stdout.split()[1]) >= 40
