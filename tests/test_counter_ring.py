"""CPU unit test of the counter ring's host-side bookkeeping
(coset_amd/csrc/counters.hpp): a slot is handed out only after the launch
that last held it has released it, so a held-back launch keeps its counter
pair through any number of later launches (a cursor-only scheme, the negative
control, is caught by the same check); with every slot held the launch gets
none; concurrent launches finishing out of order never share a slot."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_counter_ring_bookkeeping(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path / "check_ring")
    subprocess.run([cxx, "-O2", "-std=c++17", "-pthread", "-I", os.path.join(ROOT, "coset_amd", "csrc"), "-o", exe,
                    os.path.join(ROOT, "tests", "counters", "check_ring.cpp")], check=True)
    p = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stdout
    assert p.stdout.rstrip().splitlines()[-1].startswith("ok"), p.stdout
