"""CPU unit test of the counter ring's host-side bookkeeping
(coset_amd/csrc/counters.hpp): runs of counters are consecutive, never
cross the end of the ring, and concurrent takers get disjoint runs."""
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
    assert p.stdout.startswith("ok"), p.stdout
